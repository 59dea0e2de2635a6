// wf_readout.hip -- sparse attention readout over indices shared across heads (gfx950).
//
// Replaces routing_attention/kernels/fused_sparse.py:97-128 (_sparse_meat_batched) and
// :80-94 (sparse_meat_attention_reference). The reference materialises k_sel/v_sel as
// (B, H, T, K, D) tensors (2 GiB each at T=16384, H=8, K=128, bf16) and runs two batched
// GEMVs; here every gathered K/V row goes straight from memory to registers:
//
//  - one wave per (b, h, t) query row; D/8 lanes share one neighbour (8 dims, one 16-byte
//    load each), so a wave step covers 64*8/D neighbours with full 128-byte lines;
//  - all K and V rows of a batch of steps are loaded before any is used (up to 32 KiB in
//    flight per wave), scores reduce over the D/8 lanes of a neighbour with xor shuffles,
//    and an online softmax (exp2 with log2(e) folded into the scale) carries max and sum
//    across batches; fp32 accumulation, one rounding to the output dtype;
//  - workgroups are mapped so that all rows of one (b, h) pair run on one XCD: blockIdx
//    modulo 8 picks the XCD under round-robin dispatch, which keeps that head's K and V
//    (2 x T x D x s bytes, 4 MiB at the benchmark shape) in that XCD's 4 MiB L2.
#include "wf_internal.h"

namespace wf {
namespace {

constexpr int kWaves = 4;        // waves (rows) per workgroup
constexpr float kLog2e = 1.4426950408889634f;

template <typename DT, bool VEC>
__device__ __forceinline__ void load_row8(const DT* p, int64_t sd, uint4& lo, uint4& hi)
{
    if constexpr (VEC) {
        lo = *reinterpret_cast<const uint4*>(p);
        if constexpr (sizeof(DT) == 4) hi = *reinterpret_cast<const uint4*>(p + 4);
        else hi = make_uint4(0, 0, 0, 0);
    } else {
        if constexpr (sizeof(DT) == 2) {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w[e >> 1] |= uint32_t(*reinterpret_cast<const uint16_t*>(p + e * sd)) << (16 * (e & 1));
            lo = make_uint4(w[0], w[1], w[2], w[3]);
            hi = make_uint4(0, 0, 0, 0);
        } else {
            uint32_t w[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) w[e] = __float_as_uint(*reinterpret_cast<const float*>(p + e * sd));
            lo = make_uint4(w[0], w[1], w[2], w[3]);
            hi = make_uint4(w[4], w[5], w[6], w[7]);
        }
    }
}

template <typename DT>
__device__ __forceinline__ void cvt8(const uint4& lo, const uint4& hi, float* f)
{
    if constexpr (sizeof(DT) == 2) {
        unpack8(lo, DT{}, f);
    } else {
        f[0] = __uint_as_float(lo.x); f[1] = __uint_as_float(lo.y);
        f[2] = __uint_as_float(lo.z); f[3] = __uint_as_float(lo.w);
        f[4] = __uint_as_float(hi.x); f[5] = __uint_as_float(hi.y);
        f[6] = __uint_as_float(hi.z); f[7] = __uint_as_float(hi.w);
    }
}

template <typename DT, bool VEC>
__device__ __forceinline__ void store_row8(DT* p, int64_t sd, const float* f)
{
    DT v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) from_f32(f[e], v[e]);
    if constexpr (VEC) {
        if constexpr (sizeof(DT) == 2) {
            *reinterpret_cast<uint4*>(p) = __builtin_bit_cast(uint4, v);
        } else {
            *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
            *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e * sd] = v[e];
    }
}

// D: head dim (32, 64, 128). NB: wave steps whose loads are issued together.
template <typename DT, bool VEC, int D, int NB>
__global__ __launch_bounds__(64 * kWaves) void sparse_readout_kernel(ReadoutParams p)
{
    constexpr int LPN = D / 8;      // lanes per neighbour
    constexpr int NPS = 64 / LPN;   // neighbours per wave step
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane % LPN;     // 8-dim slice of the head
    const int grp = lane / LPN;     // neighbour within a step

    // XCD-aware mapping: blockIdx % 8 is the XCD; virtual pair vp runs on XCD vp % 8.
    const int64_t xcd = blockIdx.x & 7;
    const int64_t it = blockIdx.x >> 3;
    const int64_t vp = (it / p.wg_per_vpair) * 8 + xcd;
    if (vp >= p.vpairs) return;
    const int64_t chunk = it % p.wg_per_vpair;
    const int64_t pair = vp / p.seg_per_pair;
    const int64_t seg = vp % p.seg_per_pair;
    const int64_t b = pair / p.H, h = pair % p.H;
    const int64_t t0 = seg * p.rows_per_seg;
    const int64_t t1 = min(p.T, t0 + p.rows_per_seg);
    const int64_t t = t0 + chunk * kWaves + wave;
    if (t >= t1) return;

    const int64_t T = p.T;
    const int K = int(p.K);
    const bool mask_pads = (p.flags & 1u) && t < K - 1;

    const DT* qp = static_cast<const DT*>(p.q) + b * p.qs[0] + h * p.qs[1] + t * p.qs[2] + int64_t(sub) * 8 * p.qs[3];
    const DT* kbase = static_cast<const DT*>(p.k) + b * p.ks[0] + h * p.ks[1] + int64_t(sub) * 8 * p.ks[3];
    const DT* vbase = static_cast<const DT*>(p.v) + b * p.vs[0] + h * p.vs[1] + int64_t(sub) * 8 * p.vs[3];
    const int32_t* ip = p.idx + b * p.is[0] + t * p.is[1];

    float qf[8];
    {
        uint4 lo, hi;
        load_row8<DT, VEC>(qp, p.qs[3], lo, hi);
        cvt8<DT>(lo, hi, qf);
    }
    // the scale multiplies the finished dot product, as in the reference; log2(e) rides
    // along so the softmax can use exp2
    const float sl2 = p.scale * kLog2e;

    float m = -__builtin_inff();   // running max (log2 domain), wave-uniform
    float l = 0.0f;                // this lane group's share of the softmax denominator
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};

    for (int s0 = 0; s0 < K; s0 += NB * NPS) {
        uint4 klo[NB], khi[NB], vlo[NB], vhi[NB];
        bool ok[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int slot = s0 + u * NPS + grp;
            ok[u] = slot < K && !(mask_pads && slot > t);
            int64_t j = slot < K ? int64_t(ip[int64_t(slot) * p.is[2]]) : 0;
            if (j < 0) j += T;
            j = j < 0 ? 0 : (j > T - 1 ? T - 1 : j);
            load_row8<DT, VEC>(kbase + j * p.ks[2], p.ks[3], klo[u], khi[u]);
            load_row8<DT, VEC>(vbase + j * p.vs[2], p.vs[3], vlo[u], vhi[u]);
        }
        float sc[NB];
        float bm = -__builtin_inff();
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float kf[8];
            cvt8<DT>(klo[u], khi[u], kf);
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(qf[e], kf[e], d);
#pragma unroll
            for (int o = 1; o < LPN; o <<= 1) d += __shfl_xor(d, o, 64);
            sc[u] = ok[u] ? d * sl2 : -__builtin_inff();
            bm = fmaxf(bm, sc[u]);
        }
#pragma unroll
        for (int o = LPN; o < 64; o <<= 1) bm = fmaxf(bm, __shfl_xor(bm, o, 64));
        const float mn = fmaxf(m, bm);
        const float alpha = (mn == -__builtin_inff()) ? 1.0f : exp2f(m - mn);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float pu = ok[u] ? exp2f(sc[u] - mn) : 0.0f;
            l += pu;
            float vf[8];
            cvt8<DT>(vlo[u], vhi[u], vf);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(pu, vf[e], acc[e]);
        }
        m = mn;
    }
    // combine the lane groups (different neighbours, same dims)
#pragma unroll
    for (int o = LPN; o < 64; o <<= 1) {
        l += __shfl_xor(l, o, 64);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
    }
    if (grp == 0) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float o8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o8[e] = acc[e] * inv;
        DT* op = static_cast<DT*>(p.out) + b * p.os[0] + h * p.os[1] + t * p.os[2] + int64_t(sub) * 8 * p.os[3];
        store_row8<DT, VEC>(op, p.os[3], o8);
    }
}

template <typename DT, bool VEC, int D>
hipError_t launch_d(const ReadoutParams& p, hipStream_t s)
{
    const int64_t grid = 8 * (p.vpairs / 8) * p.wg_per_vpair;
    constexpr int NB = (sizeof(DT) == 4) ? 4 : 8;
    sparse_readout_kernel<DT, VEC, D, NB><<<dim3(unsigned(grid)), dim3(64 * kWaves), 0, s>>>(p);
    return hipGetLastError();
}

template <typename DT, bool VEC>
hipError_t launch_v(const ReadoutParams& p, hipStream_t s)
{
    if (p.D == 32) return launch_d<DT, VEC, 32>(p, s);
    if (p.D == 64) return launch_d<DT, VEC, 64>(p, s);
    return launch_d<DT, VEC, 128>(p, s);
}

template <typename DT>
hipError_t launch_t(bool vec, const ReadoutParams& p, hipStream_t s)
{
    return vec ? launch_v<DT, true>(p, s) : launch_v<DT, false>(p, s);
}

}  // namespace

hipError_t launch_sparse_readout(int dtype, bool vec, const ReadoutParams& p, hipStream_t s)
{
    if (dtype == 2) return launch_t<bf16_t>(vec, p, s);
    if (dtype == 1) return launch_t<_Float16>(vec, p, s);
    return launch_t<float>(vec, p, s);
}

}  // namespace wf
