// wf_fused.hip -- single-pass fused forward for gfx950: causal top-K retrieval and the sparse
// readout of the retrieved rows for every head, in one kernel.
//
// Replaces routing_attention/kernels/fused_sparse.py:327-356 (fused_sparse_attention) as one
// pass: each workgroup retrieves a block of 16 query rows (the retrieval of wf_topk_dev.h),
// keeps the emitted index rows in LDS (over its dead candidate pools) and then reads those
// rows out for all H heads before it retires, so the indices never make an HBM round trip
// and the gathers of one workgroup overlap the VALU/LDS-bound retrieval of the other
// workgroup on the same CU.
//
// Readout layout: lane l of a wave holds 16-byte slices l + 64 i (i < NI) of one token's
// H x D elements -- head (l + 64 i) / SH, dims 8 ((l + 64 i) % SH) .. +7, SH = D / 8 slices
// per head -- so one neighbour's K (or V) for all heads is NI wave loads; in the attention
// module's (B, T, H, D) memory those are one contiguous H x D x 2-byte span. The SH lanes
// of a head reduce their partial dots with DPP, keep one online softmax per head and
// accumulate p . v for their 8 dims in fp32; neighbours come in batches of NBT, the next
// batch's gathers issued before the current one is consumed.
#include "wf_topk_dev.h"
#include "wf_readout_dev.h"

namespace wf {
namespace {

template <typename DT, int SH, int NI>
struct AllHeadsReadout {
    static constexpr bool kActive = true;
    static constexpr int NBT = NI == 1 ? 8 : 4;   // neighbours per batch (even: p.v in pairs)
    FusedReadoutParams fr;

    // pools: the block's LDS pools; row r's index list (k_eff int32) starts at
    // pools + r * pool_stride. Wave w reads out rows 4w .. 4w+3 of the block.
    __device__ void run(const char* pools, size_t pool_stride, int64_t b, int64_t r0, int64_t T,
                        int K, int w, int lane) const
    {
        constexpr uint32_t ES = sizeof(DT);
        uint32_t qo[NI], ko[NI], vo[NI], oo[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int slice = lane + 64 * i;
            const int64_t h = slice / SH, d0 = int64_t(slice % SH) * 8;
            qo[i] = uint32_t((h * fr.qs[1] + d0) * ES);
            ko[i] = uint32_t((h * fr.ks[1] + d0) * ES);
            vo[i] = uint32_t((h * fr.vs[1] + d0) * ES);
            oo[i] = uint32_t((h * fr.os[1] + d0) * ES);
        }
        const char* qb = static_cast<const char*>(fr.q) + b * fr.qs[0] * ES;
        const char* kb = static_cast<const char*>(fr.k) + b * fr.ks[0] * ES;
        const char* vb = static_cast<const char*>(fr.v) + b * fr.vs[0] * ES;
        char* ob = static_cast<char*>(fr.out) + b * fr.os[0] * ES;
        const uint64_t qst = uint64_t(fr.qs[2]) * ES, kst = uint64_t(fr.ks[2]) * ES;
        const uint64_t vst = uint64_t(fr.vs[2]) * ES, ost = uint64_t(fr.os[2]) * ES;
        const float sl2 = fr.scale * kLog2e;
        const bool mask_pads = (fr.flags & 1u) != 0;

        const int row_lo = 4 * w;
        const int nrows = int(min(int64_t(4), max(int64_t(0), T - (r0 + row_lo))));
        if (nrows <= 0) return;
        const int nb = (K + NBT - 1) / NBT;
        const int ntask = nrows * nb;

        // task tau = (row row_lo + tau / nb, batch tau % nb); past the end: the last task again
        auto gather = [&](int tau, uint4 (&kx)[NBT][NI], uint4 (&vx)[NBT][NI]) {
            const int tt = min(tau, ntask - 1);
            const int32_t* li = reinterpret_cast<const int32_t*>(pools + size_t(row_lo + tt / nb) * pool_stride);
            const int s0 = (tt % nb) * NBT;
#pragma unroll
            for (int u = 0; u < NBT; ++u) {
                // in [0, T) from the retrieval; clamped as well, so a gather can never leave the keys
                const uint32_t j = min(uint32_t(__builtin_amdgcn_readfirstlane(li[min(s0 + u, K - 1)])),
                                       uint32_t(T - 1));
                const char* kr = kb + uint64_t(j) * kst;
                const char* vr = vb + uint64_t(j) * vst;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    kx[u][i] = *reinterpret_cast<const uint4*>(kr + ko[i]);
                    vx[u][i] = *reinterpret_cast<const uint4*>(vr + vo[i]);
                }
            }
        };

        uint4 qv[NI];
        float m[NI], l[NI], acc[NI][8];
        auto compute = [&](int tau, const uint4 (&kx)[NBT][NI], const uint4 (&vx)[NBT][NI]) {
            const int r = tau / nb, bat = tau % nb;
            const int64_t t = r0 + row_lo + r;
            if (bat == 0) {
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    qv[i] = *reinterpret_cast<const uint4*>(qb + uint64_t(t) * qst + qo[i]);
                    m[i] = -__builtin_inff();
                    l[i] = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[i][e] = 0.0f;
                }
            }
            const int lim = (mask_pads && t < K - 1) ? int(t) + 1 : K;   // slots >= lim: no weight
            const int s0 = bat * NBT;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                float sc[NBT];
                float bm = -__builtin_inff();
                const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int u = 0; u < NBT; ++u) {
                    const float d = group_sum<SH>(dot8<DT>(qv[i], zero, kx[u][i], zero));
                    sc[u] = s0 + u < lim ? d * sl2 : -__builtin_inff();
                    bm = fmaxf(bm, sc[u]);
                }
                const float mn = fmaxf(m[i], bm);
                const float ms = mn == -__builtin_inff() ? 0.0f : mn;
                const float alpha = __builtin_amdgcn_exp2f(m[i] - ms);
                l[i] *= alpha;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[i][e] *= alpha;
#pragma unroll
                for (int u = 0; u < NBT; u += 2) {
                    const float pa = __builtin_amdgcn_exp2f(sc[u] - ms);
                    const float pc = __builtin_amdgcn_exp2f(sc[u + 1] - ms);
                    l[i] += pa + pc;
                    pv2<DT>(acc[i], pa, pc, vx[u][i], zero, vx[u + 1][i], zero);
                }
                m[i] = mn;
            }
            if (bat == nb - 1) {
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
                    float o8[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) o8[e] = acc[i][e] * inv;
                    store_row8<DT, true>(reinterpret_cast<DT*>(ob + uint64_t(t) * ost + oo[i]), 1, o8);
                }
            }
        };

        uint4 kA[NBT][NI], vA[NBT][NI], kB[NBT][NI], vB[NBT][NI];
        gather(0, kA, vA);
        for (int tau = 0; tau < ntask; tau += 2) {
            gather(tau + 1, kB, vB);
            compute(tau, kA, vA);
            gather(tau + 2, kA, vA);
            if (tau + 1 < ntask) compute(tau + 1, kB, vB);
        }
    }
};

// Two workgroups per CU, as the retrieval kernel: the retrieval's LDS (<= 80 KiB) and
// registers (<= 256 per lane) bound the occupancy; the readout stage keeps two batches of
// gathers in flight per wave in registers instead of more waves.
template <typename DT, int KP2, int SH, int NI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void fused_single_pass_kernel(TopkParams p, FusedReadoutParams fr)
{
    causal_topk_body<DT, true, 1, KP2>(p, AllHeadsReadout<DT, SH, NI>{fr});
}

template <typename DT, int KP2>
hipError_t launch_kp(const TopkParams& p, const FusedReadoutParams& fr, hipStream_t s)
{
    const dim3 grid(unsigned(p.B * (p.rb_end - p.rb_begin))), block(256);
    const int sh = int(fr.D / 8), ni = int(fr.H * fr.D / 8 / 64);
    if (sh == 8 && ni == 1) fused_single_pass_kernel<DT, KP2, 8, 1><<<grid, block, 0, s>>>(p, fr);
    else if (sh == 8) fused_single_pass_kernel<DT, KP2, 8, 2><<<grid, block, 0, s>>>(p, fr);
    else if (ni == 1) fused_single_pass_kernel<DT, KP2, 16, 1><<<grid, block, 0, s>>>(p, fr);
    else fused_single_pass_kernel<DT, KP2, 16, 2><<<grid, block, 0, s>>>(p, fr);
    return hipGetLastError();
}

}  // namespace

bool fused_single_pass_supported(int dtype, bool topk_vec, const TopkParams& tp, const FusedReadoutParams& fr)
{
    if (dtype != 2 || !topk_vec || tp.R != 32) return false;
    if (tp.k_eff <= 64 || tp.k_eff > 256) return false;
    if (fr.D != 64 && fr.D != 128) return false;
    const int64_t slices = fr.H * fr.D / 8;
    if (slices != 64 && slices != 128) return false;
    // 32-bit lane offsets of the head/dim part; token strides are 64-bit
    const int64_t* st[4] = {fr.qs, fr.ks, fr.vs, fr.os};
    for (const int64_t* x : st)
        if (x[3] != 1 || x[1] < 0 || x[2] < 0 || (fr.H - 1) * x[1] * 2 + fr.D * 2 >= (int64_t(1) << 31)) return false;
    return true;
}

hipError_t launch_fused_single_pass(int dtype, const TopkParams& tp, const FusedReadoutParams& fr, hipStream_t s)
{
    (void)dtype;   // bf16 (fused_single_pass_supported)
    if (tp.k_eff <= 128) return launch_kp<bf16_t, 128>(tp, fr, s);
    return launch_kp<bf16_t, 256>(tp, fr, s);
}

}  // namespace wf
