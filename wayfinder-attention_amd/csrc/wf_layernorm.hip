// wf_layernorm.hip -- residual add + LayerNorm over the last dim in one pass (gfx950).
//
// Replaces, in the decoder's inference forward, the pairs of PyTorch ops that the reference
// block runs around every LayerNorm (routing_attention/models/transformer.py:50-73, and the
// final norm at :332): x = x + delta (an elementwise launch) followed by
// F.layer_norm(x) (a second launch that reads x again). Here one pass reads x and delta,
// writes the new residual stream s = x + delta and y = LayerNorm(s).
//
// Layout: 16 lanes per row (one DPP row), 4 rows per wave, 4 waves (16 rows) per workgroup.
// Lane u takes the 8-element chunks u, u + 16, ... of its row and keeps them in registers
// between the statistics and the output, so every element is read once and written once.
//
// Rounding follows the PyTorch ops it replaces: s is x + delta computed in fp32 and rounded
// to the storage type; mean and biased variance of the rounded s are accumulated in fp32
// (two passes over the registers); y = (s - mean) * rsqrt(var + eps) * w + b in fp32,
// rounded once.
#include "wf_internal.h"

namespace wf {
namespace {

constexpr int kLnRowsPerWave = 4;
constexpr int kLnWaves = 4;

// sum over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1)
__device__ __forceinline__ float ln_row_sum16(float x)
{
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x121, 0xf, 0xf, false));
    return x;
}

// eight elements at p (16-byte aligned) -> fp32
template <typename DT>
__device__ __forceinline__ void load8f(const DT* p, float* f)
{
    if constexpr (sizeof(DT) == 4) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
        unpack8(*reinterpret_cast<const uint4*>(p), DT{}, f);
    }
}

// eight fp32 values -> storage type, each rounded once, stored at p (16-byte aligned)
template <typename DT>
__device__ __forceinline__ void store8f(DT* p, const float* f)
{
    if constexpr (sizeof(DT) == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            DT lo, hi;
            from_f32(f[2 * i], lo);
            from_f32(f[2 * i + 1], hi);
            w[i] = uint32_t(__builtin_bit_cast(uint16_t, lo)) | (uint32_t(__builtin_bit_cast(uint16_t, hi)) << 16);
        }
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <typename DT>
__device__ __forceinline__ float round_st(float x)
{
    DT y;
    from_f32(x, y);
    return to_f32(y);
}

// CPL: chunks of 8 elements per lane (n <= 128 CPL)
template <typename DT, int CPL>
__global__ __launch_bounds__(64 * kLnWaves) void residual_layernorm_kernel(LayerNormParams p)
{
    const int lane = threadIdx.x & 63;
    const int u = lane & 15;
    const int64_t row = (int64_t(blockIdx.x) * kLnWaves + (threadIdx.x >> 6)) * kLnRowsPerWave + (lane >> 4);
    const bool row_ok = row < p.rows;
    const int64_t r = row_ok ? row : p.rows - 1;   // rows past the end compute the last row, store nothing
    const int nch = int(p.n / 8);
    const DT* x = static_cast<const DT*>(p.x) + r * p.x_stride;
    const DT* a = p.delta ? static_cast<const DT*>(p.delta) + r * p.delta_stride : nullptr;

    float s[CPL][8];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = u + 16 * i;
        if (c < nch) {
            load8f<DT>(x + 8 * c, s[i]);
            if (a) {
                float d[8];
                load8f<DT>(a + 8 * c, d);
#pragma unroll
                for (int e = 0; e < 8; ++e) s[i][e] = round_st<DT>(s[i][e] + d[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) s[i][e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += s[i][e];
    }
    const float inv_n = 1.0f / float(p.n);
    const float mean = ln_row_sum16(sum) * inv_n;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        if (u + 16 * i < nch) {
#pragma unroll
            for (int e = 0; e < 8; ++e) sq = fmaf(s[i][e] - mean, s[i][e] - mean, sq);
        }
    }
    const float rstd = rsqrtf(ln_row_sum16(sq) * inv_n + p.eps);
    if (!row_ok) return;
    DT* so = p.sum_out ? static_cast<DT*>(p.sum_out) + r * p.sum_stride : nullptr;
    DT* yo = static_cast<DT*>(p.y) + r * p.y_stride;
    const DT* w = static_cast<const DT*>(p.weight);
    const DT* b = static_cast<const DT*>(p.bias);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = u + 16 * i;
        if (c >= nch) continue;
        if (so && a) store8f<DT>(so + 8 * c, s[i]);
        float wv[8], bv[8], y[8];
        if (w) load8f<DT>(w + 8 * c, wv);
        if (b) load8f<DT>(b + 8 * c, bv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float t = (s[i][e] - mean) * rstd;
            if (w) t *= wv[e];
            if (b) t += bv[e];
            y[e] = t;
        }
        store8f<DT>(yo + 8 * c, y);
    }
}

template <typename DT>
hipError_t launch_ln_t(const LayerNormParams& p, hipStream_t s)
{
    const int64_t per_wg = int64_t(kLnRowsPerWave) * kLnWaves;
    const dim3 grid(unsigned((p.rows + per_wg - 1) / per_wg)), block(64 * kLnWaves);
    const int64_t cpl = (p.n / 8 + 15) / 16;
    if (cpl <= 1) residual_layernorm_kernel<DT, 1><<<grid, block, 0, s>>>(p);
    else if (cpl <= 2) residual_layernorm_kernel<DT, 2><<<grid, block, 0, s>>>(p);
    else if (cpl <= 4) residual_layernorm_kernel<DT, 4><<<grid, block, 0, s>>>(p);
    else residual_layernorm_kernel<DT, 8><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_residual_layernorm(int dtype, const LayerNormParams& p, hipStream_t s)
{
    if (dtype == 2) return launch_ln_t<bf16_t>(p, s);
    if (dtype == 1) return launch_ln_t<_Float16>(p, s);
    return launch_ln_t<float>(p, s);
}

}  // namespace wf
