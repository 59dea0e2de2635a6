// wf_topk.hip -- causal top-K address retrieval for gfx950 (MI355X): kernels and
// launchers. The algorithm and its device code are in wf_topk_dev.h.
//
// Replaces routing_attention/kernels/causal_topk.py:132-171 (_causal_topk_row_blocked) and
// :37-57 (_finalize_causal_topk).
#include "wf_topk_dev.h"

namespace wf {
namespace {

// ------------------------------------------------------------------ kernels
// Bound on |key element| per chunk of kAbsmaxChunk keys (one thread per key).
template <typename DT, bool VEC>
__global__ __launch_bounds__(kAbsmaxChunk) void key_absmax_kernel(TopkParams p)
{
    const int64_t b = blockIdx.y;
    const int64_t jk = int64_t(blockIdx.x) * kAbsmaxChunk + threadIdx.x;
    const DT* kb = static_cast<const DT*>(p.key) + b * p.ksb;
    const int R = int(p.R);
    float m = 0.0f;
    if (jk < p.T) {
        for (int d0 = 0; d0 < R; d0 += 8) {
            uint4 lo, hi;
            load8<DT, VEC>(kb + jk * p.kst, p.ksr, d0, R, lo, hi);
            float f[8];
            to_f32x8<DT>(lo, hi, f);
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(f[e]));
        }
    }
    m = wave_max(m);
    __shared__ float part[kAbsmaxChunk / 64];
    if (lane_id() == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = part[0];
        for (int i = 1; i < kAbsmaxChunk / 64; ++i) r = fmaxf(r, part[i]);
        p.chunk_absmax[b * p.n_chunks + blockIdx.x] = r;
    }
}

// Two workgroups per CU: LDS (<= 80 KiB each) and registers (<= 256 per lane) both allow 2
// waves per SIMD for address dims up to 64; the attribute keeps the register allocation
// inside that bound. Wider addresses (RC = 4) keep their registers at 1 wave per SIMD.
template <typename DT, bool VEC, int RC, int KP2>
__global__ __launch_bounds__(64 * kTopkWaves) __attribute__((amdgpu_waves_per_eu(2)))
void causal_topk_kernel(TopkParams p)
{
    causal_topk_body<DT, VEC, RC, KP2>(p);
}
template <typename DT, bool VEC, int RC, int KP2>
__global__ __launch_bounds__(64 * kTopkWaves) void causal_topk_wide_kernel(TopkParams p)
{
    causal_topk_body<DT, VEC, RC, KP2>(p);
}

template <typename DT, bool VEC, int RC, int KP2>
void launch_topk_kp(const TopkParams& p, hipStream_t s)
{
    const dim3 grid(unsigned(p.B * (p.rb_end - p.rb_begin))), block(64 * kTopkWaves);
    if constexpr (RC <= 2) causal_topk_kernel<DT, VEC, RC, KP2><<<grid, block, 0, s>>>(p);
    else causal_topk_wide_kernel<DT, VEC, RC, KP2><<<grid, block, 0, s>>>(p);
}

template <typename DT, bool VEC, int RC>
hipError_t launch_topk_k(const TopkParams& p, hipStream_t s)
{
    if (p.k_eff <= 64) launch_topk_kp<DT, VEC, RC, 64>(p, s);
    else if (p.k_eff <= 128) launch_topk_kp<DT, VEC, RC, 128>(p, s);
    else launch_topk_kp<DT, VEC, RC, 256>(p, s);
    return hipGetLastError();
}

template <typename DT, bool VEC>
hipError_t launch_topk_r(const TopkParams& p, hipStream_t s)
{
    if (p.R <= 32) return launch_topk_k<DT, VEC, 1>(p, s);
    if (p.R <= 64) return launch_topk_k<DT, VEC, 2>(p, s);
    return launch_topk_k<DT, VEC, 4>(p, s);
}

template <typename DT>
hipError_t launch_topk_t(bool vec, const TopkParams& p, hipStream_t s)
{
    return vec ? launch_topk_r<DT, true>(p, s) : launch_topk_r<DT, false>(p, s);
}

template <typename DT>
hipError_t launch_absmax_t(bool vec, const TopkParams& p, hipStream_t s)
{
    const dim3 grid(unsigned(p.n_chunks), unsigned(p.B)), block(kAbsmaxChunk);
    if (vec) key_absmax_kernel<DT, true><<<grid, block, 0, s>>>(p);
    else key_absmax_kernel<DT, false><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_key_absmax(int dtype, bool vec, const TopkParams& p, hipStream_t s)
{
    if (dtype == 2) return launch_absmax_t<bf16_t>(vec, p, s);
    if (dtype == 1) return launch_absmax_t<_Float16>(vec, p, s);
    return launch_absmax_t<float>(vec, p, s);
}

hipError_t launch_causal_topk(int dtype, bool vec, const TopkParams& p, hipStream_t s)
{
    if (dtype == 2) return launch_topk_t<bf16_t>(vec, p, s);
    if (dtype == 1) return launch_topk_t<_Float16>(vec, p, s);
    return launch_topk_t<float>(vec, p, s);
}

}  // namespace wf
