// wf_topk.hip -- causal top-K address retrieval for gfx950 (MI355X): the key-magnitude
// kernel and the launchers. The algorithm and its device code are in wf_topk_dev.h, the
// retrieval kernels' instantiations in wf_topk_inst.h (one translation unit per type).
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

// the retrieval kernels of each input type are instantiated in a translation unit of their
// own (wf_topk_bf16.hip, wf_topk_f16.hip, wf_topk_f32.hip), compiled in parallel
hipError_t launch_causal_topk(int dtype, bool vec, const TopkParams& p, hipStream_t s)
{
    if (dtype == 2) return launch_causal_topk_bf16(vec, p, s);
    if (dtype == 1) return launch_causal_topk_f16(vec, p, s);
    return launch_causal_topk_f32(vec, p, s);
}

}  // namespace wf
