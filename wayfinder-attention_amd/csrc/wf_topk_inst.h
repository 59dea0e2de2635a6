// wf_topk_inst.h -- the retrieval kernels and their launch dispatch over the template grid
// (address-dim chunks RC, top-K width KP2), included by one translation unit per input type.
#pragma once

#include "wf_topk_dev.h"

namespace wf {
namespace {

// Two workgroups per CU: LDS (<= 80 KiB each) and registers (<= 256 per lane) both allow 2
// waves per SIMD for address dims up to 64 and K up to 256; the attribute keeps the register
// allocation inside that bound. Wider addresses (RC >= 4) and K > 256 run one workgroup per
// CU (the wide kernel: up to 160 KiB of LDS, registers unbounded by occupancy).
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
    if constexpr (!kWideTopk<RC, KP2>) causal_topk_kernel<DT, VEC, RC, KP2><<<grid, block, 0, s>>>(p);
    else causal_topk_wide_kernel<DT, VEC, RC, KP2><<<grid, block, 0, s>>>(p);
}

template <typename DT, bool VEC, int RC>
hipError_t launch_topk_k(const TopkParams& p, hipStream_t s)
{
    if (p.k_eff <= 64) launch_topk_kp<DT, VEC, RC, 64>(p, s);
    else if (p.k_eff <= 128) launch_topk_kp<DT, VEC, RC, 128>(p, s);
    else if (p.k_eff <= 256) launch_topk_kp<DT, VEC, RC, 256>(p, s);
    else launch_topk_kp<DT, VEC, RC, 512>(p, s);
    return hipGetLastError();
}

template <typename DT, bool VEC>
hipError_t launch_topk_r(const TopkParams& p, hipStream_t s)
{
    if (p.R <= 32) return launch_topk_k<DT, VEC, 1>(p, s);
    if (p.R <= 64) return launch_topk_k<DT, VEC, 2>(p, s);
    if (p.R <= 128) return launch_topk_k<DT, VEC, 4>(p, s);
    return launch_topk_k<DT, VEC, 8>(p, s);
}

template <typename DT>
hipError_t launch_topk_t(bool vec, const TopkParams& p, hipStream_t s)
{
    return vec ? launch_topk_r<DT, true>(p, s) : launch_topk_r<DT, false>(p, s);
}

}  // namespace
}  // namespace wf
