// wf_topk_bf16.hip -- causal top-K retrieval kernels for bf16_t addresses (instantiations of
// wf_topk_inst.h in a translation unit of their own, so the types compile in parallel).
#include "wf_topk_inst.h"

namespace wf {

hipError_t launch_causal_topk_bf16(bool vec, const TopkParams& p, hipStream_t s)
{
    return launch_topk_t<bf16_t>(vec, p, s);
}

}  // namespace wf
