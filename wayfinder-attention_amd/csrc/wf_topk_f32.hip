// wf_topk_f32.hip -- causal top-K retrieval kernels for float addresses (instantiations of
// wf_topk_inst.h in a translation unit of their own, so the types compile in parallel).
#include "wf_topk_inst.h"

namespace wf {

hipError_t launch_causal_topk_f32(bool vec, const TopkParams& p, hipStream_t s)
{
    return launch_topk_t<float>(vec, p, s);
}

}  // namespace wf
