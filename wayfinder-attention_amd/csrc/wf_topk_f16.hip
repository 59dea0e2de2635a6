// wf_topk_f16.hip -- causal top-K retrieval kernels for _Float16 addresses (instantiations of
// wf_topk_inst.h in a translation unit of their own, so the types compile in parallel).
#include "wf_topk_inst.h"

namespace wf {

hipError_t launch_causal_topk_f16(bool vec, const TopkParams& p, hipStream_t s)
{
    return launch_topk_t<_Float16>(vec, p, s);
}

}  // namespace wf
