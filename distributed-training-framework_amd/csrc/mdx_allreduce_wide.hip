// Instantiates the widening fused all-reduce + unpack: bf16 contributions
// summed in fp32 into an fp32 bucket, unpacked into bf16 or fp32 gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_wide(int grad_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                 hipStream_t stream) {
  using namespace reduce_impl;
  if (grad_dtype == MDX_BF16) return launch_allreduce_wide<bf16, float, bf16>(world, b, p, stream);
  return launch_allreduce_wide<bf16, float, float>(world, b, p, stream);
}

hipError_t launch_allreduce_wide_dev(int grad_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  if (grad_dtype == MDX_BF16) return launch_allreduce_wide_dev<bf16, float, bf16>(world, t, blocks, p, stream);
  return launch_allreduce_wide_dev<bf16, float, float>(world, t, blocks, p, stream);
}

}  // namespace mdx
