// Instantiates the bf16-bucket all-reduce (one bf16 rounding per add): plain
// SUM, and SUM fused with the unpack into bf16 or fp32 gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_bf16(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  if (!unpack) return launch_allreduce<bf16, bf16, false>(world, b, p, stream);
  if (grad_dtype == MDX_F32) return launch_allreduce<bf16, float, true>(world, b, p, stream);
  return launch_allreduce<bf16, bf16, true>(world, b, p, stream);
}


hipError_t launch_allreduce_dev_bf16(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  if (grad_dtype == MDX_F32) return launch_allreduce_unpack_dev<bf16, float>(world, t, blocks, p, stream);
  return launch_allreduce_unpack_dev<bf16, bf16>(world, t, blocks, p, stream);
}

}  // namespace mdx
