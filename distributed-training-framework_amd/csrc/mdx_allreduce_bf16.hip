// Instantiates the bf16-bucket all-reduce (one bf16 rounding per add): plain
// SUM, and SUM fused with the unpack into bf16, fp32 or fp16 gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_bf16(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_allreduce_for<bf16>(grad_dtype, unpack, world, b, p, stream);
}

hipError_t launch_allreduce_dev_bf16(int grad_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_allreduce_dev_for<bf16>(grad_dtype, world, t, blocks, p, stream);
}

}  // namespace mdx
