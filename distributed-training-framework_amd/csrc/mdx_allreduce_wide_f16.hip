// Instantiates the widening fused all-reduce + unpack for fp16 contributions:
// summed in fp32 into an fp32 bucket, unpacked into fp32, bf16 or fp16
// gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_wide_f16(int grad_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                     hipStream_t stream) {
  return reduce_impl::launch_wide_for<f16>(grad_dtype, world, b, p, stream);
}

hipError_t launch_allreduce_wide_dev_f16(int grad_dtype, int world, const DevTable& t, int blocks,
                                         const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_wide_dev_for<f16>(grad_dtype, world, t, blocks, p, stream);
}

}  // namespace mdx
