// Instantiates the fp32-bucket all-reduce: plain SUM, and SUM fused with the
// unpack into fp32, bf16 or fp16 gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_f32(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_allreduce_for<float>(grad_dtype, unpack, world, b, p, stream);
}

hipError_t launch_allreduce_dev_f32(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_allreduce_dev_for<float>(grad_dtype, world, t, blocks, p, stream);
}

}  // namespace mdx
