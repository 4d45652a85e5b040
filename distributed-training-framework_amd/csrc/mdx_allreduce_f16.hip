// Instantiates the fp16-bucket all-reduce (one fp16 rounding per add): plain
// SUM, and SUM fused with the unpack into fp16, fp32 or bf16 gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_f16(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_allreduce_for<f16>(grad_dtype, unpack, world, b, p, stream);
}

hipError_t launch_allreduce_dev_f16(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_allreduce_dev_for<f16>(grad_dtype, world, t, blocks, p, stream);
}

}  // namespace mdx
