// Instantiates the fp32-bucket all-reduce: plain SUM, and SUM fused with the
// unpack into fp32 or bf16 gradients.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_allreduce_f32(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  if (!unpack) return launch_allreduce<float, float, false>(world, b, p, stream);
  if (grad_dtype == MDX_BF16) return launch_allreduce<float, bf16, true>(world, b, p, stream);
  return launch_allreduce<float, float, true>(world, b, p, stream);
}


hipError_t launch_allreduce_dev_f32(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  if (grad_dtype == MDX_BF16) return launch_allreduce_unpack_dev<float, bf16>(world, t, blocks, p, stream);
  return launch_allreduce_unpack_dev<float, float>(world, t, blocks, p, stream);
}

}  // namespace mdx
