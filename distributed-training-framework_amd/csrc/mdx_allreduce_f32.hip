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

}  // namespace mdx
