// Instantiates the reduce-scatter share of bf16 contributions for the
// remaining (reduction, shard) dtype pairs, at the widest class (runtime
// W <= 16).
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_share_generic_bf16(int acc_dtype, int out_dtype, const PieceBatch& b, const ReduceParams& p,
                                     hipStream_t stream) {
  return reduce_impl::launch_share_generic_for<bf16>(acc_dtype, out_dtype, b, p, stream);
}

}  // namespace mdx
