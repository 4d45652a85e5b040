// Instantiates the reduce-scatter share for the remaining dtype triples
// (bf16 reduction or bf16 shard), at the widest class (runtime W <= 16).
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_share_generic(int in_dtype, int acc_dtype, int out_dtype, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  const bool ib = in_dtype == MDX_BF16, ab = acc_dtype == MDX_BF16, ob = out_dtype == MDX_BF16;
  if (ib && ab && ob) return launch_share_w<bf16, bf16, bf16, 16>(b, p, stream);
  if (ib && ab && !ob) return launch_share_w<bf16, bf16, float, 16>(b, p, stream);
  if (ib && !ab && ob) return launch_share_w<bf16, float, bf16, 16>(b, p, stream);
  if (!ib && ab && ob) return launch_share_w<float, bf16, bf16, 16>(b, p, stream);
  if (!ib && ab && !ob) return launch_share_w<float, bf16, float, 16>(b, p, stream);
  return launch_share_w<float, float, bf16, 16>(b, p, stream);
}

}  // namespace mdx
