// Instantiates the pack fused into the all-reduce + unpack for same-dtype
// buckets (fp32, bf16, fp16 gradients in buckets of their own dtype).
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_pack_allreduce_same(int dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                      hipStream_t stream) {
  if (dtype == MDX_BF16) return reduce_impl::launch_pack_for<bf16, bf16>(world, b, p, stream);
  if (dtype == MDX_F16) return reduce_impl::launch_pack_for<f16, f16>(world, b, p, stream);
  return reduce_impl::launch_pack_for<float, float>(world, b, p, stream);
}

hipError_t launch_pack_allreduce_dev_same(int dtype, int world, const DevTable& t, int blocks,
                                          const ReduceParams& p, hipStream_t stream) {
  if (dtype == MDX_BF16) return reduce_impl::launch_pack_dev_for<bf16, bf16>(world, t, blocks, p, stream);
  if (dtype == MDX_F16) return reduce_impl::launch_pack_dev_for<f16, f16>(world, t, blocks, p, stream);
  return reduce_impl::launch_pack_dev_for<float, float>(world, t, blocks, p, stream);
}

}  // namespace mdx
