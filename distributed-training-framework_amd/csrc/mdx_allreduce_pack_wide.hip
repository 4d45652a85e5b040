// Instantiates the pack fused into the widening all-reduce + unpack: bf16 or
// fp16 gradients travel raw and are summed in fp32 into fp32 buckets.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_pack_allreduce_wide(int wire_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                      hipStream_t stream) {
  if (wire_dtype == MDX_F16) return reduce_impl::launch_pack_for<f16, float>(world, b, p, stream);
  return reduce_impl::launch_pack_for<bf16, float>(world, b, p, stream);
}

hipError_t launch_pack_allreduce_dev_wide(int wire_dtype, int world, const DevTable& t, int blocks,
                                          const ReduceParams& p, hipStream_t stream) {
  if (wire_dtype == MDX_F16) return reduce_impl::launch_pack_dev_for<f16, float>(world, t, blocks, p, stream);
  return reduce_impl::launch_pack_dev_for<bf16, float>(world, t, blocks, p, stream);
}

}  // namespace mdx
