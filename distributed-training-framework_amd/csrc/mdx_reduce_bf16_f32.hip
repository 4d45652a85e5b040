// Instantiates the W-way reduction for the dtype triples listed below.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_reduce_bff(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_types<bf16, float, float>(world, b, p, stream);
}

}  // namespace mdx
