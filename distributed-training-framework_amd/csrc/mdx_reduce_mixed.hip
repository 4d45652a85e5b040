// Instantiates the W-way reduction for the dtype triples listed below.
#include "mdx_reduce_impl.h"

namespace mdx {

hipError_t launch_reduce_bfb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_types<bf16, float, bf16>(world, b, p, stream);
}

hipError_t launch_reduce_ffb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_types<float, float, bf16>(world, b, p, stream);
}

hipError_t launch_reduce_bbf(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_types<bf16, bf16, float>(world, b, p, stream);
}

hipError_t launch_reduce_fbb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_types<float, bf16, bf16>(world, b, p, stream);
}

hipError_t launch_reduce_fbf(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return reduce_impl::launch_types<float, bf16, float>(world, b, p, stream);
}

}  // namespace mdx
