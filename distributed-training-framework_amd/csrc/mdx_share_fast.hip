// Instantiates the reduce-scatter share for FSDP's usual dtypes (fp32, bf16 or
// fp16 gradients, fp32 reduction, fp32 shard) at every width class, with
// kernel-argument tables and with device plans (many units in one dispatch).
#include "mdx_reduce_impl.h"

namespace mdx {

template <typename In>
static hipError_t by_width(int wmax, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  switch (wmax) {
    case 2: return launch_share_w<In, float, float, 2>(b, p, stream);
    case 4: return launch_share_w<In, float, float, 4>(b, p, stream);
    case 8: return launch_share_w<In, float, float, 8>(b, p, stream);
    default: return launch_share_w<In, float, float, 16>(b, p, stream);
  }
}

hipError_t launch_share_fast(int in_dtype, int wmax, const PieceBatch& b, const ReduceParams& p,
                             hipStream_t stream) {
  if (in_dtype == MDX_BF16) return by_width<bf16>(wmax, b, p, stream);
  if (in_dtype == MDX_F16) return by_width<f16>(wmax, b, p, stream);
  return by_width<float>(wmax, b, p, stream);
}

template <typename In>
static hipError_t dev_by_width(int wmax, const DevTable& t, int blocks, const ReduceParams& p, hipStream_t stream) {
  using namespace reduce_impl;
  switch (wmax) {
    case 2: return launch_share_dev_w<In, float, float, 2>(t, blocks, p, stream);
    case 4: return launch_share_dev_w<In, float, float, 4>(t, blocks, p, stream);
    case 8: return launch_share_dev_w<In, float, float, 8>(t, blocks, p, stream);
    default: return launch_share_dev_w<In, float, float, 16>(t, blocks, p, stream);
  }
}

hipError_t launch_share_fast_dev(int in_dtype, int wmax, const DevTable& t, int blocks, const ReduceParams& p,
                                 hipStream_t stream) {
  if (in_dtype == MDX_BF16) return dev_by_width<bf16>(wmax, t, blocks, p, stream);
  if (in_dtype == MDX_F16) return dev_by_width<f16>(wmax, t, blocks, p, stream);
  return dev_by_width<float>(wmax, t, blocks, p, stream);
}

}  // namespace mdx
