// Dispatch of the W-way reduction to its per-dtype-triple instantiations.
#include "mdx_internal.h"

namespace mdx {

hipError_t launch_reduce_fff(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_bbb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_bff(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_bfb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_ffb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_bbf(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_fbb(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);
hipError_t launch_reduce_fbf(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream);

int reduce_frag_elems(int in_dtype, int out_dtype) {
  return frag_elems(dtype_size(in_dtype), dtype_size(out_dtype));
}

hipError_t launch_reduce(int in_dtype, int acc_dtype, int out_dtype, int world, const PieceBatch& b,
                         const ReduceParams& p, hipStream_t stream) {
  const bool ib = in_dtype == MDX_BF16, ab = acc_dtype == MDX_BF16, ob = out_dtype == MDX_BF16;
  if (!ib && !ab && !ob) return launch_reduce_fff(world, b, p, stream);
  if (ib && !ab && !ob) return launch_reduce_bff(world, b, p, stream);
  if (ib && ab && ob) return launch_reduce_bbb(world, b, p, stream);
  if (ib && !ab && ob) return launch_reduce_bfb(world, b, p, stream);
  if (!ib && !ab && ob) return launch_reduce_ffb(world, b, p, stream);
  if (ib && ab && !ob) return launch_reduce_bbf(world, b, p, stream);
  if (!ib && ab && ob) return launch_reduce_fbb(world, b, p, stream);
  return launch_reduce_fbf(world, b, p, stream);
}

}  // namespace mdx
