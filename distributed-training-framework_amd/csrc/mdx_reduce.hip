// Dispatch of the W-way reductions to their per-dtype instantiations.
#include "mdx_internal.h"

namespace mdx {

hipError_t launch_allreduce_f32(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_bf16(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_f16(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_dev_f32(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_dev_bf16(int grad_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_dev_f16(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_wide_bf16(int grad_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                      hipStream_t stream);
hipError_t launch_allreduce_wide_f16(int grad_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                     hipStream_t stream);
hipError_t launch_allreduce_wide_dev_bf16(int grad_dtype, int world, const DevTable& t, int blocks,
                                          const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_wide_dev_f16(int grad_dtype, int world, const DevTable& t, int blocks,
                                         const ReduceParams& p, hipStream_t stream);
hipError_t launch_pack_allreduce_same(int dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                      hipStream_t stream);
hipError_t launch_pack_allreduce_dev_same(int dtype, int world, const DevTable& t, int blocks,
                                          const ReduceParams& p, hipStream_t stream);
hipError_t launch_pack_allreduce_wide(int wire_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                                      hipStream_t stream);
hipError_t launch_pack_allreduce_dev_wide(int wire_dtype, int world, const DevTable& t, int blocks,
                                          const ReduceParams& p, hipStream_t stream);
hipError_t launch_share_fast(int in_dtype, int wmax, const PieceBatch& b, const ReduceParams& p,
                             hipStream_t stream);
hipError_t launch_share_generic_f32(int acc_dtype, int out_dtype, const PieceBatch& b, const ReduceParams& p,
                                    hipStream_t stream);
hipError_t launch_share_generic_bf16(int acc_dtype, int out_dtype, const PieceBatch& b, const ReduceParams& p,
                                     hipStream_t stream);
hipError_t launch_share_generic_f16(int acc_dtype, int out_dtype, const PieceBatch& b, const ReduceParams& p,
                                    hipStream_t stream);

hipError_t launch_allreduce(int dtype, int grad_dtype, bool unpack, int world, const PieceBatch& b,
                            const ReduceParams& p, hipStream_t stream) {
  if (dtype == MDX_BF16) return launch_allreduce_bf16(grad_dtype, unpack, world, b, p, stream);
  if (dtype == MDX_F16) return launch_allreduce_f16(grad_dtype, unpack, world, b, p, stream);
  return launch_allreduce_f32(grad_dtype, unpack, world, b, p, stream);
}

hipError_t launch_allreduce_dev(int dtype, int grad_dtype, int world, const DevTable& t, int blocks,
                                const ReduceParams& p, hipStream_t stream) {
  if (dtype == MDX_BF16) return launch_allreduce_dev_bf16(grad_dtype, world, t, blocks, p, stream);
  if (dtype == MDX_F16) return launch_allreduce_dev_f16(grad_dtype, world, t, blocks, p, stream);
  return launch_allreduce_dev_f32(grad_dtype, world, t, blocks, p, stream);
}

hipError_t launch_allreduce_wide(int wire_dtype, int grad_dtype, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream) {
  if (wire_dtype == MDX_F16) return launch_allreduce_wide_f16(grad_dtype, world, b, p, stream);
  return launch_allreduce_wide_bf16(grad_dtype, world, b, p, stream);
}

hipError_t launch_allreduce_wide_dev(int wire_dtype, int grad_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream) {
  if (wire_dtype == MDX_F16) return launch_allreduce_wide_dev_f16(grad_dtype, world, t, blocks, p, stream);
  return launch_allreduce_wide_dev_bf16(grad_dtype, world, t, blocks, p, stream);
}

hipError_t launch_pack_allreduce(int wire_dtype, int reduce_dtype, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream) {
  if (wire_dtype == reduce_dtype) return launch_pack_allreduce_same(wire_dtype, world, b, p, stream);
  return launch_pack_allreduce_wide(wire_dtype, world, b, p, stream);
}

hipError_t launch_pack_allreduce_dev(int wire_dtype, int reduce_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream) {
  if (wire_dtype == reduce_dtype) return launch_pack_allreduce_dev_same(wire_dtype, world, t, blocks, p, stream);
  return launch_pack_allreduce_dev_wide(wire_dtype, world, t, blocks, p, stream);
}

static bool fast_triple(int in_dtype, int acc_dtype, int out_dtype) {
  return acc_dtype == MDX_F32 && out_dtype == MDX_F32;
}

int share_wmax(int in_dtype, int acc_dtype, int out_dtype, int world) {
  if (!fast_triple(in_dtype, acc_dtype, out_dtype)) return 16;
  return world <= 2 ? 2 : (world <= 4 ? 4 : (world <= 8 ? 8 : 16));
}

hipError_t launch_share(int in_dtype, int acc_dtype, int out_dtype, int wmax, const PieceBatch& b,
                        const ReduceParams& p, hipStream_t stream) {
  if (fast_triple(in_dtype, acc_dtype, out_dtype)) return launch_share_fast(in_dtype, wmax, b, p, stream);
  if (in_dtype == MDX_BF16) return launch_share_generic_bf16(acc_dtype, out_dtype, b, p, stream);
  if (in_dtype == MDX_F16) return launch_share_generic_f16(acc_dtype, out_dtype, b, p, stream);
  return launch_share_generic_f32(acc_dtype, out_dtype, b, p, stream);
}

}  // namespace mdx
