/*
 * mdx.h -- C ABI of libmdx.so, the MI355X (gfx950) kernels behind minidist's
 * per-rank gradient-communication path.
 *
 * The reference (minidist, pure Python on torch.distributed) has no native
 * layer: its "operator API" for this path is a handful of Python methods that
 * chain ATen ops.  Each entry point below replaces one of them; the comment
 * above it cites the reference lines (paths relative to the reference repo).
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (HBM) unless stated; the span / piece
 *     tables themselves are HOST arrays that the library copies into the
 *     kernel-argument segment of each dispatch (no device table to manage).
 *   - `stream` is a hipStream_t (NULL = the null stream).  Every call is
 *     asynchronous and stream-ordered; no call synchronises the host, and no
 *     call allocates memory.
 *   - Return 0 on success, a negative MDX_E* code for a rejected argument
 *     (checked before anything is launched), or a positive hipError_t value.
 *     mdx_strerror() names both kinds.
 *   - Arithmetic is IEEE fp32 with round-to-nearest-even, denormals kept and
 *     no contraction, in the same op order as the ATen chain it replaces, so
 *     results are bit-identical to the reference for a fixed summation order.
 *     bf16 and fp16 results are rounded to nearest even (overflow gives
 *     +-inf).  Every NaN stored as bf16 becomes 0xFFFF; a NaN stored as fp16
 *     keeps its sign and the top mantissa bits, quieted: sign | 0x7E00 |
 *     (fp32 mantissa >> 13) -- torch's CPU conversions in both cases.
 *   - found_inf, when not NULL, points to one int32 on the device that the
 *     caller zeroes; a kernel stores 1 into it if it produced any inf or NaN,
 *     and never stores 0.
 *   - No global mutable state: calls are thread-safe; calls that write the
 *     same memory must be ordered by the caller (same stream or events).  The
 *     one exception is mdx_pack_allreduce_unpack_planned_noalloc, whose
 *     per-GPU buffer every call on that GPU shares (see there).
 */
#ifndef MDX_H_
#define MDX_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MDX_ABI_VERSION 10

/* Only the entry points below are exported (the library builds with hidden
 * visibility by default). */
#if defined(__GNUC__) || defined(__clang__)
#define MDX_API __attribute__((visibility("default")))
#else
#define MDX_API
#endif

/* Element types (torch.float32, torch.bfloat16, torch.float16).  Every entry
 * point takes any of them wherever it takes a dtype code, in any combination,
 * except where stated. */
enum { MDX_F32 = 0, MDX_BF16 = 1, MDX_F16 = 2 };

/* Status codes (negative; positive values are hipError_t). */
enum {
  MDX_OK = 0,
  MDX_EINVAL = -1,    /* NULL pointer, negative count or size            */
  MDX_EDTYPE = -2,    /* dtype code not in {MDX_F32, MDX_BF16, MDX_F16}   */
  MDX_EWORLD = -3,    /* world outside [1, MDX_MAX_WORLD] or rank >= world */
  MDX_EALIAS = -4,    /* an output overlaps an input it must not overlap  */
  MDX_ESIZE = -5,     /* plan buffer missing or too small; an IPC
                         allocation of MDX_IPC_MAX_ALLOC_BYTES or more     */
  MDX_ESCRATCH = -6,  /* plan larger than MDX_NOALLOC_SCRATCH_BYTES, or the
                         stream is not on the current device (allocation-free
                         entry point only)                                  */
  MDX_EOP = -7,       /* reduction operation not one of MDX_OP_*           */
};

#define MDX_MAX_WORLD 16

/* One contiguous run copied from `src` to `dst` (both device pointers).
 * `src == NULL` reads as zeros (a parameter whose .grad is None). */
typedef struct mdx_span {
  const void* src;
  void* dst;
  int64_t numel;
} mdx_span;

/* One run of this rank's own contribution to a W-way reduction: elements
 * [pos, pos + numel) of the reduced vector come, for this rank, from `own`
 * (a device pointer, NULL = zeros) and, for every peer r, from
 * peers[r] + pos. */
typedef struct mdx_piece {
  const void* own;
  int64_t pos;
  int64_t numel;
} mdx_piece;

/* Pack: flatten gradients into a bucket, then pre-scale.
 * Replaces _Bucket.gather_into_buffer (minidist/ddp.py:75-92): per span
 * `flat.copy_(p.grad.reshape(-1))` / `flat.zero_()` (ddp.py:85-90), then
 * `buffer.mul_(scale)` (ddp.py:91) with scale = 1/W rounded to fp32 and
 * divide = 0.  Also the FSDP flatten + pre-division of reduce_scatter_grads,
 * `buf[off:off+n].copy_(p.grad.reshape(-1))` then `buf.div_(W)`
 * (minidist/fsdp.py:218-227), with scale = W and divide = 1.
 * dst[i] = rnd_dst(rnd_dst(src[i]) * scale), or ... / scale when divide != 0;
 * the scaling is skipped when scale == 1.  All spans of one call share dtypes.
 * `clear_flag` (may be NULL): a found-inf flag (int32, device memory) that the
 * call also sets to 0, ordered on `stream` like the copy -- the scaler's
 * once-per-step clear (minidist/amp.py:206 `found_inf = zeros(1)`) folded into
 * the pack that precedes the reduction which sets it, instead of a dispatch of
 * its own.  It is cleared even when there is nothing to copy. */
MDX_API int mdx_pack(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, float scale,
                     int divide, int32_t* clear_flag, void* stream);

/* Unpack, with the loss-scaler's unscale + found-inf fused as an epilogue.
 * Replaces _Bucket.scatter_from_buffer (minidist/ddp.py:94-102):
 * `p.grad.copy_(bucket_slice)` -- and, when inv_scale != 1 or found_inf is
 * given, the per-gradient body of DistributedGradScaler.unscale_
 * (minidist/amp.py:212-213): `p.grad.mul_(inv_scale)` then
 * `found_inf += (~isfinite(p.grad)).any()`.
 * dst[i] = v = rnd_dst(src[i]); if inv_scale != 1: v = rnd_dst(v * inv_scale);
 * flag if !isfinite(v).  Spans must not have src == NULL. */
MDX_API int mdx_unpack(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, float inv_scale,
               int32_t* found_inf, void* stream);

/* Multi-tensor unscale + found-inf, in place on each span's `dst`
 * (`src` is ignored).  Replaces the loop of DistributedGradScaler.unscale_
 * (minidist/amp.py:208-213) for gradients that no fused unpack has unscaled:
 * g = rnd(g * inv_scale); flag if !isfinite(g). */
MDX_API int mdx_unscale_found_inf(const mdx_span* spans, int n_spans, int dtype, float inv_scale,
                          int32_t* found_inf, void* stream);

/* W-way SUM all-reduce arithmetic over W replica buffers resident in HBM,
 * in the fixed rank order ((in[0] + in[1]) + in[2]) + ..., one rounding per
 * add in `dtype`.  The W `replicas` share one layout; the call reduces the
 * n_runs element ranges [offsets[k], offsets[k] + numels[k]) (increasing,
 * non-overlapping) of all of them into the same ranges of `out`, which may
 * be one of the replica bases (the in-place all-reduce of a bucket) and must
 * otherwise not overlap them.  One bucket is one run; a run of ready buckets
 * laid out in one buffer is reduced by a single dispatch.
 * Replaces the reduction done by comm.all_reduce -> dist.all_reduce(SUM)
 * (minidist/comm.py:223-234) on DDP buckets (minidist/ddp.py:243-247). */
MDX_API int mdx_allreduce_sum(const void* const* replicas, int world, int dtype, const int64_t* offsets,
                      const int64_t* numels, int n_runs, void* out, void* stream);

/* Reduction operations of mdx_allreduce_op: torch.distributed.ReduceOp's
 * SUM, PRODUCT, MIN and MAX. */
enum { MDX_OP_SUM = 0, MDX_OP_PRODUCT = 1, MDX_OP_MIN = 2, MDX_OP_MAX = 3 };

/* mdx_allreduce_sum with the reduction `op`: per element, in the fixed rank
 * order, acc = in[0], then acc = f(acc, in[r]) for r = 1 .. W-1, with f the
 * IEEE 754-2019 operation that torch's CPU elementwise op computes in `dtype`:
 *   MDX_OP_MAX      maximum: NaN if either is NaN, else the larger (-0 < +0)
 *   MDX_OP_MIN      minimum: NaN if either is NaN, else the smaller (-0 < +0)
 *   MDX_OP_PRODUCT  mul: one rounding per step
 * A NaN result of MAX or MIN is the dtype's quiet NaN (0x7FC00000, 0x7FC0,
 * 0x7E00); a tie of -0 and +0 gives +0 (MAX) or -0 (MIN) in either order;
 * MDX_OP_SUM is mdx_allreduce_sum.  Layout, runs and aliasing rules
 * are mdx_allreduce_sum's (`out` may be a replica base: in place).
 * Replaces the reduction of comm.all_reduce(tensor, op) (minidist/comm.py:
 * 223-234) and of comm.reduce_scatter_tensor(output, input_, op) (comm.py:
 * 252-265) for op in PRODUCT / MIN / MAX -- the reference forwards any op to
 * dist.*, e.g. the scaler's found-inf MAX (minidist/amp.py:216-217). */
MDX_API int mdx_allreduce_op(const void* const* replicas, int world, int dtype, int op, const int64_t* offsets,
                             const int64_t* numels, int n_runs, void* out, void* stream);

/* One parameter's slice of a bucket for the fused all-reduce + unpack:
 * elements [offset, offset + numel) of the replica layout are delivered to
 * `grad` (a device pointer to numel elements of grad_dtype). */
typedef struct mdx_grad_run {
  int64_t offset;
  int64_t numel;
  void* grad;
} mdx_grad_run;

/* W-way SUM all-reduce fused with the unpack into the gradients and the loss
 * scaler's unscale + found-inf.  Per run k and element j, with
 * acc = ((rep[0][o+j] + rep[1][o+j]) + ...) rounded per add in `dtype`:
 *   out[o+j] = acc                       (skipped when out == NULL)
 *   g = rnd_grad(acc); if inv_scale != 1: g = rnd_grad(g * inv_scale)
 *   grad[j] = g; flag if !isfinite(g)
 * Replaces, for one run of ready buckets, comm.all_reduce (minidist/comm.py:
 * 223-234) + _Bucket.scatter_from_buffer (minidist/ddp.py:94-102) + the
 * per-gradient body of DistributedGradScaler.unscale_ (minidist/amp.py:
 * 212-213), without reading the reduced bucket back.  Runs increase and do
 * not overlap; `out` may be one of the replica bases; gradients must not
 * overlap the replicas or `out`. */
MDX_API int mdx_allreduce_unpack(const void* const* replicas, int world, int dtype,
                                 const mdx_grad_run* runs, int n_runs, void* out, int grad_dtype,
                                 float inv_scale, int32_t* found_inf, void* stream);

/* mdx_allreduce_unpack for contributions narrower than the bucket: bf16 or
 * fp16 contributions (wire_dtype = MDX_BF16 or MDX_F16) summed into an fp32
 * bucket (reduce_dtype = MDX_F32; other pairs return MDX_EDTYPE).  Each contribution
 * is widened and pre-scaled where it is received,
 *   x_r = rnd_f32(f32(rep[r][o+j]) * prescale),
 * then acc = ((x_0 + x_1) + ...) in fp32, out[o+j] = acc (fp32, when out !=
 * NULL) and the unpack / unscale / found-inf epilogue of mdx_allreduce_unpack.
 * With prescale = fp32(1/W) this is bit-identical to the reference chain for a
 * bucket of fp32 holding bf16 (fp16) gradients: _Bucket.gather_into_buffer's
 * `flat.copy_(p.grad)` (widening) + `buffer.mul_(1/W)` (minidist/ddp.py:
 * 85-91), comm.all_reduce (minidist/comm.py:223-234), scatter_from_buffer's
 * `p.grad.copy_(reduced)` (ddp.py:100-101, fp32 -> bf16 / fp16 RNE) and unscale_
 * (minidist/amp.py:212-213) -- while the contributions travel at half the
 * bytes.  The fp32 accumulation is FSDP's reduce_dtype arithmetic
 * (minidist/fsdp.py:218-229) applied to DDP buckets.  `out` must not overlap
 * any replica. */
MDX_API int mdx_allreduce_unpack_wide(const void* const* replicas, int world, int wire_dtype,
                                      const mdx_grad_run* runs, int n_runs, void* out, int reduce_dtype,
                                      int grad_dtype, float prescale, float inv_scale, int32_t* found_inf,
                                      void* stream);

/* One parameter's gradient in a fused pack + all-reduce + unpack: elements
 * [offset, offset + numel) of the replica layout.  This rank's contribution
 * is packed from `src` (device pointer; NULL reads as zeros, a parameter
 * whose .grad is None) and the reduced values are delivered to `grad` (which
 * may be `src` itself: each element is read before it is written). */
typedef struct mdx_pack_run {
  int64_t offset;
  int64_t numel;
  const void* src;
  void* grad;
} mdx_pack_run;

/* The pack fused into the all-reduce + unpack: one dispatch for DDP's whole
 * per-rank chain of a run of ready buckets.  Gradients have the wire dtype;
 * the bucket dtype (reduce_dtype) equals it, or is MDX_F32 for bf16 / fp16
 * wires (widening).  Per run and element j (o = offset), with `scale` = 1/W
 * rounded to fp32:
 *   same dtype:  c = rnd(src[j] * scale)            (src = 0 when NULL; no
 *                                                    multiply when scale == 1)
 *   widening:    c = src[j]  (raw; every contribution x is then read as
 *                rnd_f32(f32(x) * scale), as in mdx_allreduce_unpack_wide)
 *   replicas[rank][o+j] = c          (the packed row the peers would read)
 *   acc = rank-ordered SUM of replicas[r][o+j], with c itself for r = rank
 *   out[o+j] = acc                   (the bucket; skipped when out == NULL)
 *   g = rnd_grad(acc); if inv_scale != 1: g = rnd_grad(g * inv_scale)
 *   grad[j] = g; flag if !isfinite(g)
 * Replaces, for one run of ready buckets, _Bucket.gather_into_buffer
 * (minidist/ddp.py:75-92), comm.all_reduce (minidist/comm.py:223-234),
 * _Bucket.scatter_from_buffer (minidist/ddp.py:94-102) and the per-gradient
 * body of DistributedGradScaler.unscale_ (minidist/amp.py:212-213).  The
 * bucket must not overlap the replicas (it holds the average, while row
 * `rank` keeps the packed contribution); gradients and sources must not
 * overlap the replicas or the bucket; a source either is its run's gradient
 * or does not overlap it.
 * `clear_flag` (may be NULL, must differ from found_inf): a flag the call
 * sets to 0, in stream order with the rest of the call -- the loss scaler's
 * flag for the NEXT step, which nothing reads or sets during this one.  The
 * flag this call sets cannot be cleared by the same dispatch, so the scaler
 * alternates two flags and each step's fused pack clears the other.  It is
 * cleared even when there is nothing to reduce. */
MDX_API int mdx_pack_allreduce_unpack(const void* const* replicas, int world, int rank, int wire_dtype,
                                      const mdx_pack_run* runs, int n_runs, void* out, int reduce_dtype,
                                      float scale, float inv_scale, int32_t* found_inf, int32_t* clear_flag,
                                      void* stream);

/* This rank's share of a SUM reduce-scatter, with FSDP's pre-division,
 * dtype changes and optional accumulation fused.
 * Replaces _FSDPUnit.reduce_scatter_grads (minidist/fsdp.py:215-237): widen
 * each contribution to reduce_dtype (fsdp.py:218-222), `buf.div_(W)` when
 * divide != 0 (fsdp.py:227), rank-ordered SUM of the rank's slice
 * (comm.reduce_scatter_tensor, minidist/comm.py:252-265), `out.to(shard
 * dtype)` (fsdp.py:233), then set or `flat_shard.grad.add_(out)`
 * (fsdp.py:234-237) when accumulate != 0.  Optional unscale + found-inf
 * epilogue on the final shard value as in mdx_unpack.
 * Element j of the shard: contribution of rank r = peers[r][j] for r != rank,
 * and own data from the piece covering position j for r == rank (`peers` are
 * already offset to this rank's slice; peers[rank] is ignored). */
MDX_API int mdx_reduce_scatter_share(const mdx_piece* own, int n_own, const void* const* peers, int world,
                             int rank, int in_dtype, int reduce_dtype, int divide, void* shard,
                             int shard_dtype, int accumulate, float inv_scale, int32_t* found_inf,
                             void* stream);

/* The reduce-scatter shares of several FSDP units in one call.
 * Replaces, for every unit whose gradients are ready at the same time,
 * _FSDPUnit.reduce_scatter_grads (minidist/fsdp.py:215-237) -- the units
 * FullyShardedDataParallel.finish_gradient_sync flushes after a no_sync
 * accumulation (fsdp.py:462-470) -- with the arithmetic of
 * mdx_reduce_scatter_share.  The units' contributions live in one set of
 * rows: `peers[r]` is the base of rank r's row (peers[rank] is ignored) and
 * piece k covers elements [pos, pos + numel) of every row; this rank's data
 * for it comes from pieces[k].own (NULL = zeros) and its result goes to
 * outs[k] (numel elements of shard_dtype), which may be any tensor -- each
 * unit's shard gradient is its own.  Destinations must not overlap the rows,
 * any piece's own data or each other.  divide / accumulate / inv_scale /
 * found_inf apply to every piece as in mdx_reduce_scatter_share.  One
 * dispatch per 48 pieces; the planned form below takes any number. */
MDX_API int mdx_reduce_scatter_share_multi(const mdx_piece* pieces, void* const* outs, int n_pieces,
                                           const void* const* peers, int world, int rank, int in_dtype,
                                           int reduce_dtype, int divide, int shard_dtype, int accumulate,
                                           float inv_scale, int32_t* found_inf, void* stream);

/* fp32 -> bf16 round-to-nearest-even cast (NaN -> 0xFFFF), written straight
 * into this rank's slot of the FSDP gather buffer.
 * Replaces `src = flat_shard.to(param_dtype)` in _FSDPUnit.unshard
 * (minidist/fsdp.py:178-180) for param_dtype = bf16; every other dtype pair
 * of that cast is an mdx_pack of one span with scale 1. */
MDX_API int mdx_cast_f32_bf16(const float* src, uint16_t* dst, int64_t numel, void* stream);

/* ---------------------------------------------------------------------------
 * Device-resident plans: the same work as mdx_pack / mdx_unpack /
 * mdx_allreduce_unpack, for any number of spans or runs in ONE dispatch.
 *
 * A plan is the kernel-ready form of a span or grad-run table (with every
 * run's alignment head, workgroup range and the reduction's replica bases).
 * mdx_plan_* writes it into caller-provided host memory (8-byte aligned);
 * the caller copies those bytes to device memory and then launches with both
 * copies -- the host copy supplies the grid and kernel arguments, the device
 * copy is what the workgroups read -- for as long as the addresses inside
 * stay valid.  This is the device-side pointer/offset table that lets the
 * ~150 gradients of a GPT-2 step (most of them small biases and norms) move
 * in one launch per stage.  A plan of more than 2^22 workgroups (2^30 or more
 * elements; one dispatch holds at most 2^32 - 1 work-items) goes out as
 * several dispatches in stream order over consecutive slices of its
 * workgroups: "one dispatch" below means one per 2^22 workgroups.
 *
 * Sizing: on entry *plan_bytes is the capacity of `plan`; on return it is the
 * size the plan needs.  With plan == NULL or too small a capacity nothing is
 * written and MDX_ESIZE is returned.  Inputs are validated as by the direct
 * entry points.
 * ------------------------------------------------------------------------- */

/* Plan for mdx_pack_planned / mdx_unpack_planned over `spans` (whose addresses
 * are frozen into the plan).  Replaces, for a fixed set of gradients, the
 * per-bucket tables of _Bucket.gather_into_buffer / scatter_from_buffer
 * (minidist/ddp.py:75-102). */
MDX_API int mdx_plan_spans(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, void* plan,
                           int64_t* plan_bytes);

/* Plan for mdx_allreduce_unpack_planned (arguments as mdx_allreduce_unpack). */
MDX_API int mdx_plan_allreduce_unpack(const void* const* replicas, int world, int dtype,
                                      const mdx_grad_run* runs, int n_runs, void* out, int grad_dtype,
                                      void* plan, int64_t* plan_bytes);

/* Plan for mdx_allreduce_unpack_planned with the widening of
 * mdx_allreduce_unpack_wide (arguments as there; prescale is frozen into the plan). */
MDX_API int mdx_plan_allreduce_unpack_wide(const void* const* replicas, int world, int wire_dtype,
                                           const mdx_grad_run* runs, int n_runs, void* out, int reduce_dtype,
                                           int grad_dtype, float prescale, void* plan, int64_t* plan_bytes);

/* Plan for mdx_pack_allreduce_unpack_planned (arguments as
 * mdx_pack_allreduce_unpack; rank and scale are frozen into the plan). */
MDX_API int mdx_plan_pack_allreduce_unpack(const void* const* replicas, int world, int rank, int wire_dtype,
                                           const mdx_pack_run* runs, int n_runs, void* out, int reduce_dtype,
                                           float scale, void* plan, int64_t* plan_bytes);

/* Plan for mdx_reduce_scatter_share_multi_planned (arguments as
 * mdx_reduce_scatter_share_multi, with reduce and shard dtype MDX_F32 -- the
 * FSDP default -- which is what the planned form supports). */
MDX_API int mdx_plan_reduce_scatter_share_multi(const mdx_piece* pieces, void* const* outs, int n_pieces,
                                                const void* const* peers, int world, int rank, int in_dtype,
                                                void* plan, int64_t* plan_bytes);

/* mdx_reduce_scatter_share_multi over a plan: every unit's share in one dispatch. */
MDX_API int mdx_reduce_scatter_share_multi_planned(const void* plan, const void* d_plan, int divide, int accumulate,
                                                   float inv_scale, int32_t* found_inf, void* stream);

/* mdx_pack_allreduce_unpack over a plan: one dispatch. */
MDX_API int mdx_pack_allreduce_unpack_planned(const void* plan, const void* d_plan, float inv_scale,
                                              int32_t* found_inf, int32_t* clear_flag, void* stream);

/* mdx_pack over a plan: one dispatch.  `plan` = host copy, `d_plan` = device copy. */
MDX_API int mdx_pack_planned(const void* plan, const void* d_plan, float scale, int divide, int32_t* clear_flag,
                             void* stream);

/* mdx_unpack over a plan whose every span has a source: one dispatch. */
MDX_API int mdx_unpack_planned(const void* plan, const void* d_plan, float inv_scale, int32_t* found_inf,
                               void* stream);

/* mdx_allreduce_unpack (or _wide, by the plan) over a plan: one dispatch. */
MDX_API int mdx_allreduce_unpack_planned(const void* plan, const void* d_plan, float inv_scale,
                                         int32_t* found_inf, void* stream);

/* mdx_pack_allreduce_unpack_planned without a caller-allocated device copy
 * of the plan: the library uploads `plan` (host bytes from
 * mdx_plan_pack_allreduce_unpack) into a device buffer of its own and launches
 * the same kernel on it, with the same results.
 * No counterpart in the reference: this entry point is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc); it calls no hipMalloc, hipFree or
 * other allocating routine.
 *   - The buffer is a fixed array of MDX_NOALLOC_SCRATCH_BYTES per GPU, held
 *     until the process ends; a plan whose size (`*plan_bytes` returned by the
 *     plan builder) exceeds it is rejected with MDX_ESCRATCH before anything
 *     is launched.  `stream` must belong to the current device (else
 *     MDX_ESCRATCH).
 *   - The plan travels in the kernel arguments of small upload dispatches
 *     (3 KB each) enqueued on `stream` ahead of the kernel, so `plan` may be
 *     reused or freed as soon as the call returns.
 *   - Every call on one GPU shares that GPU's buffer: calls on one stream are
 *     ordered, but calls that overlap in time on one GPU (different streams
 *     without events between them, or several threads) race and must not be
 *     made. */
#define MDX_NOALLOC_SCRATCH_BYTES (256 * 1024)
MDX_API int mdx_pack_allreduce_unpack_planned_noalloc(const void* plan, float inv_scale, int32_t* found_inf,
                                                      int32_t* clear_flag, void* stream);

/* ---------------------------------------------------------------------------
 * Peer rows over IPC: the transport of the one-shot and two-shot all-reduces.
 *
 * No counterpart in the reference, which hands every bucket to
 * dist.all_reduce (minidist/comm.py:223-234, called from ddp.py:243-247):
 * these calls let W processes map each other's contribution rows (and
 * buckets), so that each rank runs the same rank-ordered fused reduction
 * (mdx_allreduce_unpack[_planned]) over the peers' rows -- the one-shot
 * all-reduce -- or over its share of them, then copies the peers' reduced
 * shares out of their buckets -- the two-shot all-reduce.  The caller orders
 * the ranks (every rank's pack complete before any rank reads it, every read
 * complete before a rank overwrites its row).
 * ------------------------------------------------------------------------- */

#define MDX_IPC_HANDLE_BYTES 64
/* Each exported allocation stays below this size (larger shared allocations
 * have not opened reliably on this platform). */
#define MDX_IPC_MAX_ALLOC_BYTES ((int64_t)1 << 31)

typedef struct mdx_ipc_handle {
  unsigned char bytes[MDX_IPC_HANDLE_BYTES]; /* the runtime's IPC memory handle */
  int64_t offset;                            /* of the exported pointer in its allocation */
  int64_t alloc_bytes;                       /* size of that allocation */
} mdx_ipc_handle;

/* The IPC handle of the device allocation that contains `ptr`.  Returns
 * MDX_ESIZE (nothing exported) when that allocation is MDX_IPC_MAX_ALLOC_BYTES
 * or larger. */
MDX_API int mdx_ipc_export(const void* ptr, mdx_ipc_handle* out);

/* Maps another process's exported allocation into this one; *base receives
 * the allocation's base here (the exported pointer is *base + h->offset). */
MDX_API int mdx_ipc_open(const mdx_ipc_handle* h, void** base);

/* Unmaps a base mdx_ipc_open returned. */
MDX_API int mdx_ipc_close(void* base);

/* The address kernels use for pinned host memory at `host_ptr` (allocated with
 * hipHostMalloc, e.g. torch's pin_memory), so that a kernel can store a
 * found-inf flag straight into memory the host reads after a stream
 * synchronisation, without a device-to-host copy.  No counterpart in the
 * reference; it serves DistributedGradScaler.unscale_'s flag read
 * (minidist/amp.py:219). */
MDX_API int mdx_host_device_address(void* host_ptr, void** device_ptr);

/* Static description of a status code. */
MDX_API const char* mdx_strerror(int code);

/* MDX_ABI_VERSION of the loaded library. */
MDX_API int mdx_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MDX_H_ */
