// Internal declarations shared by the libmdx translation units.
//
// Work tables travel in the kernel-argument segment of each dispatch: the
// host packs up to kRunsPerLaunch runs (spans or pieces) into one struct
// passed by value; a workgroup finds its run by a binary search over
// `first_block`, which the compiler reads with scalar loads because the index
// is wave-uniform.  Runs are split on the host so that no run needs more than
// kMaxRunElems elements, which keeps every grid far below 2^32 work-items.
#pragma once

#include <hip/hip_runtime.h>
#include <climits>
#include <stdint.h>

#include "mdx.h"

#pragma clang fp contract(off)

namespace mdx {

constexpr int kBlock = 64;  // one wave64 per workgroup (measured: beats 128, 256, 512 and 1024 lanes)
constexpr int kRunsPerLaunch = 48;        // runs per dispatch (kernarg budget)
constexpr int64_t kMaxRunElems = int64_t(1) << 26;

// bf16 and fp16 storage types: raw bits, so that conversions are exact and
// explicit.
struct bf16 {
  uint16_t u;
};
struct f16 {
  uint16_t u;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// The same vector in the global address space.  Every buffer this library
// touches is device memory, but pointers read from a work table are generic
// (flat) pointers; casting them makes the compiler emit global_load/store
// instead of flat_load/store (no aperture check, no LDS counter).  The views
// assume no alignment beyond 2 bytes: every vector access of the kernels goes
// through them, so a stream that the run's head leaves unaligned still moves
// in one dwordx4 / dwordx2 instruction per lane (the target runs in
// unaligned-access mode; for an aligned address the instruction is the same).
typedef u32x4 u32x4_any __attribute__((aligned(2)));
typedef __attribute__((address_space(1))) u32x4_any gu32x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef u32x2 u32x2_any __attribute__((aligned(2)));
typedef __attribute__((address_space(1))) u32x2_any gu32x2;

// ----------------------------------------------------------------------------
// Element conversions (IEEE, round to nearest even; NaN -> 0xFFFF for bf16,
// sign | 0x7E00 | mantissa >> 13 for fp16, as torch's CPU conversions)
// ----------------------------------------------------------------------------

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return __uint_as_float(uint32_t(x.u) << 16); }
// fp16 -> fp32 is exact (v_cvt_f32_f16; fp16 subnormals are kept).
__device__ __forceinline__ float to_f32(f16 x) { return float(__builtin_bit_cast(_Float16, x.u)); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);

template <>
__device__ __forceinline__ float from_f32<float>(float x) {
  return x;
}

// fp32 -> bf16: gfx950's v_cvt_pk_bf16_f32 (round to nearest even, subnormals
// kept, overflow to +-inf), equal to the integer rounding
// (u + 0x7fff + ((u >> 16) & 1)) >> 16 on every non-NaN input (checked over
// all 2^32 fp32 patterns on the device); NaNs become 0xFFFF.
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) {
  bf16 r;
  r.u = __builtin_isnan(x) ? uint16_t(0xffffu) : __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  return r;
}

// fp32 -> fp16: v_cvt_f16_f32 in the default mode (round to nearest even,
// fp16 subnormals kept, overflow to +-inf); NaNs are rebuilt as torch does.
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) {
  const uint32_t u = __float_as_uint(x);
  f16 r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.u = uint16_t(((u >> 16) & 0x8000u) | 0x7e00u | ((u >> 13) & 0x3ffu));
  } else {
    r.u = __builtin_bit_cast(uint16_t, _Float16(x));
  }
  return r;
}

// `dst.copy_(src)` for one element: identity within a dtype (NaN payloads
// untouched), one rounding across dtypes.
template <typename S, typename D>
struct Cvt {
  __device__ __forceinline__ static D run(S x) { return from_f32<D>(to_f32(x)); }
};
template <typename T>
struct Cvt<T, T> {
  __device__ __forceinline__ static T run(T x) { return x; }
};

__device__ __forceinline__ bool is_finite(float x) { return __builtin_isfinite(x); }
__device__ __forceinline__ bool is_finite(bf16 x) { return (x.u & 0x7f80u) != 0x7f80u; }
__device__ __forceinline__ bool is_finite(f16 x) { return (x.u & 0x7c00u) != 0x7c00u; }

template <typename T>
__device__ __forceinline__ T zero_of() {
  T z;
  __builtin_memset(&z, 0, sizeof(T));
  return z;
}

// ----------------------------------------------------------------------------
// Vector loads and stores of one fragment (E elements: 8, 16 or 32 bytes)
// ----------------------------------------------------------------------------

template <typename T, int E, bool NT>
__device__ __forceinline__ void vload(T (&dst)[E], const T* p) {
  constexpr int BYTES = int(E * sizeof(T));
  static_assert(BYTES == 8 || BYTES % 16 == 0, "fragment must be 8 bytes or whole 16-byte vectors");
  if constexpr (BYTES == 8) {
    const gu32x2* q = (const gu32x2*)(p);
    u32x2 w;
    if constexpr (NT) {
      w = __builtin_nontemporal_load(q);
    } else {
      w = *q;
    }
    __builtin_memcpy(&dst[0], &w, 8);
  } else {
    constexpr int NV = BYTES / 16;
    constexpr int PER = int(16 / sizeof(T));
    const gu32x4* q = (const gu32x4*)(p);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      u32x4 w;
      if constexpr (NT) {
        w = __builtin_nontemporal_load(q + k);
      } else {
        w = q[k];
      }
      __builtin_memcpy(&dst[k * PER], &w, 16);
    }
  }
}

template <typename T, int E, bool NT>
__device__ __forceinline__ void vstore(T* p, const T (&src)[E]) {
  constexpr int BYTES = int(E * sizeof(T));
  static_assert(BYTES == 8 || BYTES % 16 == 0, "fragment must be 8 bytes or whole 16-byte vectors");
  if constexpr (BYTES == 8) {
    gu32x2* q = (gu32x2*)(p);
    u32x2 w;
    __builtin_memcpy(&w, &src[0], 8);
    if constexpr (NT) {
      __builtin_nontemporal_store(w, q);
    } else {
      *q = w;
    }
  } else {
    constexpr int NV = BYTES / 16;
    constexpr int PER = int(16 / sizeof(T));
    gu32x4* q = (gu32x4*)(p);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      u32x4 w;
      __builtin_memcpy(&w, &src[k * PER], 16);
      if constexpr (NT) {
        __builtin_nontemporal_store(w, q + k);
      } else {
        q[k] = w;
      }
    }
  }
}

// A wave's 8 four-byte values per lane, stored so that each store instruction
// writes 1 KB of consecutive bytes.  Lane t holds elements [8t, 8t + 8) of the
// wave's 512-element chunk at `chunk`; store k (0, 1) writes elements
// [256k + 4t, 256k + 4t + 4), which lane 32k + t/2 holds (its half t & 1),
// fetched with ds_bpermute.  Every lane of the wave must reach this call (the
// permutes read other lanes' registers); only elements below `limit` are
// stored, and each of them comes from a lane below limit / 8.
template <typename T>
__device__ __forceinline__ void vstore_wave8(T* chunk, const T (&src)[8], int t, int limit) {
  static_assert(sizeof(T) == 4, "four-byte elements");
  const bool upper = (t & 1) != 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int from = (32 * k + (t >> 1)) << 2;
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int lo = __builtin_amdgcn_ds_bpermute(from, __builtin_bit_cast(int, src[e]));
      const int hi = __builtin_amdgcn_ds_bpermute(from, __builtin_bit_cast(int, src[e + 4]));
      w[e] = uint32_t(upper ? hi : lo);
    }
    const int first = 256 * k + 4 * t;
    if (first + 4 <= limit) __builtin_nontemporal_store(w, (gu32x4*)(chunk + first));
  }
}

// Workgroup -> run lookup: largest s in [lo, hi) with first_block[s] <= blk
// (first_block[lo] <= blk must hold).
__device__ __forceinline__ int find_run_in(const int32_t* first_block, int lo, int hi, int blk) {
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (first_block[mid] <= blk) {
      lo = mid;
    } else {
      hi = mid;
    }
  }
  return lo;
}

// Device plans also hold one hint per kHintBlocks workgroups: hint[g] is the
// run that contains workgroup g * kHintBlocks, and hint[groups] = count - 1.
// The run of workgroup blk then lies in [hint[g], hint[g + 1]], g = blk /
// kHintBlocks, usually a range of one or two runs: a workgroup resolves its
// run with two or three dependent scalar loads instead of log2(count) of them.
constexpr int kHintShift = 6;
constexpr int kHintBlocks = 1 << kHintShift;

__device__ __forceinline__ int find_run_hinted(const int32_t* first_block, const int32_t* hint, int blk) {
  const int g = blk >> kHintShift;
  return find_run_in(first_block, hint[g], hint[g + 1] + 1, blk);
}

// One wave stores 1 into *flag if any of its lanes saw a non-finite value.
// Must be reached by every lane of the wave.
__device__ __forceinline__ void flag_nonfinite(bool bad, int32_t* flag) {
  if (__ballot(bad) != 0ull && (threadIdx.x & 63u) == 0u) {
    *flag = 1;
  }
}

// ----------------------------------------------------------------------------
// Copy / convert / scale (pack, unpack, unscale, cast)
// ----------------------------------------------------------------------------

struct SpanBatch {
  const void* src[kRunsPerLaunch];
  void* dst[kRunsPerLaunch];
  int64_t numel[kRunsPerLaunch];
  int32_t head[kRunsPerLaunch];  // scalar elements before the 16B-aligned body; -1 = no body
  int32_t first_block[kRunsPerLaunch + 1];
  int32_t count;
};

enum : int32_t { kCopyScale = 1, kCopyCheck = 2, kCopyDivide = 4 };

struct CopyParams {
  float scale;
  int32_t flags;
  int32_t* found_inf;
  int32_t* clear;  // set to 0 by the dispatch's first lane (the scaler's per-step flag clear), or NULL
};

// Fragments.  In the W-way reductions a fragment is one 16-byte vector of the
// widest type the kernel stores, so that every store instruction of a wave
// writes 64 x 16 = 1 KB of consecutive bytes; a narrower input is then read 8
// bytes per lane.  (Fragments sized by the narrow type instead store 16 bytes
// of every 32 per instruction, which measured 6-8% extra HBM writes on the
// widening kernels.)  In the copy kernel a fragment is one 16-byte vector of
// the wider of its two types: a widening copy reads 8 bytes and stores 16 per
// lane, a narrowing one (the fp32 -> bf16 gather cast) reads 16 and stores 8,
// which on the cast's shape measured 6804 GB/s against 6115 for 32-byte reads
// with 16-byte stores.  Each lane loads at least 16 bytes per input in the
// copy kernel (U fragments), and about 128 bytes across all inputs in the
// W-way reductions.
constexpr int min_size(int a, int b) { return a < b ? a : b; }
constexpr int max_size(int a, int b) { return a > b ? a : b; }
constexpr int64_t min_i64(int64_t a, int64_t b) { return a < b ? a : b; }
constexpr int store_frag_elems(int widest_store_size) { return 16 / widest_store_size; }
constexpr int copy_frag_elems_of(int src_size, int dst_size) { return 16 / max_size(src_size, dst_size); }
constexpr int copy_unroll(int frag_in_bytes) { return frag_in_bytes >= 16 ? 1 : 16 / frag_in_bytes; }
// Fragments per lane of a copy: a narrowing copy takes two (with the wave-wide
// run lookup of SpanArgView::span_run_wave), everything else enough for 16
// loaded bytes per lane.
constexpr int copy_unroll_of(int src_size, int dst_size) {
  return src_size > dst_size ? 2 : copy_unroll(copy_frag_elems_of(src_size, dst_size) * src_size);
}
// Alignment heads are searched over 16 bytes of the narrowest (2-byte) type,
// whatever the fragment, so that mixed-dtype runs keep a vector body.
constexpr int kHeadRange = 8;

hipError_t launch_copy(int src_dtype, int dst_dtype, const SpanBatch& b, const CopyParams& p,
                       hipStream_t stream);
hipError_t launch_clear_flag(int32_t* flag, hipStream_t stream);
int copy_frag_elems(int src_dtype, int dst_dtype);

// ----------------------------------------------------------------------------
// W-way reductions (all-reduce sum, fused all-reduce + unpack, reduce-scatter share)
// ----------------------------------------------------------------------------

struct PieceBatch {
  const void* own[kRunsPerLaunch];
  int64_t pos[kRunsPerLaunch];
  int64_t numel[kRunsPerLaunch];
  void* grad[kRunsPerLaunch];  // fused unpack destination (all-reduce + unpack only)
  int32_t head[kRunsPerLaunch];
  int32_t first_block[kRunsPerLaunch + 1];
  int32_t count;
};

enum : int32_t {
  kRedPreMul = 1,      // every contribution * pre, rounded to the reduce dtype
  kRedPreDiv = 2,      // every contribution / pre, rounded to the reduce dtype
  kRedAccumulate = 4,  // out = out + result (rounded to the out dtype)
  kRedUnscale = 8,     // stored value * inv_scale, rounded to its dtype
  kRedPackScale = 16,  // fused pack: this rank's gradient * pre, rounded to the bucket dtype
};

struct ReduceParams {
  const void* peer[MDX_MAX_WORLD];
  void* out;  // may be NULL for the fused unpack (bucket not written)
  int32_t world;
  int32_t rank;
  int32_t flags;
  float pre;
  float inv_scale;
  int32_t* found_inf;
  int32_t* clear;  // fused pack: a flag the dispatch's first lane sets to 0 (never found_inf), or NULL
};

// Fragments per lane and contribution (U) of the W-way reductions: each lane
// keeps U fragments of all W contributions in flight, about 128 bytes of
// loads (one 16-byte fragment per contribution at W = 8).  Measured on MI355X
// with one-wave workgroups: 256 or 512 bytes per lane cost 2-6% of the W = 8
// all-reduce's bandwidth, and a workgroup that streams several chunks in a
// double-buffered loop loses to one short-lived workgroup per chunk.
constexpr int kReduceLoadBytesPerLane = 128;
// Elements per fragment of the W-way reductions with an unpack.  A widening
// reduction (16-bit contributions, fp32 bucket) loads its contributions 16
// bytes per lane -- 8 elements, whose 4-byte results vstore_wave8 writes in
// whole 1 KB rows (measured: 4% faster than 8-byte loads with 16-byte stores);
// otherwise a fragment is one 16-byte vector of the widest stored type.
constexpr int reduce_frag_elems(int in_size, int out_size, int grad_size) {
  return in_size < out_size ? 16 / in_size : store_frag_elems(max_size(out_size, grad_size));
}
constexpr int clamp_unroll(int u) { return u < 1 ? 1 : (u > 8 ? 8 : u); }
constexpr int allreduce_unroll(int world, int frag_in_bytes) {
  return clamp_unroll(kReduceLoadBytesPerLane / (world * frag_in_bytes));
}
// The fused pack + all-reduce + unpack writes three streams (the packed row,
// the bucket, the gradient) per element and runs fastest with one fragment
// per lane and contribution for every W: measured on its access shape with
// one-wave workgroups, two fragments cost 2.5-3% at W = 3 and 4, 5% at W = 2
// and 1% at W = 8, and four 9% at W = 2 and 4.
constexpr int pack_allreduce_unroll() { return 1; }
constexpr int share_unroll(int wmax, int frag_in_bytes) {
  return clamp_unroll(kReduceLoadBytesPerLane / (wmax * frag_in_bytes));
}

// Non-SUM all-reduce (mdx_allreduce_op): runs of the replica layout in the
// kernel arguments, one-wave workgroups.  A lane takes op_unroll(WMAX)
// 16-byte vectors of every replica -- about 128 bytes of loads in flight, as
// the W-way sums keep -- where WMAX is the compile-time bound on the world.
constexpr int op_wmax(int world) { return world <= 2 ? 2 : (world <= 4 ? 4 : (world <= 8 ? 8 : 16)); }
constexpr int op_unroll(int wmax) { return wmax >= 8 ? 1 : 8 / wmax; }
constexpr int64_t op_elems_per_block(int esize, int wmax) { return int64_t(kBlock) * op_unroll(wmax) * (16 / esize); }

struct OpRuns {
  int64_t offset[kRunsPerLaunch];
  int64_t numel[kRunsPerLaunch];
  int32_t first_block[kRunsPerLaunch + 1];
  int32_t count;
};

struct OpParams {
  const void* rep[MDX_MAX_WORLD];
  void* out;
  int32_t world;
};

hipError_t launch_allreduce_op(int dtype, int op, int wmax, const OpRuns& t, int blocks, const OpParams& p,
                               hipStream_t stream);

// Host-side dispatch into the instantiating translation units.
hipError_t launch_allreduce(int dtype, int grad_dtype, bool unpack, int world, const PieceBatch& b,
                            const ReduceParams& p, hipStream_t stream);
hipError_t launch_share(int in_dtype, int acc_dtype, int out_dtype, int wmax, const PieceBatch& b,
                        const ReduceParams& p, hipStream_t stream);
int share_wmax(int in_dtype, int acc_dtype, int out_dtype, int world);
// Widening fused all-reduce + unpack: bf16 or fp16 contributions, fp32 bucket.
hipError_t launch_allreduce_wide(int wire_dtype, int grad_dtype, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream);

// ----------------------------------------------------------------------------
// Work-table views.  A kernel body reads its runs through one of two views:
// the batch passed by value in the kernel-argument segment (at most
// kRunsPerLaunch runs), or a plan resident in device memory (any number of
// runs, built once on the host and reused while the addresses hold).
// ----------------------------------------------------------------------------

struct DevTable {
  const int32_t* first_block;  // count + 1 entries
  const int32_t* hint;         // blocks / kHintBlocks + 2 entries (see find_run_hinted)
  const int32_t* head;
  const int64_t* numel;
  const uint64_t* a;  // span: src    piece: own
  const uint64_t* b;  // span: dst    piece: grad
  const int64_t* pos;  // piece position (pieces only)
  int32_t count;
  int32_t base;  // plan workgroup of this dispatch's first workgroup (see launch_plan_slices)
};

// A dispatch holds at most 2^32 - 1 work-items (the AQL packet's grid size is
// 32-bit), 2^26 - 1 workgroups of kBlock lanes.  A plan with more workgroups
// than kPlanSliceBlocks goes out as several dispatches in stream order, each
// covering the plan's workgroups [base, base + grid); the slice (2^22
// workgroups, at least 2^30 elements) keeps the extra dispatch boundaries far
// below a percent of the work.  Kernel-argument batches stay under the limit
// by construction (kRunsPerLaunch runs of at most kMaxRunElems elements).
constexpr int kPlanSliceBlocks = 1 << 22;
static_assert(int64_t(kRunsPerLaunch) * kMaxRunElems / kBlock < (int64_t(1) << 32) / kBlock,
              "a kernel-argument batch fits one dispatch");

template <typename Launch>
hipError_t launch_plan_slices(DevTable t, int blocks, Launch&& launch) {
  for (int64_t b0 = 0; b0 < blocks; b0 += kPlanSliceBlocks) {
    t.base = int32_t(b0);
    launch(t, int(min_i64(kPlanSliceBlocks, blocks - b0)));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// A workgroup's run: its chunk index within the run, the run's chunk count
// and its table fields.  Views of a kernel-argument table read run 0's fields
// in the same round of scalar loads as the table's count and first boundary,
// so a workgroup of run 0 -- every workgroup of a one-run dispatch, such as an
// FSDP unit's cast -- starts its vector loads one dependent round earlier.
struct SpanRun {
  int c;
  int nblk;
  const void* src;
  void* dst;
  int64_t numel;
  int32_t head;
};

struct PieceRun {
  int c;
  int nblk;
  const void* own;
  void* grad;
  int64_t pos;
  int64_t numel;
  int32_t head;
};

static_assert(kRunsPerLaunch < kBlock, "a wave-wide run lookup compares one table entry per lane");

struct SpanArgView {
  const SpanBatch& t;
  __device__ __forceinline__ int block() const { return int(blockIdx.x); }
  __device__ __forceinline__ SpanRun span_run(int blk) const {
    const int32_t end0 = t.first_block[1];
    const SpanRun r0{blk, end0, t.src[0], t.dst[0], t.numel[0], t.head[0]};
    if (blk < end0) return r0;  // first_block[0] == 0
    const int s = find_run_in(t.first_block, 1, t.count, blk);
    return {blk - t.first_block[s], t.first_block[s + 1] - t.first_block[s], t.src[s], t.dst[s], t.numel[s],
            t.head[s]};
  }
  // The same lookup in one round: lane k (k <= count) compares first_block[k]
  // with blk, and the runs that start at or before blk are counted from one
  // ballot.  Every lane of the wave must reach it.  (Measured on 48-span fp32
  // -> bf16 casts with two fragments per lane: 6514 GB/s, against 6149 with
  // the binary search; with one fragment per lane it is the slower of the two.)
  __device__ __forceinline__ SpanRun span_run_wave(int blk) const {
    const int k = int(threadIdx.x);
    const int32_t first = k <= t.count ? t.first_block[k] : INT32_MAX;
    const int s = __popcll(__ballot(first <= blk)) - 1;
    return {blk - t.first_block[s], t.first_block[s + 1] - t.first_block[s], t.src[s], t.dst[s], t.numel[s],
            t.head[s]};
  }
};

struct PieceArgView {
  const PieceBatch& t;
  __device__ __forceinline__ int block() const { return int(blockIdx.x); }
  __device__ __forceinline__ PieceRun piece_run(int blk) const {
    const int32_t end0 = t.first_block[1];
    const PieceRun r0{blk, end0, t.own[0], t.grad[0], t.pos[0], t.numel[0], t.head[0]};
    if (blk < end0) return r0;  // first_block[0] == 0
    const int s = find_run_in(t.first_block, 1, t.count, blk);
    return {blk - t.first_block[s], t.first_block[s + 1] - t.first_block[s], t.own[s], t.grad[s], t.pos[s],
            t.numel[s], t.head[s]};
  }
};

// One-run tables: the kernel-argument form of a dispatch with a single run,
// such as an FSDP unit's cast or reduce-scatter share.  Measured on 23 MB
// casts, a dispatch whose table is 1.6 KB of kernel arguments takes 0.25 us
// longer than one whose arguments are a few dozen bytes, and a scalar load
// that waits on another (the run lookup) 0.29 us more: these tables hold just
// the run, and every field is read in one round.
struct SpanOne {
  const void* src;
  void* dst;
  int64_t numel;
  int32_t head;
  int32_t blocks;
};

struct PieceOne {
  const void* own;
  void* grad;
  int64_t pos;
  int64_t numel;
  int32_t head;
  int32_t blocks;
};

inline SpanOne one_run_of(const SpanBatch& b) {
  return {b.src[0], b.dst[0], b.numel[0], b.head[0], b.first_block[1]};
}

inline PieceOne one_run_of(const PieceBatch& b) {
  return {b.own[0], b.grad[0], b.pos[0], b.numel[0], b.head[0], b.first_block[1]};
}

// Few-piece tables: up to kFewRuns pieces (an FSDP shard that spans a few
// parameters).  Every field of every piece is read in the same scalar round
// and the workgroup's piece is picked with compares and selects, so no load
// waits on another; the table is ~170 bytes instead of ~1.9 KB.
constexpr int kFewRuns = 4;

struct PieceFew {
  const void* own[kFewRuns];
  void* grad[kFewRuns];
  int64_t pos[kFewRuns];
  int64_t numel[kFewRuns];
  int32_t head[kFewRuns];
  int32_t first_block[kFewRuns + 1];  // entries past the last piece hold INT32_MAX
};

inline PieceFew few_runs_of(const PieceBatch& b) {
  PieceFew f{};
  for (int k = 0; k < kFewRuns; ++k) {
    const bool used = k < b.count;
    f.own[k] = used ? b.own[k] : nullptr;
    f.grad[k] = used ? b.grad[k] : nullptr;
    f.pos[k] = used ? b.pos[k] : 0;
    f.numel[k] = used ? b.numel[k] : 0;
    f.head[k] = used ? b.head[k] : -1;
  }
  for (int k = 0; k <= kFewRuns; ++k) f.first_block[k] = k <= b.count ? b.first_block[k] : INT32_MAX;
  return f;
}

struct PieceFewView {
  const PieceFew& t;
  __device__ __forceinline__ int block() const { return int(blockIdx.x); }
  __device__ __forceinline__ PieceRun piece_run(int blk) const {
    int32_t lo = t.first_block[0], hi = t.first_block[1];
    const void* own = t.own[0];
    void* grad = t.grad[0];
    int64_t pos = t.pos[0], numel = t.numel[0];
    int32_t head = t.head[0];
#pragma unroll
    for (int k = 1; k < kFewRuns; ++k) {
      const bool in = blk >= t.first_block[k];
      lo = in ? t.first_block[k] : lo;
      hi = in ? t.first_block[k + 1] : hi;
      own = in ? t.own[k] : own;
      grad = in ? t.grad[k] : grad;
      pos = in ? t.pos[k] : pos;
      numel = in ? t.numel[k] : numel;
      head = in ? t.head[k] : head;
    }
    return {blk - lo, hi - lo, own, grad, pos, numel, head};
  }
};

struct SpanOneView {
  const SpanOne& t;
  __device__ __forceinline__ int block() const { return int(blockIdx.x); }
  __device__ __forceinline__ SpanRun span_run(int blk) const { return {blk, t.blocks, t.src, t.dst, t.numel, t.head}; }
};

struct PieceOneView {
  const PieceOne& t;
  __device__ __forceinline__ int block() const { return int(blockIdx.x); }
  __device__ __forceinline__ PieceRun piece_run(int blk) const {
    return {blk, t.blocks, t.own, t.grad, t.pos, t.numel, t.head};
  }
};

// A device plan's a / b columns hold the span's src / dst or the piece's
// own / grad pointers.
struct DevView {
  DevTable t;
  __device__ __forceinline__ int block() const { return t.base + int(blockIdx.x); }
  __device__ __forceinline__ SpanRun span_run(int blk) const {
    const int s = find_run_hinted(t.first_block, t.hint, blk);
    return {blk - t.first_block[s], t.first_block[s + 1] - t.first_block[s], reinterpret_cast<const void*>(t.a[s]),
            reinterpret_cast<void*>(t.b[s]), t.numel[s], t.head[s]};
  }
  __device__ __forceinline__ PieceRun piece_run(int blk) const {
    const int s = find_run_hinted(t.first_block, t.hint, blk);
    return {blk - t.first_block[s], t.first_block[s + 1] - t.first_block[s], reinterpret_cast<const void*>(t.a[s]),
            reinterpret_cast<void*>(t.b[s]), t.pos[s], t.numel[s], t.head[s]};
  }
};

// Plan blob: this header followed by the DevTable arrays at the recorded
// byte offsets.  The same bytes live on the host (read at launch for the grid
// size and kernel arguments) and in device memory (read by the kernel).
constexpr uint32_t kPlanMagic = 0x5058444du;  // "MDXP"
enum : int32_t { kPlanSpans = 1, kPlanGradRuns = 2, kPlanPackRuns = 3, kPlanSharePieces = 4 };

struct PlanHeader {
  uint32_t magic;
  int32_t kind;
  int32_t count;
  int32_t blocks;
  int32_t dtype_a;  // spans: source dtype   grad runs: contribution dtype
  int32_t dtype_b;  // spans: dest dtype     grad runs: gradient dtype
  int32_t world;
  int32_t reserved;
  int32_t reduce_dtype;  // grad runs: bucket (out) dtype; differs from dtype_a when widening
  float prescale;        // grad runs: receiver-side pre-scale of every contribution (widening only);
                         // pack runs: the 1/W factor (pack side, or receiver side when widening)
  int32_t rank;          // pack runs: the replica this rank packs into
  int32_t pad;
  uint64_t replicas[MDX_MAX_WORLD];
  uint64_t out;
  int64_t off_first_block, off_head, off_numel, off_a, off_b, off_pos;
  int64_t bytes;
  int64_t off_hint;
};

hipError_t launch_copy_dev(int src_dtype, int dst_dtype, const DevTable& t, int blocks, const CopyParams& p,
                           hipStream_t stream);
hipError_t launch_allreduce_dev(int dtype, int grad_dtype, int world, const DevTable& t, int blocks,
                                const ReduceParams& p, hipStream_t stream);
hipError_t launch_allreduce_wide_dev(int wire_dtype, int grad_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream);
// Pack fused into the all-reduce + unpack (gradients of the wire dtype; the
// bucket dtype equals it or is fp32 for bf16 / fp16 wires).
hipError_t launch_pack_allreduce(int wire_dtype, int reduce_dtype, int world, const PieceBatch& b,
                                 const ReduceParams& p, hipStream_t stream);
hipError_t launch_pack_allreduce_dev(int wire_dtype, int reduce_dtype, int world, const DevTable& t, int blocks,
                                     const ReduceParams& p, hipStream_t stream);
// Multi-unit reduce-scatter share over a plan (fp32 reduction into fp32 shards).
hipError_t launch_share_fast_dev(int in_dtype, int wmax, const DevTable& t, int blocks, const ReduceParams& p,
                                 hipStream_t stream);

inline int dtype_size(int dt) { return dt == MDX_F32 ? 4 : 2; }

}  // namespace mdx
