// extern "C" entry points of libmdx.so (declared in include/mdx.h).
//
// Host-side work per call: validate every argument before anything is
// launched, cut the caller's span / piece list into runs of at most
// kMaxRunElems elements, compute for each run the element offset ("head")
// that brings all of its pointers to 16-byte alignment and its workgroup
// count, then either pack the runs into kernel-argument batches of at most
// kRunsPerLaunch (the direct entry points) or write them into a plan that the
// caller keeps in device memory (the mdx_plan_* / *_planned entry points: one
// dispatch for any number of runs).  Nothing here allocates device memory or
// synchronises.
#include <string.h>

#include <algorithm>
#include <mutex>

#include "mdx_internal.h"

namespace mdx {
namespace {

inline bool valid_dtype(int d) { return d == MDX_F32 || d == MDX_BF16 || d == MDX_F16; }

inline int status(hipError_t e) { return e == hipSuccess ? MDX_OK : int(e); }

inline uintptr_t addr(const void* p) { return reinterpret_cast<uintptr_t>(p); }

// The run's head: the h in [0, kHeadRange) after which the most pointers --
// each (pointer, element size, weight), stored streams weighing double --
// are 16-byte aligned (the smallest such h on a tie); -1 if the run has no
// full fragment of E elements after it.  The vector body accesses every
// stream with 16-byte (or 8-byte) vector instructions whatever its alignment
// (the memory pipeline splits an unaligned access); the head picks which
// streams get the aligned ones, so a gradient view that shares no alignment
// with its bucket rows still moves in vectors.
int aligned_head(const uintptr_t* ptrs, const int* sizes, const int* weights, int count, int E, int64_t n) {
  int best = 0, best_score = -1;
  for (int h = 0; h < kHeadRange; ++h) {
    int score = 0;
    for (int k = 0; k < count; ++k) {
      if (((ptrs[k] + uintptr_t(h) * uintptr_t(sizes[k])) & 15u) == 0) score += weights[k];
    }
    if (score > best_score) {
      best = h;
      best_score = score;
    }
  }
  return (n >= int64_t(best) + E) ? best : -1;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroups needed by one run: the aligned body in chunks of `vec_per_block`
// fragments, or the whole run in chunks of `elems_per_block` scalars.
int32_t run_blocks(int64_t n, int head, int E, int64_t vec_per_block, int64_t elems_per_block) {
  if (head >= 0) {
    const int64_t nvec = (n - head) / E;
    return int32_t(std::max<int64_t>(1, ceil_div(nvec, vec_per_block)));
  }
  return int32_t(std::max<int64_t>(1, ceil_div(n, elems_per_block)));
}

// One run of kernel work, whichever table it ends up in.
struct Rec {
  const void* a;  // span src / piece own
  void* b;        // span dst / piece grad
  int64_t pos;
  int64_t numel;
  int32_t head;
  int32_t blocks;
};

// ---------------------------------------------------------------------------
// Run generation
// ---------------------------------------------------------------------------

template <typename Emit>
int for_each_span_run(const mdx_span* spans, int n_spans, int sdt, int ddt, bool in_place, Emit&& emit) {
  const int E = copy_frag_elems(sdt, ddt);
  const int ss = dtype_size(sdt), ds = dtype_size(ddt);
  const int64_t VPB = int64_t(kBlock) * copy_unroll_of(ss, ds);
  const int64_t EPB = VPB * E;
  for (int i = 0; i < n_spans; ++i) {
    const mdx_span& sp = spans[i];
    const char* src = static_cast<const char*>(in_place ? sp.dst : sp.src);
    char* dst = static_cast<char*>(sp.dst);
    for (int64_t done = 0; done < sp.numel; done += kMaxRunElems) {
      const int64_t n = std::min<int64_t>(kMaxRunElems, sp.numel - done);
      const void* rs = src ? src + done * ss : nullptr;
      void* rd = dst + done * ds;
      uintptr_t ptrs[2];
      int sizes[2], weights[2] = {2, 1};  // the destination (stored) first
      int np = 0;
      ptrs[np] = addr(rd);
      sizes[np++] = ds;
      if (rs) {
        ptrs[np] = addr(rs);
        sizes[np++] = ss;
      }
      const int head = aligned_head(ptrs, sizes, weights, np, E, n);
      const int rc = emit(Rec{rs, rd, 0, n, head, run_blocks(n, head, E, VPB, EPB)});
      if (rc != MDX_OK) return rc;
    }
  }
  return MDX_OK;
}

// `grads` (may be NULL) adds each piece's gradient pointer, of `grad_size`
// bytes per element, to the alignment requirement (fused unpack); `own_row`
// adds replica `rank`'s row (written by the fused pack).
template <typename Emit>
int for_each_piece_run(const mdx_piece* pieces, void* const* grads, int n_pieces, const ReduceParams& params,
                       int in_size, int out_size, int grad_size, int E, int U, Emit&& emit,
                       bool own_row = false) {
  const int64_t VPB = int64_t(kBlock) * U;
  const int64_t EPB = VPB * E;
  for (int i = 0; i < n_pieces; ++i) {
    const mdx_piece& pc = pieces[i];
    const char* own = static_cast<const char*>(pc.own);
    char* grad = grads ? static_cast<char*>(grads[i]) : nullptr;
    for (int64_t done = 0; done < pc.numel; done += kMaxRunElems) {
      const int64_t n = std::min<int64_t>(kMaxRunElems, pc.numel - done);
      const int64_t pos = pc.pos + done;
      uintptr_t ptrs[MDX_MAX_WORLD + 3];
      int sizes[MDX_MAX_WORLD + 3], weights[MDX_MAX_WORLD + 3];
      int np = 0;
      const void* ro = own ? own + done * in_size : nullptr;
      void* rg = grad ? grad + done * grad_size : nullptr;
      if (ro) {
        ptrs[np] = addr(ro);
        weights[np] = 1;
        sizes[np++] = in_size;
      }
      for (int r = 0; r < params.world; ++r) {
        if (r == params.rank && !own_row) continue;
        ptrs[np] = addr(params.peer[r]) + uintptr_t(pos) * uintptr_t(in_size);
        weights[np] = (r == params.rank) ? 2 : 1;  // the fused pack stores this rank's row
        sizes[np++] = in_size;
      }
      if (params.out) {
        ptrs[np] = addr(params.out) + uintptr_t(pos) * uintptr_t(out_size);
        weights[np] = 2;
        sizes[np++] = out_size;
      }
      if (rg) {
        ptrs[np] = addr(rg);
        weights[np] = 2;
        sizes[np++] = grad_size;
      }
      const int head = aligned_head(ptrs, sizes, weights, np, E, n);
      const int rc = emit(Rec{ro, rg, pos, n, head, run_blocks(n, head, E, VPB, EPB)});
      if (rc != MDX_OK) return rc;
    }
  }
  return MDX_OK;
}

// ---------------------------------------------------------------------------
// Kernel-argument batches (direct entry points)
// ---------------------------------------------------------------------------

int run_copy(const mdx_span* spans, int n_spans, int sdt, int ddt, const CopyParams& params, bool in_place,
             hipStream_t stream) {
  SpanBatch b;
  memset(&b, 0, sizeof(b));
  CopyParams p = params;  // a requested flag clear rides on the first dispatch only
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int rc = status(launch_copy(sdt, ddt, b, p, stream));
    p.clear = nullptr;
    memset(&b, 0, sizeof(b));
    return rc;
  };
  const int rc = for_each_span_run(spans, n_spans, sdt, ddt, in_place, [&](const Rec& r) -> int {
    const int k = b.count;
    b.src[k] = r.a;
    b.dst[k] = r.b;
    b.numel[k] = r.numel;
    b.head[k] = r.head;
    b.first_block[k + 1] = b.first_block[k] + r.blocks;
    b.count = k + 1;
    return b.count == kRunsPerLaunch ? flush() : MDX_OK;
  });
  if (rc != MDX_OK) return rc;
  const int frc = flush();
  if (frc != MDX_OK) return frc;
  // nothing was launched: the clear still has to happen, in stream order
  return p.clear != nullptr ? status(launch_clear_flag(p.clear, stream)) : MDX_OK;
}

// Appends a run to a piece batch; `flush` launches and clears a full batch.
template <typename Flush>
int push_piece(PieceBatch& b, const Rec& r, Flush&& flush) {
  const int k = b.count;
  b.own[k] = r.a;
  b.grad[k] = r.b;
  b.pos[k] = r.pos;
  b.numel[k] = r.numel;
  b.head[k] = r.head;
  b.first_block[k + 1] = b.first_block[k] + r.blocks;
  b.count = k + 1;
  return b.count == kRunsPerLaunch ? flush() : MDX_OK;
}

template <typename Launch>
int run_pieces(const mdx_piece* pieces, void* const* grads, int n_pieces, const ReduceParams& params,
               int in_size, int out_size, int grad_size, int E, int U, Launch&& launch) {
  PieceBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int rc = status(launch(b));
    memset(&b, 0, sizeof(b));
    return rc;
  };
  const int rc = for_each_piece_run(pieces, grads, n_pieces, params, in_size, out_size, grad_size, E, U,
                                    [&](const Rec& r) { return push_piece(b, r, flush); });
  return rc != MDX_OK ? rc : flush();
}

// ---------------------------------------------------------------------------
// Device plans
// ---------------------------------------------------------------------------

inline int64_t align8(int64_t x) { return (x + 7) & ~int64_t(7); }

inline int64_t hint_groups(int64_t blocks) { return (blocks + kHintBlocks - 1) >> kHintShift; }

void plan_layout(PlanHeader* h, int count, int64_t blocks) {
  int64_t off = align8(sizeof(PlanHeader));
  h->off_first_block = off;
  off = align8(off + int64_t(count + 1) * 4);
  h->off_head = off;
  off = align8(off + int64_t(count) * 4);
  h->off_numel = off;
  off += int64_t(count) * 8;
  h->off_a = off;
  off += int64_t(count) * 8;
  h->off_b = off;
  off += int64_t(count) * 8;
  h->off_pos = off;
  off += int64_t(count) * 8;
  h->off_hint = off;
  off = align8(off + (hint_groups(blocks) + 1) * 4);
  h->bytes = off;
}

// Two passes over the runs: count, then (if the caller's buffer is large
// enough) write.  `gen(emit)` replays the same runs both times.
template <typename Gen>
int build_plan(PlanHeader proto, Gen&& gen, void* plan, int64_t* plan_bytes) {
  int count = 0;
  int64_t blocks = 0;
  int rc = gen([&](const Rec& r) -> int {
    ++count;
    blocks += r.blocks;
    return MDX_OK;
  });
  if (rc != MDX_OK) return rc;
  if (blocks > INT32_MAX) return MDX_EINVAL;
  PlanHeader h = proto;
  h.magic = kPlanMagic;
  h.count = count;
  h.blocks = int32_t(blocks);
  plan_layout(&h, count, blocks);
  const int64_t cap = *plan_bytes;
  *plan_bytes = h.bytes;
  if (plan == nullptr || cap < h.bytes || (addr(plan) & 7u) != 0) return MDX_ESIZE;
  char* base = static_cast<char*>(plan);
  memcpy(base, &h, sizeof(h));
  int32_t* fb = reinterpret_cast<int32_t*>(base + h.off_first_block);
  int32_t* hd = reinterpret_cast<int32_t*>(base + h.off_head);
  int64_t* nm = reinterpret_cast<int64_t*>(base + h.off_numel);
  uint64_t* a = reinterpret_cast<uint64_t*>(base + h.off_a);
  uint64_t* b = reinterpret_cast<uint64_t*>(base + h.off_b);
  int64_t* ps = reinterpret_cast<int64_t*>(base + h.off_pos);
  int k = 0;
  fb[0] = 0;
  rc = gen([&](const Rec& r) -> int {
    hd[k] = r.head;
    nm[k] = r.numel;
    a[k] = addr(r.a);
    b[k] = addr(r.b);
    ps[k] = r.pos;
    fb[k + 1] = fb[k] + r.blocks;
    ++k;
    return MDX_OK;
  });
  if (rc != MDX_OK) return rc;
  // Run hints (find_run_hinted): every run has at least one workgroup, so
  // first_block is strictly increasing and one forward sweep finds them.
  int32_t* hint = reinterpret_cast<int32_t*>(base + h.off_hint);
  const int64_t groups = hint_groups(blocks);
  int run = 0;
  for (int64_t g = 0; g < groups; ++g) {
    const int64_t b0 = g << kHintShift;
    while (run + 1 < count && fb[run + 1] <= b0) ++run;
    hint[g] = run;
  }
  hint[groups] = count - 1;
  return MDX_OK;
}

// Validates the host copy of a plan and derives the device table view.
int plan_view(const void* plan, const void* d_plan, int32_t kind, const PlanHeader** hdr, DevTable* t) {
  if (plan == nullptr || d_plan == nullptr) return MDX_EINVAL;
  const PlanHeader* h = static_cast<const PlanHeader*>(plan);
  if (h->magic != kPlanMagic || h->kind != kind) return MDX_EINVAL;
  const char* d = static_cast<const char*>(d_plan);
  t->first_block = reinterpret_cast<const int32_t*>(d + h->off_first_block);
  t->head = reinterpret_cast<const int32_t*>(d + h->off_head);
  t->numel = reinterpret_cast<const int64_t*>(d + h->off_numel);
  t->a = reinterpret_cast<const uint64_t*>(d + h->off_a);
  t->b = reinterpret_cast<const uint64_t*>(d + h->off_b);
  t->pos = reinterpret_cast<const int64_t*>(d + h->off_pos);
  t->hint = reinterpret_cast<const int32_t*>(d + h->off_hint);
  t->count = h->count;
  t->base = 0;
  *hdr = h;
  return MDX_OK;
}

// ---------------------------------------------------------------------------
// Validation helpers
// ---------------------------------------------------------------------------

int check_spans(const mdx_span* spans, int n_spans, bool need_src) {
  if (n_spans < 0 || (n_spans > 0 && spans == nullptr)) return MDX_EINVAL;
  for (int i = 0; i < n_spans; ++i) {
    if (spans[i].numel < 0) return MDX_EINVAL;
    if (spans[i].numel > 0 && spans[i].dst == nullptr) return MDX_EINVAL;
    if (need_src && spans[i].numel > 0 && spans[i].src == nullptr) return MDX_EINVAL;
  }
  return MDX_OK;
}

// [a, a+na) and [b, b+nb) share at least one byte.
bool any_overlap(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t a0 = addr(a), a1 = a0 + uintptr_t(na), b0 = addr(b), b1 = b0 + uintptr_t(nb);
  return na > 0 && nb > 0 && a0 < b1 && b0 < a1;
}

bool is_pow2(int w) { return w > 0 && (w & (w - 1)) == 0; }

// Arguments of a fused all-reduce + unpack, validated, with the kernel
// parameters and launch geometry they imply.
struct FusedArgs {
  ReduceParams p;
  int es, os, gs, E, U;
  bool any;
};

// `dtype` is the contributions' dtype, `out_dtype` the bucket's (equal, or
// bf16 / fp16 -> fp32 for the widening variant).
int check_fused(const void* const* replicas, int world, int dtype, int out_dtype, const mdx_grad_run* runs,
                int n_runs, void* out, int grad_dtype, FusedArgs* f) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype) || !valid_dtype(grad_dtype)) return MDX_EDTYPE;
  if (world < 1 || world > MDX_MAX_WORLD) return MDX_EWORLD;
  if (n_runs < 0 || (n_runs > 0 && runs == nullptr) || replicas == nullptr) return MDX_EINVAL;
  const int es = dtype_size(dtype), os = dtype_size(out_dtype), gs = dtype_size(grad_dtype);
  int64_t end = 0;
  bool any = false;
  for (int k = 0; k < n_runs; ++k) {
    if (runs[k].offset < 0 || runs[k].numel < 0 || runs[k].offset < end) return MDX_EINVAL;
    if (runs[k].numel > 0 && runs[k].grad == nullptr) return MDX_EINVAL;
    end = runs[k].offset + runs[k].numel;
    any = any || runs[k].numel > 0;
  }
  f->any = any;
  if (!any) return MDX_OK;
  // In place (out == a replica's base) is the same element read then written
  // by one lane, which needs equal element sizes; every other overlap races.
  const bool same_size = es == os;
  for (int r = 0; r < world; ++r) {
    if (replicas[r] == nullptr) return MDX_EINVAL;
    if (out && !(same_size && replicas[r] == out) && any_overlap(replicas[r], end * es, out, end * os)) {
      return MDX_EALIAS;
    }
  }
  for (int k = 0; k < n_runs; ++k) {
    const int64_t gb = runs[k].numel * gs;
    for (int r = 0; r < world; ++r) {
      if (any_overlap(runs[k].grad, gb, replicas[r], end * es)) return MDX_EALIAS;
    }
    if (out && any_overlap(runs[k].grad, gb, out, end * os)) return MDX_EALIAS;
  }
  memset(&f->p, 0, sizeof(f->p));
  for (int r = 0; r < world; ++r) f->p.peer[r] = replicas[r];
  f->p.out = out;
  f->p.world = world;
  f->p.rank = 0;  // replica 0 is read through the pieces, the others through peer[r] + pos
  f->p.pre = 1.0f;
  f->p.inv_scale = 1.0f;
  f->es = es;
  f->os = os;
  f->gs = gs;
  f->E = reduce_frag_elems(es, os, gs);  // as the kernel's compile-time fragment
  f->U = allreduce_unroll(world, f->E * es);
  return MDX_OK;
}

// The widening variant exists for bf16 or fp16 contributions into fp32 buckets.
bool wide_dtypes(int dtype, int out_dtype) {
  return (dtype == MDX_BF16 || dtype == MDX_F16) && out_dtype == MDX_F32;
}

// Replays the fused runs as (piece, grad) runs.
template <typename Emit>
int for_each_fused_run(const void* const* replicas, const mdx_grad_run* runs, int n_runs, const FusedArgs& f,
                       Emit&& emit) {
  const char* base0 = static_cast<const char*>(replicas[0]);
  for (int k = 0; k < n_runs; ++k) {
    if (runs[k].numel == 0) continue;
    const mdx_piece pc{base0 + runs[k].offset * f.es, runs[k].offset, runs[k].numel};
    void* grad = runs[k].grad;
    const int rc = for_each_piece_run(&pc, &grad, 1, f.p, f.es, f.os, f.gs, f.E, f.U, emit);
    if (rc != MDX_OK) return rc;
  }
  return MDX_OK;
}

// Plan of a fused all-reduce + unpack (widening when out_dtype != dtype).
int plan_grad_runs(const void* const* replicas, int world, int dtype, int out_dtype, const mdx_grad_run* runs,
                   int n_runs, void* out, int grad_dtype, float prescale, void* plan, int64_t* plan_bytes) {
  if (plan_bytes == nullptr) return MDX_EINVAL;
  FusedArgs f;
  const int rc = check_fused(replicas, world, dtype, out_dtype, runs, n_runs, out, grad_dtype, &f);
  if (rc != MDX_OK) return rc;
  PlanHeader proto;
  memset(&proto, 0, sizeof(proto));
  proto.kind = kPlanGradRuns;
  proto.dtype_a = dtype;
  proto.dtype_b = grad_dtype;
  proto.reduce_dtype = out_dtype;
  proto.prescale = prescale;
  proto.world = world;
  if (f.any) {
    for (int r = 0; r < world; ++r) proto.replicas[r] = addr(replicas[r]);
    proto.out = addr(out);
  }
  auto gen = [&](auto&& emit) { return f.any ? for_each_fused_run(replicas, runs, n_runs, f, emit) : MDX_OK; };
  return build_plan(proto, gen, plan, plan_bytes);
}

// Arguments of a fused pack + all-reduce + unpack, validated.  The kernel
// parameters are those of the fused all-reduce + unpack with replica `rank`
// read from each run's gradient and written by the pack.
int check_pack_fused(const void* const* replicas, int world, int rank, int dtype, int out_dtype,
                     const mdx_pack_run* runs, int n_runs, void* out, float scale, int32_t* found_inf,
                     int32_t* clear_flag, FusedArgs* f) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return MDX_EDTYPE;
  if (dtype != out_dtype && !wide_dtypes(dtype, out_dtype)) return MDX_EDTYPE;
  if (world < 1 || world > MDX_MAX_WORLD || rank < 0 || rank >= world) return MDX_EWORLD;
  if (n_runs < 0 || (n_runs > 0 && runs == nullptr) || replicas == nullptr) return MDX_EINVAL;
  if (clear_flag != nullptr && clear_flag == found_inf) return MDX_EALIAS;
  const int es = dtype_size(dtype), os = dtype_size(out_dtype);
  int64_t end = 0;
  bool any = false;
  for (int k = 0; k < n_runs; ++k) {
    if (runs[k].offset < 0 || runs[k].numel < 0 || runs[k].offset < end) return MDX_EINVAL;
    if (runs[k].numel > 0 && runs[k].grad == nullptr) return MDX_EINVAL;
    end = runs[k].offset + runs[k].numel;
    any = any || runs[k].numel > 0;
  }
  memset(&f->p, 0, sizeof(f->p));
  f->any = any;
  f->p.clear = clear_flag;
  if (!any) return MDX_OK;
  // The pack writes row `rank` and the bucket is written beside the rows: the
  // bucket must not overlap any replica, a gradient (read and written by the
  // same lane) neither the replicas nor the bucket.
  for (int r = 0; r < world; ++r) {
    if (replicas[r] == nullptr) return MDX_EINVAL;
    if (out && any_overlap(replicas[r], end * es, out, end * os)) return MDX_EALIAS;
  }
  for (int k = 0; k < n_runs; ++k) {
    const int64_t gb = runs[k].numel * es;
    for (int r = 0; r < world; ++r) {
      if (any_overlap(runs[k].grad, gb, replicas[r], end * es)) return MDX_EALIAS;
      if (runs[k].src && any_overlap(runs[k].src, gb, replicas[r], end * es)) return MDX_EALIAS;
    }
    if (out && any_overlap(runs[k].grad, gb, out, end * os)) return MDX_EALIAS;
    if (out && runs[k].src && any_overlap(runs[k].src, gb, out, end * os)) return MDX_EALIAS;
    if (runs[k].src && runs[k].src != runs[k].grad && any_overlap(runs[k].src, gb, runs[k].grad, gb)) {
      return MDX_EALIAS;
    }
  }
  for (int r = 0; r < world; ++r) f->p.peer[r] = replicas[r];
  f->p.out = out;
  f->p.world = world;
  f->p.rank = rank;
  f->p.pre = scale;
  f->p.inv_scale = 1.0f;
  f->p.found_inf = found_inf;
  f->p.flags = (dtype == out_dtype && scale != 1.0f) ? kRedPackScale : 0;
  f->es = es;
  f->os = os;
  f->gs = es;
  f->E = reduce_frag_elems(es, os, es);  // as the kernel's compile-time fragment
  f->U = pack_allreduce_unroll();
  return MDX_OK;
}

// Replays the pack runs as (gradient source, gradient) runs of the kernel.
template <typename Emit>
int for_each_pack_run(const mdx_pack_run* runs, int n_runs, const FusedArgs& f, Emit&& emit) {
  for (int k = 0; k < n_runs; ++k) {
    if (runs[k].numel == 0) continue;
    const mdx_piece pc{runs[k].src, runs[k].offset, runs[k].numel};
    void* grad = runs[k].grad;
    const int rc = for_each_piece_run(&pc, &grad, 1, f.p, f.es, f.os, f.gs, f.E, f.U, emit, true);
    if (rc != MDX_OK) return rc;
  }
  return MDX_OK;
}

// The pre-scale / accumulate / unscale flags of a reduce-scatter share.
void share_flags(int world, int divide, int accumulate, float inv_scale, ReduceParams* p) {
  int32_t flags = 0;
  p->pre = 1.0f;
  if (divide && world > 1) {
    // x / W and x * (1/W) are the same correctly rounded value when 1/W is
    // exact, i.e. for power-of-two W; the multiply is the cheaper instruction.
    if (is_pow2(world)) {
      flags |= kRedPreMul;
      p->pre = 1.0f / float(world);
    } else {
      flags |= kRedPreDiv;
      p->pre = float(world);
    }
  }
  if (accumulate) flags |= kRedAccumulate;
  if (inv_scale != 1.0f) flags |= kRedUnscale;
  p->flags = flags;
  p->inv_scale = inv_scale;
}

// Arguments of a multi-unit share, validated: pieces at absolute positions of
// the contribution rows `peers`, each with a destination of its own.
int check_share_multi(const mdx_piece* pieces, void* const* outs, int n, const void* const* peers, int world,
                      int rank, int in_dtype, int reduce_dtype, int shard_dtype, ReduceParams* p, bool* any) {
  if (!valid_dtype(in_dtype) || !valid_dtype(reduce_dtype) || !valid_dtype(shard_dtype)) return MDX_EDTYPE;
  if (world < 1 || world > MDX_MAX_WORLD || rank < 0 || rank >= world) return MDX_EWORLD;
  if (n < 0 || (n > 0 && (pieces == nullptr || outs == nullptr))) return MDX_EINVAL;
  if (world > 1 && peers == nullptr) return MDX_EINVAL;
  const int is = dtype_size(in_dtype), os = dtype_size(shard_dtype);
  int64_t extent = 0;
  *any = false;
  for (int i = 0; i < n; ++i) {
    if (pieces[i].numel < 0 || pieces[i].pos < 0) return MDX_EINVAL;
    if (pieces[i].numel == 0) continue;
    if (outs[i] == nullptr) return MDX_EINVAL;
    *any = true;
    extent = std::max<int64_t>(extent, pieces[i].pos + pieces[i].numel);
  }
  memset(p, 0, sizeof(*p));
  p->rank = rank;
  p->world = world;
  if (!*any) return MDX_OK;
  for (int r = 0; r < world; ++r) {
    if (r == rank) continue;
    if (peers[r] == nullptr) return MDX_EINVAL;
    p->peer[r] = peers[r];
  }
  // Every destination must be clear of the rows, of every piece's own data and
  // of every other destination (workgroups of different pieces run unordered).
  for (int i = 0; i < n; ++i) {
    const int64_t ob = pieces[i].numel * os;
    if (ob == 0) continue;
    for (int r = 0; r < world; ++r) {
      if (r != rank && any_overlap(peers[r], extent * is, outs[i], ob)) return MDX_EALIAS;
    }
    for (int j = 0; j < n; ++j) {
      if (pieces[j].own && any_overlap(pieces[j].own, pieces[j].numel * is, outs[i], ob)) return MDX_EALIAS;
      if (j != i && any_overlap(outs[j], pieces[j].numel * os, outs[i], ob)) return MDX_EALIAS;
    }
  }
  return MDX_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free plan launch (mdx_pack_allreduce_unpack_planned_noalloc)
// ---------------------------------------------------------------------------

// The device copy of a plan launched without caller-allocated memory.  Each
// GPU the library runs on holds its own instance until the process ends.  In
// host code the name `scratch` is only a stand-in for the symbol: kernels and
// copies get the address hipGetSymbolAddress returns on the device
// (scratch_on), never the name.
__device__ __align__(256) unsigned char scratch[MDX_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];
hipError_t g_scratch_status[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];

// This device's address of `scratch`, resolved once per device while that
// device is current (the caller checked that it is).
hipError_t scratch_on(int device, unsigned char** out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_scratch_once[device], [device]() {
    void* p = nullptr;
    g_scratch_status[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[device] = p;
  });
  *out = static_cast<unsigned char*>(g_scratch[device]);
  return g_scratch_status[device];
}

// Plan bytes per upload dispatch.  The chunk is a kernel argument: the
// runtime copies it when the dispatch is enqueued, so the caller's host plan
// is free to change once the call returns, and nothing waits for the stream.
constexpr int kUploadWords = 768;  // 3 KB

struct UploadChunk {
  uint32_t word[kUploadWords];
  int64_t offset;  // byte offset of word[0] in the buffer (a multiple of 4)
  int32_t count;   // words of this chunk, at most kUploadWords
};

__global__ void __launch_bounds__(kBlock) upload_kernel(UploadChunk c, unsigned char* dst) {
  uint32_t* out = reinterpret_cast<uint32_t*>(dst + c.offset);
  for (int i = int(threadIdx.x); i < c.count; i += kBlock) out[i] = c.word[i];
}

// Copies plan bytes [0, bytes) into `dst` with upload dispatches on `stream`.
int upload_plan(const void* plan, int64_t bytes, unsigned char* dst, hipStream_t stream) {
  const unsigned char* src = static_cast<const unsigned char*>(plan);
  UploadChunk c;
  for (int64_t off = 0; off < bytes; off += int64_t(kUploadWords) * 4) {
    const int64_t n = std::min<int64_t>(int64_t(kUploadWords) * 4, bytes - off);
    c.offset = off;
    c.count = int32_t(n / 4);
    memcpy(c.word, src + off, size_t(n));
    hipLaunchKernelGGL(upload_kernel, dim3(1), dim3(kBlock), 0, stream, c, dst);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return int(e);
  }
  return MDX_OK;
}

// A plan's table offsets are the ones its own counts give (plan_layout), so
// every array the kernel reads lies inside its `bytes`.
bool plan_layout_matches(const PlanHeader* h) {
  if (h->count < 0 || h->blocks < 0) return false;
  PlanHeader ref = *h;
  plan_layout(&ref, h->count, h->blocks);
  return ref.bytes == h->bytes && ref.off_first_block == h->off_first_block && ref.off_head == h->off_head &&
         ref.off_numel == h->off_numel && ref.off_a == h->off_a && ref.off_b == h->off_b &&
         ref.off_pos == h->off_pos && ref.off_hint == h->off_hint;
}

// The device `stream` runs on, which must be the current one.
int stream_device(hipStream_t stream, int* device) {
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return int(e);
  int owner = current;
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, &owner);
    if (e != hipSuccess) return int(e);
  }
  if (owner != current) return MDX_ESCRATCH;
  *device = current;
  return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" {

int mdx_abi_version(void) { return MDX_ABI_VERSION; }

const char* mdx_strerror(int code) {
  switch (code) {
    case MDX_OK: return "success";
    case MDX_EINVAL: return "mdx: invalid argument (NULL pointer, negative count or size, bad plan)";
    case MDX_EDTYPE: return "mdx: unsupported dtype code or combination (MDX_F32, MDX_BF16, MDX_F16)";
    case MDX_EWORLD: return "mdx: world size outside [1, MDX_MAX_WORLD] or rank outside [0, world)";
    case MDX_EALIAS: return "mdx: output overlaps an input it must not overlap";
    case MDX_ESIZE: return "mdx: plan buffer missing or too small (required size returned)";
    case MDX_ESCRATCH:
      return "mdx: plan larger than MDX_NOALLOC_SCRATCH_BYTES (256 KiB), or stream not on the current device";
    case MDX_EOP: return "mdx: unsupported reduction op (MDX_OP_SUM, MDX_OP_PRODUCT, MDX_OP_MIN, MDX_OP_MAX)";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "mdx: unknown status code";
}

int mdx_pack(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, float scale,
             int divide, int32_t* clear_flag, void* stream) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return MDX_EDTYPE;
  int rc = check_spans(spans, n_spans, false);
  if (rc != MDX_OK) return rc;
  int32_t flags = 0;
  if (scale != 1.0f) flags = divide ? kCopyDivide : kCopyScale;
  CopyParams p{scale, flags, nullptr, clear_flag};
  return run_copy(spans, n_spans, src_dtype, dst_dtype, p, false, static_cast<hipStream_t>(stream));
}

int mdx_unpack(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, float inv_scale,
               int32_t* found_inf, void* stream) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return MDX_EDTYPE;
  int rc = check_spans(spans, n_spans, true);
  if (rc != MDX_OK) return rc;
  CopyParams p{inv_scale, (inv_scale != 1.0f ? kCopyScale : 0) | (found_inf ? kCopyCheck : 0),
               found_inf, nullptr};
  return run_copy(spans, n_spans, src_dtype, dst_dtype, p, false, static_cast<hipStream_t>(stream));
}

int mdx_unscale_found_inf(const mdx_span* spans, int n_spans, int dtype, float inv_scale,
                          int32_t* found_inf, void* stream) {
  if (!valid_dtype(dtype)) return MDX_EDTYPE;
  int rc = check_spans(spans, n_spans, false);
  if (rc != MDX_OK) return rc;
  CopyParams p{inv_scale, (inv_scale != 1.0f ? kCopyScale : 0) | (found_inf ? kCopyCheck : 0),
               found_inf, nullptr};
  return run_copy(spans, n_spans, dtype, dtype, p, true, static_cast<hipStream_t>(stream));
}

int mdx_cast_f32_bf16(const float* src, uint16_t* dst, int64_t numel, void* stream) {
  if (numel < 0 || (numel > 0 && (src == nullptr || dst == nullptr))) return MDX_EINVAL;
  if (any_overlap(src, numel * 4, dst, numel * 2)) return MDX_EALIAS;
  mdx_span sp{src, dst, numel};
  CopyParams p{1.0f, 0, nullptr, nullptr};
  return run_copy(&sp, 1, MDX_F32, MDX_BF16, p, false, static_cast<hipStream_t>(stream));
}

int mdx_allreduce_op(const void* const* replicas, int world, int dtype, int op, const int64_t* offsets,
                     const int64_t* numels, int n_runs, void* out, void* stream) {
  if (op == MDX_OP_SUM) return mdx_allreduce_sum(replicas, world, dtype, offsets, numels, n_runs, out, stream);
  if (op != MDX_OP_PRODUCT && op != MDX_OP_MIN && op != MDX_OP_MAX) return MDX_EOP;
  if (!valid_dtype(dtype)) return MDX_EDTYPE;
  if (world < 1 || world > MDX_MAX_WORLD) return MDX_EWORLD;
  if (n_runs < 0 || replicas == nullptr) return MDX_EINVAL;
  if (n_runs > 0 && (offsets == nullptr || numels == nullptr)) return MDX_EINVAL;
  int64_t end = 0;
  bool any = false;
  for (int k = 0; k < n_runs; ++k) {
    if (offsets[k] < 0 || numels[k] < 0 || offsets[k] < end) return MDX_EINVAL;
    end = offsets[k] + numels[k];
    any = any || numels[k] > 0;
  }
  if (!any) return MDX_OK;
  if (out == nullptr) return MDX_EINVAL;
  const int es = dtype_size(dtype);
  OpParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < world; ++r) {
    if (replicas[r] == nullptr) return MDX_EINVAL;
    // Same base = the in-place case; any other overlap of the reduced extent is rejected.
    if (replicas[r] != out && any_overlap(replicas[r], end * es, out, end * es)) return MDX_EALIAS;
    p.rep[r] = replicas[r];
  }
  p.out = out;
  p.world = world;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int wmax = op_wmax(world);
  const int64_t elems_per_block = op_elems_per_block(es, wmax);
  OpRuns t;
  memset(&t, 0, sizeof(t));
  int blocks = 0;
  auto flush = [&]() -> int {
    if (t.count == 0) return MDX_OK;
    t.first_block[t.count] = blocks;
    const int r = status(launch_allreduce_op(dtype, op, wmax, t, blocks, p, st));
    memset(&t, 0, sizeof(t));
    blocks = 0;
    return r;
  };
  for (int k = 0; k < n_runs; ++k) {
    // runs of at most kMaxRunElems elements keep every dispatch far below 2^31 workgroups
    for (int64_t a = 0; a < numels[k]; a += kMaxRunElems) {
      if (t.count == kRunsPerLaunch) {
        const int rc = flush();
        if (rc != MDX_OK) return rc;
      }
      const int64_t n = min_i64(kMaxRunElems, numels[k] - a);
      t.offset[t.count] = offsets[k] + a;
      t.numel[t.count] = n;
      t.first_block[t.count] = blocks;
      blocks += int((n + elems_per_block - 1) / elems_per_block);
      ++t.count;
    }
  }
  return flush();
}

int mdx_allreduce_sum(const void* const* replicas, int world, int dtype, const int64_t* offsets,
                      const int64_t* numels, int n_runs, void* out, void* stream) {
  if (!valid_dtype(dtype)) return MDX_EDTYPE;
  if (world < 1 || world > MDX_MAX_WORLD) return MDX_EWORLD;
  if (n_runs < 0 || replicas == nullptr) return MDX_EINVAL;
  if (n_runs > 0 && (offsets == nullptr || numels == nullptr)) return MDX_EINVAL;
  int64_t end = 0;
  bool any = false;
  for (int k = 0; k < n_runs; ++k) {
    if (offsets[k] < 0 || numels[k] < 0 || offsets[k] < end) return MDX_EINVAL;
    end = offsets[k] + numels[k];
    any = any || numels[k] > 0;
  }
  if (!any) return MDX_OK;
  if (out == nullptr) return MDX_EINVAL;
  const int es = dtype_size(dtype);
  for (int r = 0; r < world; ++r) {
    if (replicas[r] == nullptr) return MDX_EINVAL;
    // Same base = the in-place case; any other overlap of the reduced extent is rejected.
    if (replicas[r] != out && any_overlap(replicas[r], end * es, out, end * es)) return MDX_EALIAS;
  }
  ReduceParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < world; ++r) p.peer[r] = replicas[r];
  p.out = out;
  p.world = world;
  p.rank = 0;  // replica 0 is read through the pieces, the others through peer[r] + pos
  p.pre = 1.0f;
  p.inv_scale = 1.0f;
  const char* base0 = static_cast<const char*>(replicas[0]);
  const int E = store_frag_elems(es);
  const int U = allreduce_unroll(world, E * es);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](const PieceBatch& b) { return launch_allreduce(dtype, dtype, false, world, b, p, st); };
  PieceBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int r = status(launch(b));
    memset(&b, 0, sizeof(b));
    return r;
  };
  for (int k = 0; k < n_runs; ++k) {
    if (numels[k] == 0) continue;
    const mdx_piece pc{base0 + offsets[k] * es, offsets[k], numels[k]};
    const int rc = for_each_piece_run(&pc, nullptr, 1, p, es, es, 0, E, U,
                                      [&](const Rec& r) { return push_piece(b, r, flush); });
    if (rc != MDX_OK) return rc;
  }
  return flush();
}

int mdx_allreduce_unpack(const void* const* replicas, int world, int dtype, const mdx_grad_run* runs,
                         int n_runs, void* out, int grad_dtype, float inv_scale, int32_t* found_inf,
                         void* stream) {
  FusedArgs f;
  int rc = check_fused(replicas, world, dtype, dtype, runs, n_runs, out, grad_dtype, &f);
  if (rc != MDX_OK || !f.any) return rc;
  f.p.inv_scale = inv_scale;
  f.p.flags = inv_scale != 1.0f ? kRedUnscale : 0;
  f.p.found_inf = found_inf;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  PieceBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int r = status(launch_allreduce(dtype, grad_dtype, true, world, b, f.p, st));
    memset(&b, 0, sizeof(b));
    return r;
  };
  rc = for_each_fused_run(replicas, runs, n_runs, f, [&](const Rec& r) { return push_piece(b, r, flush); });
  return rc != MDX_OK ? rc : flush();
}

int mdx_allreduce_unpack_wide(const void* const* replicas, int world, int wire_dtype, const mdx_grad_run* runs,
                              int n_runs, void* out, int reduce_dtype, int grad_dtype, float prescale,
                              float inv_scale, int32_t* found_inf, void* stream) {
  if (!wide_dtypes(wire_dtype, reduce_dtype)) return MDX_EDTYPE;
  FusedArgs f;
  int rc = check_fused(replicas, world, wire_dtype, reduce_dtype, runs, n_runs, out, grad_dtype, &f);
  if (rc != MDX_OK || !f.any) return rc;
  f.p.pre = prescale;
  f.p.inv_scale = inv_scale;
  f.p.flags = inv_scale != 1.0f ? kRedUnscale : 0;
  f.p.found_inf = found_inf;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  PieceBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int r = status(launch_allreduce_wide(wire_dtype, grad_dtype, world, b, f.p, st));
    memset(&b, 0, sizeof(b));
    return r;
  };
  rc = for_each_fused_run(replicas, runs, n_runs, f, [&](const Rec& r) { return push_piece(b, r, flush); });
  return rc != MDX_OK ? rc : flush();
}

int mdx_pack_allreduce_unpack(const void* const* replicas, int world, int rank, int wire_dtype,
                              const mdx_pack_run* runs, int n_runs, void* out, int reduce_dtype, float scale,
                              float inv_scale, int32_t* found_inf, int32_t* clear_flag, void* stream) {
  FusedArgs f;
  int rc = check_pack_fused(replicas, world, rank, wire_dtype, reduce_dtype, runs, n_runs, out, scale, found_inf,
                            clear_flag, &f);
  if (rc != MDX_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (!f.any) return clear_flag != nullptr ? status(launch_clear_flag(clear_flag, st)) : MDX_OK;
  f.p.inv_scale = inv_scale;
  if (inv_scale != 1.0f) f.p.flags |= kRedUnscale;
  PieceBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int r = status(launch_pack_allreduce(wire_dtype, reduce_dtype, world, b, f.p, st));
    f.p.clear = nullptr;  // the flag clear rides on the first dispatch only
    memset(&b, 0, sizeof(b));
    return r;
  };
  rc = for_each_pack_run(runs, n_runs, f, [&](const Rec& r) { return push_piece(b, r, flush); });
  return rc != MDX_OK ? rc : flush();
}

int mdx_reduce_scatter_share(const mdx_piece* own, int n_own, const void* const* peers, int world,
                             int rank, int in_dtype, int reduce_dtype, int divide, void* shard,
                             int shard_dtype, int accumulate, float inv_scale, int32_t* found_inf,
                             void* stream) {
  if (!valid_dtype(in_dtype) || !valid_dtype(reduce_dtype) || !valid_dtype(shard_dtype)) {
    return MDX_EDTYPE;
  }
  if (world < 1 || world > MDX_MAX_WORLD || rank < 0 || rank >= world) return MDX_EWORLD;
  if (n_own < 0 || (n_own > 0 && own == nullptr)) return MDX_EINVAL;
  if (world > 1 && peers == nullptr) return MDX_EINVAL;
  int64_t extent = 0;
  bool any = false;
  for (int i = 0; i < n_own; ++i) {
    if (own[i].numel < 0 || own[i].pos < 0) return MDX_EINVAL;
    if (own[i].numel == 0) continue;
    any = true;
    extent = std::max<int64_t>(extent, own[i].pos + own[i].numel);
  }
  if (!any) return MDX_OK;
  if (shard == nullptr) return MDX_EINVAL;
  const int64_t out_bytes = extent * dtype_size(shard_dtype);
  ReduceParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < world; ++r) {
    if (r == rank) continue;
    if (peers[r] == nullptr) return MDX_EINVAL;
    if (any_overlap(peers[r], extent * dtype_size(in_dtype), shard, out_bytes)) return MDX_EALIAS;
    p.peer[r] = peers[r];
  }
  for (int i = 0; i < n_own; ++i) {
    if (own[i].own && any_overlap(own[i].own, own[i].numel * dtype_size(in_dtype), shard, out_bytes)) {
      return MDX_EALIAS;
    }
  }
  p.out = shard;
  p.rank = rank;
  p.world = world;
  p.found_inf = found_inf;
  share_flags(world, divide, accumulate, inv_scale, &p);
  const int is = dtype_size(in_dtype), os = dtype_size(shard_dtype);
  const int wmax = share_wmax(in_dtype, reduce_dtype, shard_dtype, world);
  const int E = reduce_frag_elems(is, os, os);  // as the kernel's compile-time fragment
  const int U = share_unroll(wmax, E * is);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](const PieceBatch& b) {
    return launch_share(in_dtype, reduce_dtype, shard_dtype, wmax, b, p, st);
  };
  return run_pieces(own, nullptr, n_own, p, is, os, 0, E, U, launch);
}

int mdx_reduce_scatter_share_multi(const mdx_piece* pieces, void* const* outs, int n_pieces,
                                   const void* const* peers, int world, int rank, int in_dtype, int reduce_dtype,
                                   int divide, int shard_dtype, int accumulate, float inv_scale, int32_t* found_inf,
                                   void* stream) {
  ReduceParams p;
  bool any = false;
  const int rc = check_share_multi(pieces, outs, n_pieces, peers, world, rank, in_dtype, reduce_dtype, shard_dtype,
                                   &p, &any);
  if (rc != MDX_OK || !any) return rc;
  p.found_inf = found_inf;
  share_flags(world, divide, accumulate, inv_scale, &p);
  const int is = dtype_size(in_dtype), os = dtype_size(shard_dtype);
  const int wmax = share_wmax(in_dtype, reduce_dtype, shard_dtype, world);
  const int E = reduce_frag_elems(is, os, os);  // as the kernel's compile-time fragment
  const int U = share_unroll(wmax, E * is);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](const PieceBatch& b) {
    return launch_share(in_dtype, reduce_dtype, shard_dtype, wmax, b, p, st);
  };
  return run_pieces(pieces, outs, n_pieces, p, is, os, os, E, U, launch);
}

int mdx_plan_reduce_scatter_share_multi(const mdx_piece* pieces, void* const* outs, int n_pieces,
                                        const void* const* peers, int world, int rank, int in_dtype, void* plan,
                                        int64_t* plan_bytes) {
  if (plan_bytes == nullptr) return MDX_EINVAL;
  ReduceParams p;
  bool any = false;
  const int rc = check_share_multi(pieces, outs, n_pieces, peers, world, rank, in_dtype, MDX_F32, MDX_F32, &p, &any);
  if (rc != MDX_OK) return rc;
  PlanHeader proto;
  memset(&proto, 0, sizeof(proto));
  proto.kind = kPlanSharePieces;
  proto.dtype_a = in_dtype;
  proto.dtype_b = MDX_F32;
  proto.reduce_dtype = MDX_F32;
  proto.world = world;
  proto.rank = rank;
  for (int r = 0; r < world; ++r) proto.replicas[r] = addr(p.peer[r]);
  const int is = dtype_size(in_dtype), os = 4;
  const int wmax = share_wmax(in_dtype, MDX_F32, MDX_F32, world);
  const int E = reduce_frag_elems(is, os, os);
  const int U = share_unroll(wmax, E * is);
  auto gen = [&](auto&& emit) {
    return any ? for_each_piece_run(pieces, outs, n_pieces, p, is, os, os, E, U, emit) : MDX_OK;
  };
  return build_plan(proto, gen, plan, plan_bytes);
}

int mdx_reduce_scatter_share_multi_planned(const void* plan, const void* d_plan, int divide, int accumulate,
                                           float inv_scale, int32_t* found_inf, void* stream) {
  const PlanHeader* h;
  DevTable t;
  const int rc = plan_view(plan, d_plan, kPlanSharePieces, &h, &t);
  if (rc != MDX_OK) return rc;
  if (h->count == 0) return MDX_OK;
  ReduceParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < h->world; ++r) p.peer[r] = reinterpret_cast<const void*>(h->replicas[r]);
  p.world = h->world;
  p.rank = h->rank;
  p.found_inf = found_inf;
  share_flags(h->world, divide, accumulate, inv_scale, &p);
  const int wmax = share_wmax(h->dtype_a, MDX_F32, MDX_F32, h->world);
  return status(launch_share_fast_dev(h->dtype_a, wmax, t, h->blocks, p, static_cast<hipStream_t>(stream)));
}

// -- device plans -------------------------------------------------------------

int mdx_plan_spans(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, void* plan,
                   int64_t* plan_bytes) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return MDX_EDTYPE;
  if (plan_bytes == nullptr) return MDX_EINVAL;
  const int rc = check_spans(spans, n_spans, false);
  if (rc != MDX_OK) return rc;
  PlanHeader proto;
  memset(&proto, 0, sizeof(proto));
  proto.kind = kPlanSpans;
  proto.dtype_a = src_dtype;
  proto.dtype_b = dst_dtype;
  for (int i = 0; i < n_spans; ++i) {
    if (spans[i].numel > 0 && spans[i].src == nullptr) proto.reserved = 1;  // some span reads zeros
  }
  auto gen = [&](auto&& emit) { return for_each_span_run(spans, n_spans, src_dtype, dst_dtype, false, emit); };
  return build_plan(proto, gen, plan, plan_bytes);
}

int mdx_plan_allreduce_unpack(const void* const* replicas, int world, int dtype, const mdx_grad_run* runs,
                              int n_runs, void* out, int grad_dtype, void* plan, int64_t* plan_bytes) {
  return plan_grad_runs(replicas, world, dtype, dtype, runs, n_runs, out, grad_dtype, 1.0f, plan, plan_bytes);
}

int mdx_plan_allreduce_unpack_wide(const void* const* replicas, int world, int wire_dtype,
                                   const mdx_grad_run* runs, int n_runs, void* out, int reduce_dtype,
                                   int grad_dtype, float prescale, void* plan, int64_t* plan_bytes) {
  if (!wide_dtypes(wire_dtype, reduce_dtype)) return MDX_EDTYPE;
  return plan_grad_runs(replicas, world, wire_dtype, reduce_dtype, runs, n_runs, out, grad_dtype, prescale, plan,
                        plan_bytes);
}

int mdx_plan_pack_allreduce_unpack(const void* const* replicas, int world, int rank, int wire_dtype,
                                   const mdx_pack_run* runs, int n_runs, void* out, int reduce_dtype, float scale,
                                   void* plan, int64_t* plan_bytes) {
  if (plan_bytes == nullptr) return MDX_EINVAL;
  FusedArgs f;
  const int rc = check_pack_fused(replicas, world, rank, wire_dtype, reduce_dtype, runs, n_runs, out, scale,
                                  nullptr, nullptr, &f);
  if (rc != MDX_OK) return rc;
  PlanHeader proto;
  memset(&proto, 0, sizeof(proto));
  proto.kind = kPlanPackRuns;
  proto.dtype_a = wire_dtype;
  proto.dtype_b = wire_dtype;
  proto.reduce_dtype = reduce_dtype;
  proto.prescale = scale;
  proto.world = world;
  proto.rank = rank;
  if (f.any) {
    for (int r = 0; r < world; ++r) proto.replicas[r] = addr(replicas[r]);
    proto.out = addr(out);
  }
  auto gen = [&](auto&& emit) { return f.any ? for_each_pack_run(runs, n_runs, f, emit) : MDX_OK; };
  return build_plan(proto, gen, plan, plan_bytes);
}

int mdx_pack_allreduce_unpack_planned(const void* plan, const void* d_plan, float inv_scale, int32_t* found_inf,
                                      int32_t* clear_flag, void* stream) {
  const PlanHeader* h;
  DevTable t;
  const int rc = plan_view(plan, d_plan, kPlanPackRuns, &h, &t);
  if (rc != MDX_OK) return rc;
  if (clear_flag != nullptr && clear_flag == found_inf) return MDX_EALIAS;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (h->count == 0) return clear_flag != nullptr ? status(launch_clear_flag(clear_flag, st)) : MDX_OK;
  ReduceParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < h->world; ++r) p.peer[r] = reinterpret_cast<const void*>(h->replicas[r]);
  p.out = reinterpret_cast<void*>(h->out);
  p.world = h->world;
  p.rank = h->rank;
  p.pre = h->prescale;
  p.inv_scale = inv_scale;
  p.flags = (h->dtype_a == h->reduce_dtype && h->prescale != 1.0f ? kRedPackScale : 0) |
            (inv_scale != 1.0f ? kRedUnscale : 0);
  p.found_inf = found_inf;
  p.clear = clear_flag;
  return status(launch_pack_allreduce_dev(h->dtype_a, h->reduce_dtype, h->world, t, h->blocks, p, st));
}

int mdx_pack_planned(const void* plan, const void* d_plan, float scale, int divide, int32_t* clear_flag,
                     void* stream) {
  const PlanHeader* h;
  DevTable t;
  const int rc = plan_view(plan, d_plan, kPlanSpans, &h, &t);
  if (rc != MDX_OK) return rc;
  if (h->count == 0) {
    return clear_flag != nullptr ? status(launch_clear_flag(clear_flag, static_cast<hipStream_t>(stream))) : MDX_OK;
  }
  int32_t flags = 0;
  if (scale != 1.0f) flags = divide ? kCopyDivide : kCopyScale;
  CopyParams p{scale, flags, nullptr, clear_flag};
  return status(launch_copy_dev(h->dtype_a, h->dtype_b, t, h->blocks, p, static_cast<hipStream_t>(stream)));
}

int mdx_unpack_planned(const void* plan, const void* d_plan, float inv_scale, int32_t* found_inf,
                       void* stream) {
  const PlanHeader* h;
  DevTable t;
  const int rc = plan_view(plan, d_plan, kPlanSpans, &h, &t);
  if (rc != MDX_OK) return rc;
  if (h->reserved) return MDX_EINVAL;  // unpack needs a source for every span
  if (h->count == 0) return MDX_OK;
  CopyParams p{inv_scale, (inv_scale != 1.0f ? kCopyScale : 0) | (found_inf ? kCopyCheck : 0), found_inf, nullptr};
  return status(launch_copy_dev(h->dtype_a, h->dtype_b, t, h->blocks, p, static_cast<hipStream_t>(stream)));
}

int mdx_allreduce_unpack_planned(const void* plan, const void* d_plan, float inv_scale, int32_t* found_inf,
                                 void* stream) {
  const PlanHeader* h;
  DevTable t;
  const int rc = plan_view(plan, d_plan, kPlanGradRuns, &h, &t);
  if (rc != MDX_OK) return rc;
  if (h->count == 0) return MDX_OK;
  ReduceParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < h->world; ++r) p.peer[r] = reinterpret_cast<const void*>(h->replicas[r]);
  p.out = reinterpret_cast<void*>(h->out);
  p.world = h->world;
  p.rank = 0;
  p.pre = h->prescale;
  p.inv_scale = inv_scale;
  p.flags = inv_scale != 1.0f ? kRedUnscale : 0;
  p.found_inf = found_inf;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (h->reduce_dtype != h->dtype_a) {
    return status(launch_allreduce_wide_dev(h->dtype_a, h->dtype_b, h->world, t, h->blocks, p, st));
  }
  return status(launch_allreduce_dev(h->dtype_a, h->dtype_b, h->world, t, h->blocks, p, st));
}

int mdx_pack_allreduce_unpack_planned_noalloc(const void* plan, float inv_scale, int32_t* found_inf,
                                              int32_t* clear_flag, void* stream) {
  if (plan == nullptr) return MDX_EINVAL;
  const PlanHeader* h = static_cast<const PlanHeader*>(plan);
  if (h->magic != kPlanMagic || h->kind != kPlanPackRuns || !plan_layout_matches(h)) return MDX_EINVAL;
  if (clear_flag != nullptr && clear_flag == found_inf) return MDX_EALIAS;
  if (h->bytes > MDX_NOALLOC_SCRATCH_BYTES) return MDX_ESCRATCH;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (h->count == 0) return clear_flag != nullptr ? status(launch_clear_flag(clear_flag, st)) : MDX_OK;
  int device = -1;
  int rc = stream_device(st, &device);
  if (rc != MDX_OK) return rc;
  unsigned char* d_plan = nullptr;
  rc = status(scratch_on(device, &d_plan));
  if (rc != MDX_OK) return rc;
  rc = upload_plan(plan, h->bytes, d_plan, st);
  if (rc != MDX_OK) return rc;
  return mdx_pack_allreduce_unpack_planned(plan, d_plan, inv_scale, found_inf, clear_flag, stream);
}

int mdx_host_device_address(void* host_ptr, void** device_ptr) {
  if (host_ptr == nullptr || device_ptr == nullptr) return MDX_EINVAL;
  return status(hipHostGetDevicePointer(device_ptr, host_ptr, 0));
}

int mdx_ipc_export(const void* ptr, mdx_ipc_handle* out) {
  if (ptr == nullptr || out == nullptr) return MDX_EINVAL;
  static_assert(sizeof(hipIpcMemHandle_t) == MDX_IPC_HANDLE_BYTES, "IPC handle size");
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  hipError_t e = hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(const_cast<void*>(ptr)));
  if (e != hipSuccess) return int(e);
  if (int64_t(size) >= MDX_IPC_MAX_ALLOC_BYTES) return MDX_ESIZE;
  hipIpcMemHandle_t h;
  e = hipIpcGetMemHandle(&h, reinterpret_cast<void*>(base));
  if (e != hipSuccess) return int(e);
  memcpy(out->bytes, &h, sizeof(h));
  out->offset = int64_t(addr(ptr) - addr(reinterpret_cast<const void*>(base)));
  out->alloc_bytes = int64_t(size);
  return MDX_OK;
}

int mdx_ipc_open(const mdx_ipc_handle* h, void** base) {
  if (h == nullptr || base == nullptr) return MDX_EINVAL;
  if (h->alloc_bytes <= 0 || h->alloc_bytes >= MDX_IPC_MAX_ALLOC_BYTES) return MDX_ESIZE;
  if (h->offset < 0 || h->offset >= h->alloc_bytes) return MDX_EINVAL;
  hipIpcMemHandle_t mh;
  memcpy(&mh, h->bytes, sizeof(mh));
  return status(hipIpcOpenMemHandle(base, mh, hipIpcMemLazyEnablePeerAccess));
}

int mdx_ipc_close(void* base) {
  if (base == nullptr) return MDX_EINVAL;
  return status(hipIpcCloseMemHandle(base));
}

}  // extern "C"
