// extern "C" entry points of libmdx.so (declared in include/mdx.h).
//
// Host-side work per call: validate every argument before anything is
// launched, cut the caller's span / piece list into dispatches of at most
// kRunsPerLaunch runs of at most kMaxRunElems elements, compute for each run
// the element offset ("head") that brings all of its pointers to 16-byte
// alignment, lay out the workgroups of each run, and launch.  Nothing here
// allocates or synchronises.
#include <string.h>

#include <algorithm>

#include "mdx_internal.h"

namespace mdx {
namespace {

inline bool valid_dtype(int d) { return d == MDX_F32 || d == MDX_BF16; }

inline int status(hipError_t e) { return e == hipSuccess ? MDX_OK : int(e); }

inline uintptr_t addr(const void* p) { return reinterpret_cast<uintptr_t>(p); }

// Smallest h in [0, E) such that every (pointer, element size) advanced by h
// elements is 16-byte aligned; -1 if none exists or the run has no full
// fragment after it.
int aligned_head(const uintptr_t* ptrs, const int* sizes, int count, int E, int64_t n) {
  for (int h = 0; h < E; ++h) {
    bool ok = true;
    for (int k = 0; k < count && ok; ++k) {
      ok = ((ptrs[k] + uintptr_t(h) * uintptr_t(sizes[k])) & 15u) == 0;
    }
    if (ok) return (n >= int64_t(h) + E) ? h : -1;
  }
  return -1;
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

// ---------------------------------------------------------------------------
// copy family
// ---------------------------------------------------------------------------

int run_copy(const mdx_span* spans, int n_spans, int sdt, int ddt, const CopyParams& params,
             bool in_place, hipStream_t stream) {
  const int E = copy_frag_elems(sdt, ddt);
  const int64_t VPB = int64_t(kBlock) * (kCopyElemsPerThread / E);
  const int64_t EPB = int64_t(kBlock) * kCopyElemsPerThread;
  const int ss = dtype_size(sdt), ds = dtype_size(ddt);

  SpanBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int rc = status(launch_copy(sdt, ddt, b, params, stream));
    memset(&b, 0, sizeof(b));
    return rc;
  };

  for (int i = 0; i < n_spans; ++i) {
    const mdx_span& sp = spans[i];
    const char* src = static_cast<const char*>(in_place ? sp.dst : sp.src);
    char* dst = static_cast<char*>(sp.dst);
    for (int64_t done = 0; done < sp.numel; done += kMaxRunElems) {
      const int64_t n = std::min<int64_t>(kMaxRunElems, sp.numel - done);
      const void* rs = src ? src + done * ss : nullptr;
      void* rd = dst + done * ds;
      uintptr_t ptrs[2];
      int sizes[2];
      int np = 0;
      ptrs[np] = addr(rd);
      sizes[np++] = ds;
      if (rs) {
        ptrs[np] = addr(rs);
        sizes[np++] = ss;
      }
      const int head = aligned_head(ptrs, sizes, np, E, n);
      const int k = b.count;
      b.src[k] = rs;
      b.dst[k] = rd;
      b.numel[k] = n;
      b.head[k] = head;
      b.first_block[k + 1] = b.first_block[k] + run_blocks(n, head, E, VPB, EPB);
      b.count = k + 1;
      if (b.count == kRunsPerLaunch) {
        const int rc = flush();
        if (rc != MDX_OK) return rc;
      }
    }
  }
  return flush();
}

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

// ---------------------------------------------------------------------------
// reduce family
// ---------------------------------------------------------------------------

// Lays out pieces into dispatches.  `grad_size` > 0 adds each piece's grad
// pointer to the alignment requirement (fused unpack).
template <typename Launch>
int run_pieces(const mdx_piece* pieces, void* const* grads, int n_pieces, const ReduceParams& params,
               int in_size, int out_size, int grad_size, int E, int U, Launch&& launch) {
  const int64_t VPB = int64_t(kBlock) * U;
  const int64_t EPB = VPB * E;
  PieceBatch b;
  memset(&b, 0, sizeof(b));
  auto flush = [&]() -> int {
    if (b.count == 0) return MDX_OK;
    const int rc = status(launch(b));
    memset(&b, 0, sizeof(b));
    return rc;
  };
  for (int i = 0; i < n_pieces; ++i) {
    const mdx_piece& pc = pieces[i];
    const char* own = static_cast<const char*>(pc.own);
    char* grad = grads ? static_cast<char*>(grads[i]) : nullptr;
    for (int64_t done = 0; done < pc.numel; done += kMaxRunElems) {
      const int64_t n = std::min<int64_t>(kMaxRunElems, pc.numel - done);
      const int64_t pos = pc.pos + done;
      uintptr_t ptrs[MDX_MAX_WORLD + 3];
      int sizes[MDX_MAX_WORLD + 3];
      int np = 0;
      const void* ro = own ? own + done * in_size : nullptr;
      void* rg = grad ? grad + done * grad_size : nullptr;
      if (ro) {
        ptrs[np] = addr(ro);
        sizes[np++] = in_size;
      }
      for (int r = 0; r < params.world; ++r) {
        if (r == params.rank) continue;
        ptrs[np] = addr(params.peer[r]) + uintptr_t(pos) * uintptr_t(in_size);
        sizes[np++] = in_size;
      }
      if (params.out) {
        ptrs[np] = addr(params.out) + uintptr_t(pos) * uintptr_t(out_size);
        sizes[np++] = out_size;
      }
      if (rg) {
        ptrs[np] = addr(rg);
        sizes[np++] = grad_size;
      }
      const int head = aligned_head(ptrs, sizes, np, E, n);
      const int k = b.count;
      b.own[k] = ro;
      b.pos[k] = pos;
      b.numel[k] = n;
      b.grad[k] = rg;
      b.head[k] = head;
      b.first_block[k + 1] = b.first_block[k] + run_blocks(n, head, E, VPB, EPB);
      b.count = k + 1;
      if (b.count == kRunsPerLaunch) {
        const int rc = flush();
        if (rc != MDX_OK) return rc;
      }
    }
  }
  return flush();
}

// Validates W replica bases and increasing, non-overlapping runs; returns the
// extent (one past the last element) through `end`.
int check_runs(const void* const* replicas, int world, const int64_t* offs, const int64_t* nums,
               int n_runs, int64_t* end, bool* any) {
  if (world < 1 || world > MDX_MAX_WORLD) return MDX_EWORLD;
  if (n_runs < 0 || replicas == nullptr) return MDX_EINVAL;
  *end = 0;
  *any = false;
  for (int k = 0; k < n_runs; ++k) {
    if (offs[k] < 0 || nums[k] < 0 || offs[k] < *end) return MDX_EINVAL;
    *end = offs[k] + nums[k];
    *any = *any || nums[k] > 0;
  }
  if (!*any) return MDX_OK;
  for (int r = 0; r < world; ++r) {
    if (replicas[r] == nullptr) return MDX_EINVAL;
  }
  return MDX_OK;
}

bool is_pow2(int w) { return w > 0 && (w & (w - 1)) == 0; }

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" {

int mdx_abi_version(void) { return MDX_ABI_VERSION; }

const char* mdx_strerror(int code) {
  switch (code) {
    case MDX_OK: return "success";
    case MDX_EINVAL: return "mdx: invalid argument (NULL pointer, negative count or size)";
    case MDX_EDTYPE: return "mdx: unsupported dtype code (expected MDX_F32 or MDX_BF16)";
    case MDX_EWORLD: return "mdx: world size outside [1, MDX_MAX_WORLD] or rank outside [0, world)";
    case MDX_EALIAS: return "mdx: output overlaps an input it must not overlap";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "mdx: unknown status code";
}

int mdx_pack(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, float scale,
             int divide, void* stream) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return MDX_EDTYPE;
  int rc = check_spans(spans, n_spans, false);
  if (rc != MDX_OK) return rc;
  int32_t flags = 0;
  if (scale != 1.0f) flags = divide ? kCopyDivide : kCopyScale;
  CopyParams p{scale, flags, nullptr};
  return run_copy(spans, n_spans, src_dtype, dst_dtype, p, false, static_cast<hipStream_t>(stream));
}

int mdx_unpack(const mdx_span* spans, int n_spans, int src_dtype, int dst_dtype, float inv_scale,
               int32_t* found_inf, void* stream) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return MDX_EDTYPE;
  int rc = check_spans(spans, n_spans, true);
  if (rc != MDX_OK) return rc;
  CopyParams p{inv_scale, (inv_scale != 1.0f ? kCopyScale : 0) | (found_inf ? kCopyCheck : 0),
               found_inf};
  return run_copy(spans, n_spans, src_dtype, dst_dtype, p, false, static_cast<hipStream_t>(stream));
}

int mdx_unscale_found_inf(const mdx_span* spans, int n_spans, int dtype, float inv_scale,
                          int32_t* found_inf, void* stream) {
  if (!valid_dtype(dtype)) return MDX_EDTYPE;
  int rc = check_spans(spans, n_spans, false);
  if (rc != MDX_OK) return rc;
  CopyParams p{inv_scale, (inv_scale != 1.0f ? kCopyScale : 0) | (found_inf ? kCopyCheck : 0),
               found_inf};
  return run_copy(spans, n_spans, dtype, dtype, p, true, static_cast<hipStream_t>(stream));
}

int mdx_cast_f32_bf16(const float* src, uint16_t* dst, int64_t numel, void* stream) {
  if (numel < 0 || (numel > 0 && (src == nullptr || dst == nullptr))) return MDX_EINVAL;
  if (any_overlap(src, numel * 4, dst, numel * 2)) return MDX_EALIAS;
  mdx_span sp{src, dst, numel};
  CopyParams p{1.0f, 0, nullptr};
  return run_copy(&sp, 1, MDX_F32, MDX_BF16, p, false, static_cast<hipStream_t>(stream));
}

int mdx_allreduce_sum(const void* const* replicas, int world, int dtype, const int64_t* offsets,
                      const int64_t* numels, int n_runs, void* out, void* stream) {
  if (!valid_dtype(dtype)) return MDX_EDTYPE;
  if (n_runs > 0 && (offsets == nullptr || numels == nullptr)) return MDX_EINVAL;
  int64_t end = 0;
  bool any = false;
  int rc = check_runs(replicas, world, offsets, numels, n_runs, &end, &any);
  if (rc != MDX_OK || !any) return rc;
  if (out == nullptr) return MDX_EINVAL;
  const int es = dtype_size(dtype);
  for (int r = 0; r < world; ++r) {
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
  const int E = frag_elems(es, es);
  const int U = allreduce_unroll(world, E * es);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  mdx_piece pieces[kRunsPerLaunch];
  int np = 0;
  auto launch = [&](const PieceBatch& b) { return launch_allreduce(dtype, dtype, false, world, b, p, st); };
  for (int k = 0; k < n_runs; ++k) {
    if (numels[k] == 0) continue;
    pieces[np++] = mdx_piece{base0 + offsets[k] * es, offsets[k], numels[k]};
    if (np == kRunsPerLaunch) {
      rc = run_pieces(pieces, nullptr, np, p, es, es, 0, E, U, launch);
      if (rc != MDX_OK) return rc;
      np = 0;
    }
  }
  return run_pieces(pieces, nullptr, np, p, es, es, 0, E, U, launch);
}

int mdx_allreduce_unpack(const void* const* replicas, int world, int dtype, const mdx_grad_run* runs,
                         int n_runs, void* out, int grad_dtype, float inv_scale, int32_t* found_inf,
                         void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(grad_dtype)) return MDX_EDTYPE;
  if (world < 1 || world > MDX_MAX_WORLD) return MDX_EWORLD;
  if (n_runs < 0 || (n_runs > 0 && runs == nullptr) || replicas == nullptr) return MDX_EINVAL;
  const int es = dtype_size(dtype), gs = dtype_size(grad_dtype);
  int64_t end = 0;
  bool any = false;
  for (int k = 0; k < n_runs; ++k) {
    if (runs[k].offset < 0 || runs[k].numel < 0 || runs[k].offset < end) return MDX_EINVAL;
    if (runs[k].numel > 0 && runs[k].grad == nullptr) return MDX_EINVAL;
    end = runs[k].offset + runs[k].numel;
    any = any || runs[k].numel > 0;
  }
  if (!any) return MDX_OK;
  for (int r = 0; r < world; ++r) {
    if (replicas[r] == nullptr) return MDX_EINVAL;
    if (out && replicas[r] != out && any_overlap(replicas[r], end * es, out, end * es)) return MDX_EALIAS;
  }
  for (int k = 0; k < n_runs; ++k) {
    const int64_t gb = runs[k].numel * gs;
    for (int r = 0; r < world; ++r) {
      if (any_overlap(runs[k].grad, gb, replicas[r], end * es)) return MDX_EALIAS;
    }
    if (out && any_overlap(runs[k].grad, gb, out, end * es)) return MDX_EALIAS;
  }
  ReduceParams p;
  memset(&p, 0, sizeof(p));
  for (int r = 0; r < world; ++r) p.peer[r] = replicas[r];
  p.out = out;
  p.world = world;
  p.rank = 0;
  p.pre = 1.0f;
  p.inv_scale = inv_scale;
  p.flags = inv_scale != 1.0f ? kRedUnscale : 0;
  p.found_inf = found_inf;
  const char* base0 = static_cast<const char*>(replicas[0]);
  const int E = frag_elems(es, gs);
  const int U = allreduce_unroll(world, E * es);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](const PieceBatch& b) { return launch_allreduce(dtype, grad_dtype, true, world, b, p, st); };
  mdx_piece pieces[kRunsPerLaunch];
  void* grads[kRunsPerLaunch];
  int np = 0;
  for (int k = 0; k < n_runs; ++k) {
    if (runs[k].numel == 0) continue;
    pieces[np] = mdx_piece{base0 + runs[k].offset * es, runs[k].offset, runs[k].numel};
    grads[np++] = runs[k].grad;
    if (np == kRunsPerLaunch) {
      const int rc = run_pieces(pieces, grads, np, p, es, es, gs, E, U, launch);
      if (rc != MDX_OK) return rc;
      np = 0;
    }
  }
  return run_pieces(pieces, grads, np, p, es, es, gs, E, U, launch);
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
  p.inv_scale = inv_scale;
  p.found_inf = found_inf;
  p.pre = 1.0f;
  int32_t flags = 0;
  if (divide && world > 1) {
    // x / W and x * (1/W) are the same correctly rounded value when 1/W is
    // exact, i.e. for power-of-two W; the multiply is the cheaper instruction.
    if (is_pow2(world)) {
      flags |= kRedPreMul;
      p.pre = 1.0f / float(world);
    } else {
      flags |= kRedPreDiv;
      p.pre = float(world);
    }
  }
  if (accumulate) flags |= kRedAccumulate;
  if (inv_scale != 1.0f) flags |= kRedUnscale;
  p.flags = flags;
  p.world = world;
  const int is = dtype_size(in_dtype), os = dtype_size(shard_dtype);
  const int wmax = share_wmax(in_dtype, reduce_dtype, shard_dtype, world);
  const int E = frag_elems(is, os);
  const int U = share_unroll(wmax, E * is);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](const PieceBatch& b) {
    return launch_share(in_dtype, reduce_dtype, shard_dtype, wmax, b, p, st);
  };
  return run_pieces(own, nullptr, n_own, p, is, os, 0, E, U, launch);
}

}  // extern "C"
