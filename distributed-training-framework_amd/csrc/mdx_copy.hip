// Multi-tensor copy / convert / scale kernel: the pack, unpack (+ fused
// unscale and found-inf), in-place unscale and fp32->bf16 cast entry points
// all run this one kernel with different dtype pairs and modes.
//
// Per element:  v = cvt_dst(src);  SCALE: v = rnd_dst(f32(v) * s)  or  rnd_dst(f32(v) / s)
//               dst = v;           CHECK: bad |= !isfinite(v)
// which is `dst.copy_(src)` followed by `dst.mul_(s)` / `dst.div_(s)` in
// ATen's op order.  The scaling and the check are compile-time modes, so a
// plain pack or unpack carries no dead arithmetic.
//
// Layout of the work: each span is cut into chunks of kBlock * U fragments
// (a fragment = E elements = one 16-byte vector of the wider of the two
// types, so 8 or 16 bytes of the other).  Lane t of chunk c handles
// fragments c*VPB + u*kBlock + t, so every vector instruction of a wave
// touches 64 consecutive fragments; all U fragments are loaded (non-temporal:
// each byte is read once per step) before the first store, and stored
// non-temporally (the next reader is a later pipeline stage).  The body
// starts at the run's head, the element offset that 16-byte aligns the most
// streams (the destination first); a stream it leaves unaligned still moves
// in vectors.  The head before the body and the tail after it go one element
// per lane, and a run shorter than its head plus one fragment goes entirely
// that way.
#include <type_traits>

#include "mdx_internal.h"

namespace mdx {
namespace {

enum : int { kScaleNone = 0, kScaleMul = 1, kScaleDiv = 2 };

template <typename S, typename D, int SCALE, bool CHECK>
struct CopyOp {
  float scale;
  __device__ __forceinline__ D operator()(S x, bool& bad) const {
    D v = Cvt<S, D>::run(x);
    if constexpr (SCALE == kScaleMul) v = from_f32<D>(to_f32(v) * scale);
    if constexpr (SCALE == kScaleDiv) v = from_f32<D>(to_f32(v) / scale);
    if constexpr (CHECK) bad |= !is_finite(v);
    return v;
  }
};

template <typename S, typename D, int SCALE, bool CHECK, typename View>
__device__ __forceinline__ void copy_body(const View& tab, const CopyParams& p) {
  constexpr int E = copy_frag_elems_of(int(sizeof(S)), int(sizeof(D)));
  constexpr int U = copy_unroll_of(int(sizeof(S)), int(sizeof(D)));
  constexpr int VPB = kBlock * U;
  constexpr int EPT = U * E;
  constexpr int EPB = kBlock * EPT;

  const int blk = tab.block();
  SpanRun run;
  if constexpr (sizeof(S) > sizeof(D) && std::is_same_v<View, SpanArgView>) {
    run = tab.span_run_wave(blk);
  } else {
    run = tab.span_run(blk);
  }
  const int c = run.c;
  const int nblk = run.nblk;
  const S* src = static_cast<const S*>(run.src);
  D* dst = static_cast<D*>(run.dst);
  const int64_t n = run.numel;
  const int32_t h = run.head;
  const int t = int(threadIdx.x);
  const bool zero_src = (src == nullptr);
  const CopyOp<S, D, SCALE, CHECK> op{p.scale};
  bool bad = false;
  // The scaler's per-step flag clear rides on the pack: one lane of the first
  // workgroup (a per-lane store under the lane predicate).
  if (p.clear != nullptr && blk == 0 && t == 0) *p.clear = 0;

  if (h >= 0) {
    const int64_t nvec = (n - h) / E;
    const S* vs = src + h;
    D* vd = dst + h;
    S in[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = int64_t(c) * VPB + int64_t(u) * kBlock + t;
      if (v < nvec) {
        if (zero_src) {
#pragma unroll
          for (int k = 0; k < E; ++k) in[u][k] = zero_of<S>();
        } else {
          vload<S, E, true>(in[u], vs + v * E);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = int64_t(c) * VPB + int64_t(u) * kBlock + t;
      if (v < nvec) {
        D out[E];
#pragma unroll
        for (int k = 0; k < E; ++k) out[k] = op(in[u][k], bad);
        vstore<D, E, true>(vd + v * E, out);
      }
    }
    // Ragged edges: the head before the aligned body (first chunk) and the
    // tail after it (last chunk), one element per lane.
    if (c == 0 && t < h && t < n) {
      const S x = zero_src ? zero_of<S>() : src[t];
      dst[t] = op(x, bad);
    }
    const int64_t tail0 = h + nvec * E;
    if (c == nblk - 1 && tail0 + t < n) {
      const int64_t i = tail0 + t;
      const S x = zero_src ? zero_of<S>() : src[i];
      dst[i] = op(x, bad);
    }
  } else {
    S in[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int64_t i = int64_t(c) * EPB + int64_t(k) * kBlock + t;
      in[k] = (i < n && !zero_src) ? src[i] : zero_of<S>();
    }
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int64_t i = int64_t(c) * EPB + int64_t(k) * kBlock + t;
      if (i < n) dst[i] = op(in[k], bad);
    }
  }
  if constexpr (CHECK) flag_nonfinite(bad, p.found_inf);
}

// Table in the kernel-argument segment.
template <typename S, typename D, int SCALE, bool CHECK>
__global__ void __launch_bounds__(kBlock) copy_kernel(SpanBatch b, CopyParams p) {
  copy_body<S, D, SCALE, CHECK>(SpanArgView{b}, p);
}

// One run in the kernel-argument segment.
template <typename S, typename D, int SCALE, bool CHECK>
__global__ void __launch_bounds__(kBlock) copy_kernel_one(SpanOne b, CopyParams p) {
  copy_body<S, D, SCALE, CHECK>(SpanOneView{b}, p);
}

// Table (plan) in device memory.
template <typename S, typename D, int SCALE, bool CHECK>
__global__ void __launch_bounds__(kBlock) copy_kernel_dev(DevTable t, CopyParams p) {
  copy_body<S, D, SCALE, CHECK>(DevView{t}, p);
}

// Either table kind: a kernel-argument SpanBatch (grid from its prefix; one run goes
// out as a SpanOne) or a DevTable.
struct ArgLaunch {
  const SpanBatch& b;
  template <typename S, typename D, int SCALE, bool CHECK>
  hipError_t go(const CopyParams& p, hipStream_t stream) const {
    if (b.count == 1) {
      hipLaunchKernelGGL((copy_kernel_one<S, D, SCALE, CHECK>), dim3(b.first_block[1]), dim3(kBlock), 0, stream,
                         one_run_of(b), p);
    } else {
      hipLaunchKernelGGL((copy_kernel<S, D, SCALE, CHECK>), dim3(b.first_block[b.count]), dim3(kBlock), 0,
                         stream, b, p);
    }
    return hipGetLastError();
  }
};
struct DevLaunch {
  const DevTable& t;
  int blocks;
  template <typename S, typename D, int SCALE, bool CHECK>
  hipError_t go(const CopyParams& p, hipStream_t stream) const {
    return launch_plan_slices(t, blocks, [&](const DevTable& slice, int grid) {
      hipLaunchKernelGGL((copy_kernel_dev<S, D, SCALE, CHECK>), dim3(grid), dim3(kBlock), 0, stream, slice, p);
    });
  }
};

template <typename S, typename D, typename L>
hipError_t launch_typed(const L& l, const CopyParams& p, hipStream_t stream) {
  const bool check = (p.flags & kCopyCheck) != 0;
  if (p.flags & kCopyScale) {
    return check ? l.template go<S, D, kScaleMul, true>(p, stream) : l.template go<S, D, kScaleMul, false>(p, stream);
  }
  if (p.flags & kCopyDivide) {
    return check ? l.template go<S, D, kScaleDiv, true>(p, stream) : l.template go<S, D, kScaleDiv, false>(p, stream);
  }
  return check ? l.template go<S, D, kScaleNone, true>(p, stream) : l.template go<S, D, kScaleNone, false>(p, stream);
}

template <typename S, typename L>
hipError_t launch_to(int dst_dtype, const L& l, const CopyParams& p, hipStream_t stream) {
  if (dst_dtype == MDX_F32) return launch_typed<S, float>(l, p, stream);
  if (dst_dtype == MDX_BF16) return launch_typed<S, bf16>(l, p, stream);
  return launch_typed<S, f16>(l, p, stream);
}

template <typename L>
hipError_t launch_any(int src_dtype, int dst_dtype, const L& l, const CopyParams& p, hipStream_t stream) {
  if (src_dtype == MDX_F32) return launch_to<float>(dst_dtype, l, p, stream);
  if (src_dtype == MDX_BF16) return launch_to<bf16>(dst_dtype, l, p, stream);
  return launch_to<f16>(dst_dtype, l, p, stream);
}

__global__ void __launch_bounds__(kBlock) clear_flag_kernel(int32_t* flag) {
  if (threadIdx.x == 0) *flag = 0;
}

}  // namespace

hipError_t launch_clear_flag(int32_t* flag, hipStream_t stream) {
  hipLaunchKernelGGL(clear_flag_kernel, dim3(1), dim3(kBlock), 0, stream, flag);
  return hipGetLastError();
}

int copy_frag_elems(int src_dtype, int dst_dtype) {
  return copy_frag_elems_of(dtype_size(src_dtype), dtype_size(dst_dtype));
}

hipError_t launch_copy(int src_dtype, int dst_dtype, const SpanBatch& b, const CopyParams& p,
                       hipStream_t stream) {
  return launch_any(src_dtype, dst_dtype, ArgLaunch{b}, p, stream);
}

hipError_t launch_copy_dev(int src_dtype, int dst_dtype, const DevTable& t, int blocks, const CopyParams& p,
                           hipStream_t stream) {
  return launch_any(src_dtype, dst_dtype, DevLaunch{t, blocks}, p, stream);
}

}  // namespace mdx
