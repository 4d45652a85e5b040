#pragma once
// W-way streaming reduction over contributions resident in HBM (kernel template;
// instantiated per dtype triple by the mdx_reduce_*.hip translation units).
//
// For element j of a piece (reduced-vector position p = pos + j):
//   x_r  = cvt_acc(contribution_r[p])          r = 0..W-1, own data for r == rank
//   x_r  = rnd_acc(x_r * pre) | rnd_acc(x_r / pre)   (optional pre-scale)
//   acc  = x_0; acc = rnd_acc(acc + x_r) for r = 1..W-1   (fixed rank order)
//   y    = cvt_out(acc); y = rnd_out(out[p] + y) (accumulate); y = rnd_out(y * inv)
//   out[p] = y; bad |= !isfinite(y)
// which reproduces, op for op, the ATen chains of DDP's all-reduce and of
// FSDP's reduce_scatter_grads for a rank-ordered sum.
//
// Each lane keeps U fragments of every contribution in flight (W*U 16-byte
// loads issued before the first add), which is what feeds HBM: for W = 8 and
// fp32 that is 16 outstanding 16-byte loads per lane.  Peer contributions are
// read once per step and use non-temporal loads; the rank's own data and the
// output use normal accesses because the neighbouring pipeline stages touch
// the same bytes just before and after.
#include "mdx_internal.h"

namespace mdx {
namespace reduce_impl {

template <typename In, typename Acc, typename Out>
struct ReduceOp {
  int32_t flags;
  float pre;
  float inv_scale;
  __device__ __forceinline__ Acc widen(In x) const {
    Acc a = Cvt<In, Acc>::run(x);
    if (flags & kRedPreMul) a = from_f32<Acc>(to_f32(a) * pre);
    if (flags & kRedPreDiv) a = from_f32<Acc>(to_f32(a) / pre);
    return a;
  }
  __device__ __forceinline__ Acc add(Acc a, Acc b) const {
    return from_f32<Acc>(to_f32(a) + to_f32(b));
  }
  __device__ __forceinline__ Out finish(Acc a, Out prev, bool& bad) const {
    Out y = Cvt<Acc, Out>::run(a);
    if (flags & kRedAccumulate) y = from_f32<Out>(to_f32(prev) + to_f32(y));
    if (flags & kRedUnscale) y = from_f32<Out>(to_f32(y) * inv_scale);
    if (flags & kRedCheck) bad |= !is_finite(y);
    return y;
  }
};

template <typename In, typename Acc, typename Out, int W>
__global__ void __launch_bounds__(kBlock) reduce_kernel(PieceBatch b, ReduceParams p) {
  constexpr int E = frag_elems(int(sizeof(In)), int(sizeof(Out)));
  constexpr int U = reduce_unroll(W);
  constexpr int VPB = kBlock * U;
  constexpr int EPB = VPB * E;

  const int blk = int(blockIdx.x);
  const int s = find_run(b.first_block, b.count, blk);
  const int c = blk - b.first_block[s];
  const int nblk = b.first_block[s + 1] - b.first_block[s];
  const int64_t pos = b.pos[s];
  const int64_t n = b.numel[s];
  const int32_t h = b.head[s];
  const int rank = p.rank;
  const bool own_zero = (b.own[s] == nullptr);
  const bool accumulate = (p.flags & kRedAccumulate) != 0;
  const ReduceOp<In, Acc, Out> op{p.flags, p.pre, p.inv_scale};
  const int t = int(threadIdx.x);

  const In* src[W];
#pragma unroll
  for (int r = 0; r < W; ++r) {
    src[r] = (r == rank) ? static_cast<const In*>(b.own[s])
                         : static_cast<const In*>(p.peer[r]) + pos;
  }
  Out* out = static_cast<Out*>(p.out) + pos;
  bool bad = false;

  // One element, used for ragged edges and the unaligned path.
  auto element = [&](int64_t i) {
    Acc acc = zero_of<Acc>();
#pragma unroll
    for (int r = 0; r < W; ++r) {
      const In x = (r == rank && own_zero) ? zero_of<In>() : src[r][i];
      const Acc a = op.widen(x);
      acc = (r == 0) ? a : op.add(acc, a);
    }
    const Out prev = accumulate ? out[i] : zero_of<Out>();
    out[i] = op.finish(acc, prev, bad);
  };

  if (h >= 0) {
    const int64_t nvec = (n - h) / E;
    In x[U][W][E];
    Out prev[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = int64_t(c) * VPB + int64_t(u) * kBlock + t;
      if (v < nvec) {
        const int64_t i = h + v * E;
#pragma unroll
        for (int r = 0; r < W; ++r) {
          if (r == rank) {
            if (own_zero) {
#pragma unroll
              for (int k = 0; k < E; ++k) x[u][r][k] = zero_of<In>();
            } else {
              vload<In, E, false>(x[u][r], src[r] + i);
            }
          } else {
            vload<In, E, true>(x[u][r], src[r] + i);
          }
        }
        if (accumulate) vload<Out, E, false>(prev[u], out + i);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = int64_t(c) * VPB + int64_t(u) * kBlock + t;
      if (v < nvec) {
        const int64_t i = h + v * E;
        Out y[E];
#pragma unroll
        for (int k = 0; k < E; ++k) {
          Acc acc = op.widen(x[u][0][k]);
#pragma unroll
          for (int r = 1; r < W; ++r) acc = op.add(acc, op.widen(x[u][r][k]));
          y[k] = op.finish(acc, accumulate ? prev[u][k] : zero_of<Out>(), bad);
        }
        vstore<Out, E, false>(out + i, y);
      }
    }
    if (c == 0 && t < h && t < n) element(t);
    const int64_t tail0 = h + nvec * E;
    if (c == nblk - 1 && tail0 + t < n) element(tail0 + t);
  } else {
#pragma unroll 4
    for (int k = 0; k < U * E; ++k) {
      const int64_t i = int64_t(c) * EPB + int64_t(k) * kBlock + t;
      if (i < n) element(i);
    }
  }
  if (p.flags & kRedCheck) flag_nonfinite(bad, p.found_inf);
}

template <typename In, typename Acc, typename Out, int W>
hipError_t launch_w(const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  const int blocks = b.first_block[b.count];
  hipLaunchKernelGGL((reduce_kernel<In, Acc, Out, W>), dim3(blocks), dim3(kBlock), 0, stream, b, p);
  return hipGetLastError();
}

template <typename In, typename Acc, typename Out>
hipError_t launch_types(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  switch (world) {
    case 1: return launch_w<In, Acc, Out, 1>(b, p, stream);
    case 2: return launch_w<In, Acc, Out, 2>(b, p, stream);
    case 3: return launch_w<In, Acc, Out, 3>(b, p, stream);
    case 4: return launch_w<In, Acc, Out, 4>(b, p, stream);
    case 5: return launch_w<In, Acc, Out, 5>(b, p, stream);
    case 6: return launch_w<In, Acc, Out, 6>(b, p, stream);
    case 7: return launch_w<In, Acc, Out, 7>(b, p, stream);
    case 8: return launch_w<In, Acc, Out, 8>(b, p, stream);
    case 9: return launch_w<In, Acc, Out, 9>(b, p, stream);
    case 10: return launch_w<In, Acc, Out, 10>(b, p, stream);
    case 11: return launch_w<In, Acc, Out, 11>(b, p, stream);
    case 12: return launch_w<In, Acc, Out, 12>(b, p, stream);
    case 13: return launch_w<In, Acc, Out, 13>(b, p, stream);
    case 14: return launch_w<In, Acc, Out, 14>(b, p, stream);
    case 15: return launch_w<In, Acc, Out, 15>(b, p, stream);
    default: return launch_w<In, Acc, Out, 16>(b, p, stream);
  }
}

}  // namespace reduce_impl
}  // namespace mdx
