// W-way streaming reductions over contributions resident in HBM (kernel
// templates; instantiated per dtype by the mdx_reduce_*.hip translation units).
//
// allreduce_kernel<T, G, W, UNPACK>: DDP's bucket all-reduce.  For element j
// of a piece (replica position p = pos + j):
//     acc = x_0[p]; acc = rnd_T(acc + x_r[p]) for r = 1..W-1      (rank order)
//     out[p] = acc                                  (the in-place all-reduce)
//   UNPACK additionally writes the bucket slice straight into the gradient,
//   with the loss scaler's epilogue:
//     g = cvt_G(acc); g = rnd_G(g * inv_scale); grad[j] = g; bad |= !isfinite(g)
//   which is scatter_from_buffer's copy_ followed by unscale_'s mul_ and
//   isfinite, fused so the bucket is not read back.
//
// allreduce_wide_kernel<In, T, G, W> (+ _dev): the same fused all-reduce +
// unpack for contributions that travel in a narrower dtype In than the bucket
// dtype T (bf16 or fp16 gradients summed into fp32 buckets).  Each contribution is
// widened and pre-scaled at the receiver, x_r = rnd_T(cvt_T(c_r[p]) * pre),
// which is exactly the value the sender's pack (`copy_` into a T bucket, then
// `mul_(1/W)`) would have put on the wire; the rank-ordered sum, the write of
// the T bucket and the unpack epilogue are as above.
//
// allreduce_pack_kernel<In, T, W> (+ _dev): the pack fused in front of the
// fused all-reduce + unpack, for gradients of the wire dtype In.  Replica
// `rank` is read from the run's gradient (NULL = zeros) and packed in
// registers, c = rnd_T(g * pre) for a bucket of the same dtype (the pack's
// `copy_` + `mul_(1/W)`) or the raw gradient for a widening bucket (which
// pre-scales every contribution where it is widened, as above); c is stored
// to replica `rank`'s row -- what the peers read -- and enters the rank-ordered
// sum without being read back, and the bucket is a separate output.  Per
// element: the gradient and W-1 peer rows read; the packed row, the bucket
// and the gradient written.  The dispatch also clears the loss scaler's flag
// for the next step (ReduceParams::clear).
//
// share_kernel<In, Acc, Out, WMAX>: FSDP's reduce-scatter share, runtime
// W <= WMAX.  x_r = cvt_Acc(contribution_r[p]); x_r = rnd_Acc(x_r * pre | x_r / pre);
// acc = rank-ordered sum in Acc; y = cvt_Out(acc); y = rnd_Out(out + y) when
// accumulating; optional unscale + found-inf epilogue.  The pre-scale and the
// accumulate are compile-time variants selected once per workgroup.  A piece
// may carry its own destination (PieceRun::grad), so that one dispatch writes
// the shard gradients of several FSDP units (the multi-unit share); otherwise
// it writes out + its position.
//
// Every contribution is read once per step, so every load is non-temporal;
// each lane keeps U fragments of all W contributions in flight before the
// first add (about 128 bytes per lane: U * W = 8 16-byte loads for the fp32
// all-reduce at W = 8).
#pragma once

#include "mdx_internal.h"

namespace mdx {
namespace reduce_impl {

// ---------------------------------------------------------------------------
// all-reduce (+ fused unpack)
// ---------------------------------------------------------------------------

template <typename In, typename T, typename G, int W, bool UNPACK, bool PRE, bool PACK, typename View>
__device__ __forceinline__ void allreduce_body(const View& tab, const ReduceParams& p) {
  static_assert(!PACK || (UNPACK && sizeof(G) == sizeof(In)), "the fused pack reads gradients of the wire dtype");
  constexpr int E = UNPACK ? reduce_frag_elems(int(sizeof(In)), int(sizeof(T)), int(sizeof(G)))
                            : store_frag_elems(int(sizeof(T)));
  constexpr int U = PACK ? pack_allreduce_unroll() : allreduce_unroll(W, E * int(sizeof(In)));
  constexpr int VPB = kBlock * U;
  constexpr int EPB = VPB * E;
  // 32-byte fragments of a stored type go out through vstore_wave8, which
  // every lane of the wave takes part in: lanes past the end then compute on
  // zeros (finite: they never raise the flag) and store nothing.
  constexpr bool kWaveT = E * int(sizeof(T)) == 32;
  constexpr bool kWaveG = UNPACK && E * int(sizeof(G)) == 32;
  constexpr bool kWave = kWaveT || kWaveG;
  static_assert(!kWave || E == 8, "wave-permuted stores take 8 four-byte elements per lane");

  const int blk = tab.block();
  const PieceRun run = tab.piece_run(blk);
  const int c = run.c;
  const int nblk = run.nblk;
  const int64_t pos = run.pos;
  const int64_t n = run.numel;
  const int32_t h = run.head;
  const int rank = p.rank;
  const int t = int(threadIdx.x);
  const bool unscale = (p.flags & kRedUnscale) != 0;
  const float inv = p.inv_scale;
  const float pre = p.pre;

  // Replica `rank` is read through the run's own pointer: the rank's packed
  // row, or with PACK its gradient (NULL = zeros), packed here.
  const In* src[W];
#pragma unroll
  for (int r = 0; r < W; ++r) {
    src[r] = (r == rank) ? static_cast<const In*>(run.own) : static_cast<const In*>(p.peer[r]) + pos;
  }
  const bool own_zero = PACK && run.own == nullptr;
  In* own_row = PACK ? static_cast<In*>(const_cast<void*>(p.peer[rank])) + pos : nullptr;
  const bool pack_scale = PACK && !PRE && (p.flags & kRedPackScale) != 0;
  T* out = p.out ? static_cast<T*>(p.out) + pos : nullptr;
  G* grad = static_cast<G*>(run.grad);
  bool bad = false;
  // The next step's found-inf flag rides on the fused pack (nothing reads or
  // sets it during this step): one lane of the first workgroup.
  if (PACK && p.clear != nullptr && blk == 0 && t == 0) *p.clear = 0;

  // The pack's `copy_` + `mul_(1/W)` of this rank's gradient (same-dtype
  // buckets; a widening bucket carries the raw gradient and pre-scales where
  // every contribution is widened).
  auto pack_op = [&](In x) -> In {
    if constexpr (PACK && !PRE) {
      const In xs = from_f32<In>(to_f32(x) * pre);
      return pack_scale ? xs : x;
    }
    return x;
  };
  auto widen = [&](In x) -> T {
    T a = Cvt<In, T>::run(x);
    if constexpr (PRE) a = from_f32<T>(to_f32(a) * pre);
    return a;
  };

  auto finish = [&](T acc) -> G {
    G g = Cvt<T, G>::run(acc);
    const G gs = from_f32<G>(to_f32(g) * inv);
    g = unscale ? gs : g;
    bad |= !is_finite(g);
    return g;
  };
  auto element = [&](int64_t i) {
    T acc = zero_of<T>();
    In packed = zero_of<In>();
#pragma unroll
    for (int r = 0; r < W; ++r) {
      In xr;
      if (PACK && r == rank) {
        xr = pack_op(own_zero ? zero_of<In>() : src[r][i]);
        packed = xr;
      } else {
        xr = src[r][i];
      }
      const T a = widen(xr);
      acc = (r == 0) ? a : from_f32<T>(to_f32(acc) + to_f32(a));
    }
    if constexpr (PACK) own_row[i] = packed;
    if (out) out[i] = acc;
    if constexpr (UNPACK) grad[i] = finish(acc);
  };

  if (h >= 0) {
    const int64_t nvec = (n - h) / E;
    In x[U][W][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = int64_t(c) * VPB + int64_t(u) * kBlock + t;
      if constexpr (kWave) {
#pragma unroll
        for (int r = 0; r < W; ++r) {
#pragma unroll
          for (int e = 0; e < E; ++e) x[u][r][e] = zero_of<In>();
        }
      }
      if (v < nvec) {
#pragma unroll
        for (int r = 0; r < W; ++r) {
          if (PACK && r == rank && own_zero) {
#pragma unroll
            for (int e = 0; e < E; ++e) x[u][r][e] = zero_of<In>();
          } else {
            vload<In, E, true>(x[u][r], src[r] + h + v * E);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v0 = int64_t(c) * VPB + int64_t(u) * kBlock;  // the fragment of lane 0
      const int64_t v = v0 + t;
      const bool active = v < nvec;
      // elements of this wave's fragment that exist (wave-permuted stores only)
      const int limit = int(max_size(0, int(min_i64(nvec - v0, kBlock)))) * E;
      if (kWave || active) {
        const int64_t i = h + v * E;
        if constexpr (PACK) {
          // This rank's fragment, packed in registers (static indices: the
          // branch on the wave-uniform rank picks the replica slot).
          In po[E];
#pragma unroll
          for (int e = 0; e < E; ++e) po[e] = zero_of<In>();
#pragma unroll
          for (int r = 0; r < W; ++r) {
            if (r == rank) {
#pragma unroll
              for (int e = 0; e < E; ++e) {
                x[u][r][e] = pack_op(x[u][r][e]);
                po[e] = x[u][r][e];
              }
            }
          }
          if (active) vstore<In, E, true>(own_row + i, po);
        }
        T y[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
          T acc = widen(x[u][0][e]);
#pragma unroll
          for (int r = 1; r < W; ++r) acc = from_f32<T>(to_f32(acc) + to_f32(widen(x[u][r][e])));
          y[e] = acc;
        }
        if (out) {
          if constexpr (kWaveT) {
            vstore_wave8<T>(out + h + v0 * E, y, t, limit);
          } else if (active) {
            vstore<T, E, true>(out + i, y);
          }
        }
        if constexpr (UNPACK) {
          G gy[E];
#pragma unroll
          for (int e = 0; e < E; ++e) gy[e] = finish(y[e]);
          if constexpr (kWaveG) {
            vstore_wave8<G>(grad + h + v0 * E, gy, t, limit);
          } else if (active) {
            vstore<G, E, true>(grad + i, gy);
          }
        }
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
  if constexpr (UNPACK) {
    if (p.found_inf) flag_nonfinite(bad, p.found_inf);
  }
}

// Table in the kernel-argument segment.
template <typename T, typename G, int W, bool UNPACK>
__global__ void __launch_bounds__(kBlock) allreduce_kernel(PieceBatch b, ReduceParams p) {
  allreduce_body<T, T, G, W, UNPACK, false, false>(PieceArgView{b}, p);
}

// Table (plan) in device memory; the fused all-reduce + unpack only.
template <typename T, typename G, int W>
__global__ void __launch_bounds__(kBlock) allreduce_unpack_kernel_dev(DevTable t, ReduceParams p) {
  allreduce_body<T, T, G, W, true, false, false>(DevView{t}, p);
}

// Widening variants (fused all-reduce + unpack with pre-scale at the receiver).
template <typename In, typename T, typename G, int W>
__global__ void __launch_bounds__(kBlock) allreduce_wide_kernel(PieceBatch b, ReduceParams p) {
  allreduce_body<In, T, G, W, true, true, false>(PieceArgView{b}, p);
}

template <typename In, typename T, typename G, int W>
__global__ void __launch_bounds__(kBlock) allreduce_wide_kernel_dev(DevTable t, ReduceParams p) {
  allreduce_body<In, T, G, W, true, true, false>(DevView{t}, p);
}

// Pack fused into the all-reduce + unpack: gradients of the wire dtype In,
// bucket dtype T (T != In: widening, pre-scaled at the receiver).
template <typename In, typename T, int W>
__global__ void __launch_bounds__(kBlock) allreduce_pack_kernel(PieceBatch b, ReduceParams p) {
  allreduce_body<In, T, In, W, true, (sizeof(In) != sizeof(T)), true>(PieceArgView{b}, p);
}

template <typename In, typename T, int W>
__global__ void __launch_bounds__(kBlock) allreduce_pack_kernel_dev(DevTable t, ReduceParams p) {
  allreduce_body<In, T, In, W, true, (sizeof(In) != sizeof(T)), true>(DevView{t}, p);
}

template <typename T, typename G, bool UNPACK>
struct ArgAllreduce {
  const PieceBatch& b;
  template <int W>
  hipError_t go(const ReduceParams& p, hipStream_t stream) const {
    hipLaunchKernelGGL((allreduce_kernel<T, G, W, UNPACK>), dim3(b.first_block[b.count]), dim3(kBlock), 0,
                       stream, b, p);
    return hipGetLastError();
  }
};

template <typename T, typename G>
struct DevAllreduceUnpack {
  const DevTable& t;
  int blocks;
  template <int W>
  hipError_t go(const ReduceParams& p, hipStream_t stream) const {
    return launch_plan_slices(t, blocks, [&](const DevTable& slice, int grid) {
      hipLaunchKernelGGL((allreduce_unpack_kernel_dev<T, G, W>), dim3(grid), dim3(kBlock), 0, stream, slice, p);
    });
  }
};

template <typename In, typename T, typename G>
struct ArgWide {
  const PieceBatch& b;
  template <int W>
  hipError_t go(const ReduceParams& p, hipStream_t stream) const {
    hipLaunchKernelGGL((allreduce_wide_kernel<In, T, G, W>), dim3(b.first_block[b.count]), dim3(kBlock), 0,
                       stream, b, p);
    return hipGetLastError();
  }
};

template <typename In, typename T, typename G>
struct DevWide {
  const DevTable& t;
  int blocks;
  template <int W>
  hipError_t go(const ReduceParams& p, hipStream_t stream) const {
    return launch_plan_slices(t, blocks, [&](const DevTable& slice, int grid) {
      hipLaunchKernelGGL((allreduce_wide_kernel_dev<In, T, G, W>), dim3(grid), dim3(kBlock), 0, stream, slice, p);
    });
  }
};

template <typename In, typename T>
struct ArgPack {
  const PieceBatch& b;
  template <int W>
  hipError_t go(const ReduceParams& p, hipStream_t stream) const {
    hipLaunchKernelGGL((allreduce_pack_kernel<In, T, W>), dim3(b.first_block[b.count]), dim3(kBlock), 0, stream,
                       b, p);
    return hipGetLastError();
  }
};

template <typename In, typename T>
struct DevPack {
  const DevTable& t;
  int blocks;
  template <int W>
  hipError_t go(const ReduceParams& p, hipStream_t stream) const {
    return launch_plan_slices(t, blocks, [&](const DevTable& slice, int grid) {
      hipLaunchKernelGGL((allreduce_pack_kernel_dev<In, T, W>), dim3(grid), dim3(kBlock), 0, stream, slice, p);
    });
  }
};

template <typename L>
hipError_t by_world(int world, const L& l, const ReduceParams& p, hipStream_t stream) {
  switch (world) {
    case 1: return l.template go<1>(p, stream);
    case 2: return l.template go<2>(p, stream);
    case 3: return l.template go<3>(p, stream);
    case 4: return l.template go<4>(p, stream);
    case 5: return l.template go<5>(p, stream);
    case 6: return l.template go<6>(p, stream);
    case 7: return l.template go<7>(p, stream);
    case 8: return l.template go<8>(p, stream);
    case 9: return l.template go<9>(p, stream);
    case 10: return l.template go<10>(p, stream);
    case 11: return l.template go<11>(p, stream);
    case 12: return l.template go<12>(p, stream);
    case 13: return l.template go<13>(p, stream);
    case 14: return l.template go<14>(p, stream);
    case 15: return l.template go<15>(p, stream);
    default: return l.template go<16>(p, stream);
  }
}

template <typename T, typename G, bool UNPACK>
hipError_t launch_allreduce(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return by_world(world, ArgAllreduce<T, G, UNPACK>{b}, p, stream);
}

template <typename T, typename G>
hipError_t launch_allreduce_unpack_dev(int world, const DevTable& t, int blocks, const ReduceParams& p,
                                       hipStream_t stream) {
  return by_world(world, DevAllreduceUnpack<T, G>{t, blocks}, p, stream);
}

template <typename In, typename T, typename G>
hipError_t launch_allreduce_wide(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return by_world(world, ArgWide<In, T, G>{b}, p, stream);
}

template <typename In, typename T, typename G>
hipError_t launch_allreduce_wide_dev(int world, const DevTable& t, int blocks, const ReduceParams& p,
                                     hipStream_t stream) {
  return by_world(world, DevWide<In, T, G>{t, blocks}, p, stream);
}

// Per-dtype instantiation sets, one call each from the instantiating
// translation units: T is the bucket dtype (plain SUM and fused unpack into
// any gradient dtype); In is the wire dtype of the widening variant.
template <typename T>
hipError_t launch_allreduce_for(int grad_dtype, bool unpack, int world, const PieceBatch& b,
                                const ReduceParams& p, hipStream_t stream) {
  if (!unpack) return launch_allreduce<T, T, false>(world, b, p, stream);
  if (grad_dtype == MDX_F32) return launch_allreduce<T, float, true>(world, b, p, stream);
  if (grad_dtype == MDX_BF16) return launch_allreduce<T, bf16, true>(world, b, p, stream);
  return launch_allreduce<T, f16, true>(world, b, p, stream);
}

template <typename T>
hipError_t launch_allreduce_dev_for(int grad_dtype, int world, const DevTable& t, int blocks,
                                    const ReduceParams& p, hipStream_t stream) {
  if (grad_dtype == MDX_F32) return launch_allreduce_unpack_dev<T, float>(world, t, blocks, p, stream);
  if (grad_dtype == MDX_BF16) return launch_allreduce_unpack_dev<T, bf16>(world, t, blocks, p, stream);
  return launch_allreduce_unpack_dev<T, f16>(world, t, blocks, p, stream);
}

template <typename In>
hipError_t launch_wide_for(int grad_dtype, int world, const PieceBatch& b, const ReduceParams& p,
                           hipStream_t stream) {
  if (grad_dtype == MDX_F32) return launch_allreduce_wide<In, float, float>(world, b, p, stream);
  if (grad_dtype == MDX_BF16) return launch_allreduce_wide<In, float, bf16>(world, b, p, stream);
  return launch_allreduce_wide<In, float, f16>(world, b, p, stream);
}

template <typename In>
hipError_t launch_wide_dev_for(int grad_dtype, int world, const DevTable& t, int blocks, const ReduceParams& p,
                               hipStream_t stream) {
  if (grad_dtype == MDX_F32) return launch_allreduce_wide_dev<In, float, float>(world, t, blocks, p, stream);
  if (grad_dtype == MDX_BF16) return launch_allreduce_wide_dev<In, float, bf16>(world, t, blocks, p, stream);
  return launch_allreduce_wide_dev<In, float, f16>(world, t, blocks, p, stream);
}

// The fused pack + all-reduce + unpack of one (wire, bucket) dtype pair.
template <typename In, typename T>
hipError_t launch_pack_for(int world, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  return by_world(world, ArgPack<In, T>{b}, p, stream);
}

template <typename In, typename T>
hipError_t launch_pack_dev_for(int world, const DevTable& t, int blocks, const ReduceParams& p,
                               hipStream_t stream) {
  return by_world(world, DevPack<In, T>{t, blocks}, p, stream);
}

// ---------------------------------------------------------------------------
// reduce-scatter share
// ---------------------------------------------------------------------------

enum : int { kPreNone = 0, kPreMul = 1, kPreDiv = 2 };

template <typename In, typename Acc, typename Out, int WMAX, int PRE, bool ACC>
__device__ __forceinline__ void share_body(const PieceRun& run, const ReduceParams& p) {
  constexpr int E = reduce_frag_elems(int(sizeof(In)), int(sizeof(Out)), int(sizeof(Out)));
  constexpr int U = share_unroll(WMAX, E * int(sizeof(In)));
  constexpr int VPB = kBlock * U;
  constexpr int EPB = VPB * E;
  // 32-byte fragments of the shard dtype go out through vstore_wave8 (16-bit
  // contributions into an fp32 shard), as in allreduce_body.
  constexpr bool kWave = E * int(sizeof(Out)) == 32;
  static_assert(!kWave || E == 8, "wave-permuted stores take 8 four-byte elements per lane");

  const int c = run.c;
  const int nblk = run.nblk;
  const int64_t pos = run.pos;
  const int64_t n = run.numel;
  const int32_t h = run.head;
  const int world = p.world;
  const int rank = p.rank;
  const bool own_zero = (run.own == nullptr);
  const int t = int(threadIdx.x);
  const float pre = p.pre;
  const bool unscale = (p.flags & kRedUnscale) != 0;
  const float inv = p.inv_scale;

  const In* src[WMAX];
#pragma unroll
  for (int r = 0; r < WMAX; ++r) {
    src[r] = (r == rank) ? static_cast<const In*>(run.own) : static_cast<const In*>(p.peer[r]) + pos;
  }
  // A piece of a multi-unit share carries its own destination (each unit's
  // shard gradient is a tensor of its own); otherwise the shard is p.out.
  Out* out = run.grad ? static_cast<Out*>(run.grad) : static_cast<Out*>(p.out) + pos;
  bool bad = false;

  auto widen = [&](In x) -> Acc {
    Acc a = Cvt<In, Acc>::run(x);
    if constexpr (PRE == kPreMul) a = from_f32<Acc>(to_f32(a) * pre);
    if constexpr (PRE == kPreDiv) a = from_f32<Acc>(to_f32(a) / pre);
    return a;
  };
  auto finish = [&](Acc acc, Out prev) -> Out {
    Out y = Cvt<Acc, Out>::run(acc);
    if constexpr (ACC) y = from_f32<Out>(to_f32(prev) + to_f32(y));
    const Out ys = from_f32<Out>(to_f32(y) * inv);
    y = unscale ? ys : y;
    bad |= !is_finite(y);
    return y;
  };
  auto element = [&](int64_t i) {
    Acc acc = zero_of<Acc>();
#pragma unroll
    for (int r = 0; r < WMAX; ++r) {
      if (r < world) {
        const In x = (r == rank && own_zero) ? zero_of<In>() : src[r][i];
        const Acc a = widen(x);
        acc = (r == 0) ? a : from_f32<Acc>(to_f32(acc) + to_f32(a));
      }
    }
    const Out prev = ACC ? out[i] : zero_of<Out>();
    out[i] = finish(acc, prev);
  };

  if (h >= 0) {
    const int64_t nvec = (n - h) / E;
    In x[U][WMAX][E];
    Out prev[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = int64_t(c) * VPB + int64_t(u) * kBlock + t;
      if constexpr (kWave) {
#pragma unroll
        for (int k = 0; k < E; ++k) {
#pragma unroll
          for (int r = 0; r < WMAX; ++r) x[u][r][k] = zero_of<In>();
          prev[u][k] = zero_of<Out>();
        }
      }
      if (v < nvec) {
        const int64_t i = h + v * E;
#pragma unroll
        for (int r = 0; r < WMAX; ++r) {
          if (r < world) {
            if (r == rank && own_zero) {
#pragma unroll
              for (int k = 0; k < E; ++k) x[u][r][k] = zero_of<In>();
            } else {
              vload<In, E, true>(x[u][r], src[r] + i);
            }
          }
        }
        if constexpr (ACC) vload<Out, E, false>(prev[u], out + i);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v0 = int64_t(c) * VPB + int64_t(u) * kBlock;  // the fragment of lane 0
      const int64_t v = v0 + t;
      const bool active = v < nvec;
      const int limit = int(max_size(0, int(min_i64(nvec - v0, kBlock)))) * E;
      if (kWave || active) {
        Out y[E];
#pragma unroll
        for (int k = 0; k < E; ++k) {
          Acc acc = widen(x[u][0][k]);
#pragma unroll
          for (int r = 1; r < WMAX; ++r) {
            if (r < world) acc = from_f32<Acc>(to_f32(acc) + to_f32(widen(x[u][r][k])));
          }
          y[k] = finish(acc, ACC ? prev[u][k] : zero_of<Out>());
        }
        if constexpr (kWave) {
          vstore_wave8<Out>(out + h + v0 * E, y, t, limit);
        } else {
          vstore<Out, E, true>(out + h + v * E, y);
        }
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
  if (p.found_inf) flag_nonfinite(bad, p.found_inf);
}

template <typename In, typename Acc, typename Out, int WMAX>
__device__ __forceinline__ void share_run(const PieceRun& run, const ReduceParams& p) {
  const bool acc = (p.flags & kRedAccumulate) != 0;
  if (p.flags & kRedPreMul) {
    if (acc) share_body<In, Acc, Out, WMAX, kPreMul, true>(run, p);
    else share_body<In, Acc, Out, WMAX, kPreMul, false>(run, p);
  } else if (p.flags & kRedPreDiv) {
    if (acc) share_body<In, Acc, Out, WMAX, kPreDiv, true>(run, p);
    else share_body<In, Acc, Out, WMAX, kPreDiv, false>(run, p);
  } else {
    if (acc) share_body<In, Acc, Out, WMAX, kPreNone, true>(run, p);
    else share_body<In, Acc, Out, WMAX, kPreNone, false>(run, p);
  }
}

template <typename In, typename Acc, typename Out, int WMAX>
__global__ void __launch_bounds__(kBlock) share_kernel(PieceBatch b, ReduceParams p) {
  share_run<In, Acc, Out, WMAX>(PieceArgView{b}.piece_run(int(blockIdx.x)), p);
}

// One piece (an FSDP unit's shard) in the kernel-argument segment.
template <typename In, typename Acc, typename Out, int WMAX>
__global__ void __launch_bounds__(kBlock) share_kernel_one(PieceOne b, ReduceParams p) {
  share_run<In, Acc, Out, WMAX>(PieceOneView{b}.piece_run(int(blockIdx.x)), p);
}

// Up to kFewRuns pieces in the kernel-argument segment.
template <typename In, typename Acc, typename Out, int WMAX>
__global__ void __launch_bounds__(kBlock) share_kernel_few(PieceFew b, ReduceParams p) {
  share_run<In, Acc, Out, WMAX>(PieceFewView{b}.piece_run(int(blockIdx.x)), p);
}

// Pieces of a device plan: the shares of many FSDP units in one dispatch.
template <typename In, typename Acc, typename Out, int WMAX>
__global__ void __launch_bounds__(kBlock) share_kernel_dev(DevTable t, ReduceParams p) {
  const DevView v{t};
  share_run<In, Acc, Out, WMAX>(v.piece_run(v.block()), p);
}

template <typename In, typename Acc, typename Out, int WMAX>
hipError_t launch_share_dev_w(const DevTable& t, int blocks, const ReduceParams& p, hipStream_t stream) {
  return launch_plan_slices(t, blocks, [&](const DevTable& slice, int grid) {
    hipLaunchKernelGGL((share_kernel_dev<In, Acc, Out, WMAX>), dim3(grid), dim3(kBlock), 0, stream, slice, p);
  });
}

template <typename In, typename Acc, typename Out, int WMAX>
hipError_t launch_share_w(const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  if (b.count == 1) {
    hipLaunchKernelGGL((share_kernel_one<In, Acc, Out, WMAX>), dim3(b.first_block[1]), dim3(kBlock), 0, stream,
                       one_run_of(b), p);
  } else if (b.count <= kFewRuns) {
    hipLaunchKernelGGL((share_kernel_few<In, Acc, Out, WMAX>), dim3(b.first_block[b.count]), dim3(kBlock), 0,
                       stream, few_runs_of(b), p);
  } else {
    hipLaunchKernelGGL((share_kernel<In, Acc, Out, WMAX>), dim3(b.first_block[b.count]), dim3(kBlock), 0, stream,
                       b, p);
  }
  return hipGetLastError();
}

// Every (Acc, Out) pair for contributions of type In at the widest class
// (runtime W <= 16), except (fp32, fp32), which has width-specialised kernels.
template <typename In, typename Acc>
hipError_t share16_out(int out_dtype, const PieceBatch& b, const ReduceParams& p, hipStream_t stream) {
  if (out_dtype == MDX_BF16) return launch_share_w<In, Acc, bf16, 16>(b, p, stream);
  if (out_dtype == MDX_F16) return launch_share_w<In, Acc, f16, 16>(b, p, stream);
  if constexpr (sizeof(Acc) == 4) {
    return hipErrorInvalidValue;  // (fp32, fp32) goes to the width-specialised kernels
  } else {
    return launch_share_w<In, Acc, float, 16>(b, p, stream);
  }
}

template <typename In>
hipError_t launch_share_generic_for(int acc_dtype, int out_dtype, const PieceBatch& b, const ReduceParams& p,
                                    hipStream_t stream) {
  if (acc_dtype == MDX_F32) return share16_out<In, float>(out_dtype, b, p, stream);
  if (acc_dtype == MDX_BF16) return share16_out<In, bf16>(out_dtype, b, p, stream);
  return share16_out<In, f16>(out_dtype, b, p, stream);
}

}  // namespace reduce_impl
}  // namespace mdx
