// W-way all-reduce with a non-SUM operation (MAX, MIN, PRODUCT) over W
// replica buffers resident in HBM: comm.all_reduce(tensor, op) and
// comm.reduce_scatter_tensor(..., op) for the ops the gradient path itself
// never uses (the found-inf flag's MAX, a caller's own MIN or PRODUCT).
//
// Per element, in the fixed rank order:
//   acc = x_0;  acc = f(acc, x_r) for r = 1 .. W-1;  out = acc
// with f the IEEE 754-2019 operations that torch's CPU maximum, minimum and
// mul compute:
//   MAX      NaN if either is NaN, else the larger, with -0 < +0
//   MIN      NaN if either is NaN, else the smaller, with -0 < +0
//   PRODUCT  rnd_T(f32(acc) * f32(x))
// MAX and MIN round nothing: the result is an input, or for a tie of equal
// values (whose bits differ only for zeros) the AND (MAX) or OR (MIN) of the
// two patterns -- +0 or -0 whatever the rank order; a NaN result is the
// dtype's quiet NaN.  A product of two bf16 or fp16 values is exact in fp32,
// so each step rounds once, to T, as torch's CPU multiply does.
//
// Layout of the work: one-wave workgroups; a lane takes U 16-byte vectors (E
// elements each) of every replica, all loaded (non-temporal) before the first
// fold, U = op_unroll(WMAX) so that about 128 bytes are in flight per lane,
// with WMAX >= W a compile-time bound and the ranks past W predicated off.
// Vector accesses go through the library's 2-byte-aligned vector views, so a
// run at any element offset moves in vectors; the last fewer-than-E elements
// of a run are folded one per lane by its last workgroup.  The runs travel in
// the dispatch's kernel arguments.
#include <type_traits>

#include "mdx_internal.h"

namespace mdx {
namespace {

template <typename T>
__device__ __forceinline__ bool is_nan(T x) {
  return __builtin_isnan(to_f32(x));
}

template <typename T>
__device__ __forceinline__ T quiet_nan() {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(0x7fc00000u);
  } else if constexpr (std::is_same_v<T, bf16>) {
    return T{uint16_t(0x7fc0u)};
  } else {
    return T{uint16_t(0x7e00u)};
  }
}

__device__ __forceinline__ uint32_t bits_of(float x) { return __float_as_uint(x); }
__device__ __forceinline__ uint32_t bits_of(bf16 x) { return x.u; }
__device__ __forceinline__ uint32_t bits_of(f16 x) { return x.u; }

template <typename T>
__device__ __forceinline__ T from_bits(uint32_t u) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(u);
  } else {
    return T{uint16_t(u)};
  }
}

template <typename T, int OP>
__device__ __forceinline__ T fold(T acc, T x) {
  if constexpr (OP == MDX_OP_PRODUCT) {
    return from_f32<T>(to_f32(acc) * to_f32(x));
  } else {
    if (is_nan(acc) || is_nan(x)) return quiet_nan<T>();
    const float a = to_f32(acc), b = to_f32(x);
    if (a < b) return OP == MDX_OP_MAX ? x : acc;
    if (b < a) return OP == MDX_OP_MAX ? acc : x;
    return OP == MDX_OP_MAX ? from_bits<T>(bits_of(acc) & bits_of(x)) : from_bits<T>(bits_of(acc) | bits_of(x));
  }
}

template <typename T, int OP, int WMAX>
__global__ void __launch_bounds__(kBlock) allreduce_op_kernel(OpRuns t, OpParams p) {
  constexpr int E = 16 / int(sizeof(T));
  constexpr int U = op_unroll(WMAX);
  const int blk = int(blockIdx.x);
  const int s = find_run_in(t.first_block, 0, t.count, blk);
  const int64_t c = blk - t.first_block[s];
  const int64_t nblk = t.first_block[s + 1] - t.first_block[s];
  const int64_t off = t.offset[s];
  const int64_t n = t.numel[s];
  const int64_t nvec = n / E;
  const int lane = int(threadIdx.x);
  const int world = p.world;
  const T* rows[WMAX];
#pragma unroll
  for (int r = 0; r < WMAX; ++r) rows[r] = r < world ? static_cast<const T*>(p.rep[r]) + off : nullptr;
  T* out = static_cast<T*>(p.out) + off;

  T x[U][WMAX][E];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t v = c * (kBlock * U) + int64_t(u) * kBlock + lane;
    if (v < nvec) {
#pragma unroll
      for (int r = 0; r < WMAX; ++r) {
        if (r < world) vload<T, E, true>(x[u][r], rows[r] + v * E);
      }
    }
  }
  // Every replica's vectors are loaded before the first store: the in-place form (out = a
  // replica's base) only rewrites elements this lane alone reads.
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t v = c * (kBlock * U) + int64_t(u) * kBlock + lane;
    if (v < nvec) {
      T acc[E];
#pragma unroll
      for (int k = 0; k < E; ++k) acc[k] = x[u][0][k];
#pragma unroll
      for (int r = 1; r < WMAX; ++r) {
        if (r < world) {
#pragma unroll
          for (int k = 0; k < E; ++k) acc[k] = fold<T, OP>(acc[k], x[u][r][k]);
        }
      }
      vstore<T, E, true>(out + v * E, acc);
    }
  }
  // The run's last fewer-than-E elements, one per lane of its last workgroup.
  const int64_t i = nvec * E + lane;
  if (c == nblk - 1 && i < n) {
    T acc = rows[0][i];
    for (int r = 1; r < world; ++r) acc = fold<T, OP>(acc, rows[r][i]);
    out[i] = acc;
  }
}

template <typename T, int OP>
hipError_t launch_op(int wmax, const OpRuns& t, int blocks, const OpParams& p, hipStream_t stream) {
  const dim3 grid(blocks), block(kBlock);
  if (wmax == 2) {
    hipLaunchKernelGGL((allreduce_op_kernel<T, OP, 2>), grid, block, 0, stream, t, p);
  } else if (wmax == 4) {
    hipLaunchKernelGGL((allreduce_op_kernel<T, OP, 4>), grid, block, 0, stream, t, p);
  } else if (wmax == 8) {
    hipLaunchKernelGGL((allreduce_op_kernel<T, OP, 8>), grid, block, 0, stream, t, p);
  } else {
    hipLaunchKernelGGL((allreduce_op_kernel<T, OP, 16>), grid, block, 0, stream, t, p);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(int op, int wmax, const OpRuns& t, int blocks, const OpParams& p, hipStream_t stream) {
  if (op == MDX_OP_MAX) return launch_op<T, MDX_OP_MAX>(wmax, t, blocks, p, stream);
  if (op == MDX_OP_MIN) return launch_op<T, MDX_OP_MIN>(wmax, t, blocks, p, stream);
  return launch_op<T, MDX_OP_PRODUCT>(wmax, t, blocks, p, stream);
}

}  // namespace

hipError_t launch_allreduce_op(int dtype, int op, int wmax, const OpRuns& t, int blocks, const OpParams& p,
                               hipStream_t stream) {
  if (dtype == MDX_BF16) return launch_t<bf16>(op, wmax, t, blocks, p, stream);
  if (dtype == MDX_F16) return launch_t<f16>(op, wmax, t, blocks, p, stream);
  return launch_t<float>(op, wmax, t, blocks, p, stream);
}

}  // namespace mdx
