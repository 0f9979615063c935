// Weighted combine of the expert outputs of a routed MoE layer, atomic-free: one
// block per token row t, out[t][:] = sum_k w[t][k] * x[pos[t][k]][:], accumulated in
// fp32 (fp64 for fp64 rows) and rounded once. Each output row is owned by one block, so no atomics.
// A position outside [0, x_rows) contributes nothing (it is never dereferenced).
// x may hold `splits` partial products of a K-split GEMM (fp32, split_stride apart):
// they are summed per row before the weighting, and the output dtype is separate.
// HBM-bound: k rows read, one row written; 16-byte vector accesses when the rows allow.
#include <type_traits>

#include "common.h"

namespace mls {

namespace {

// Accumulator of a combine: fp32, or fp64 for fp64 rows (the reference's ACC64 keeps
// fp64 expert outputs at full precision, kernels/moe_routing.py:54-72, 112, so that a
// finite-difference gradcheck sees through the op). Weights are converted to it.
template <typename T> struct CombineAcc { using type = float; };
template <> struct CombineAcc<double> { using type = double; };

template <typename A, typename T>
__device__ __forceinline__ A to_acc(T v) {
  if constexpr (std::is_same_v<T, double>) return (A)v;
  else return (A)to_f32(v);
}

template <typename OT, typename A>
__device__ __forceinline__ OT from_acc(A v) {
  if constexpr (std::is_same_v<A, double>) return v;  // fp64 rows give fp64 output
  else return from_f32<OT>(v);
}

template <typename T, typename WT, typename OT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const T* __restrict__ x, int64_t ldx, int64_t x_rows,
                                                          int splits, int64_t sstride,
                                                          const WT* __restrict__ w,
                                                          const int64_t* __restrict__ pos, int k,
                                                          OT* __restrict__ out, int64_t ldo, int64_t D,
                                                          bool vec) {
  using A = typename CombineAcc<T>::type;
  const int64_t t = blockIdx.x;
  if (vec) {
    // 8 elements per thread and step: one 16-byte access of 16-bit data, two of fp32,
    // four of fp64 (rows and d are multiples of 8 elements, so every access is aligned)
    constexpr int V = 8, XQ = V * (int)sizeof(T) / 16, OQ = V * (int)sizeof(OT) / 16;
    for (int64_t d = (int64_t)threadIdx.x * V; d < D; d += (int64_t)blockDim.x * V) {
      A acc[V];
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = 0;
      for (int s = 0; s < k; ++s) {
        const int64_t r = pos[t * k + s];
        if (r < 0 || r >= x_rows) continue;
        const A ws = to_acc<A>(w[t * k + s]);
        A row[V];
#pragma unroll
        for (int i = 0; i < V; ++i) row[i] = 0;
        for (int sp = 0; sp < splits; ++sp) {  // the partial products of a K split
          const T* src = x + sp * sstride + r * ldx + d;
          T v[V];
#pragma unroll
          for (int q = 0; q < XQ; ++q) reinterpret_cast<uint4*>(v)[q] = reinterpret_cast<const uint4*>(src)[q];
#pragma unroll
          for (int i = 0; i < V; ++i) row[i] += to_acc<A>(v[i]);
        }
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = fma(ws, row[i], acc[i]);
      }
      OT o[V];
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = from_acc<OT>(acc[i]);
#pragma unroll
      for (int q = 0; q < OQ; ++q)
        reinterpret_cast<uint4*>(out + t * ldo + d)[q] = reinterpret_cast<const uint4*>(o)[q];
    }
  } else {
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
      A acc = 0;
      for (int s = 0; s < k; ++s) {
        const int64_t r = pos[t * k + s];
        if (r < 0 || r >= x_rows) continue;
        A row = 0;
        for (int sp = 0; sp < splits; ++sp) row += to_acc<A>(x[sp * sstride + r * ldx + d]);
        acc = fma(to_acc<A>(w[t * k + s]), row, acc);
      }
      out[t * ldo + d] = from_acc<OT>(acc);
    }
  }
}

template <typename T, typename OT>
int launch_combine(const void* x, int64_t ldx, int64_t x_rows, int splits, int64_t sstride, const void* w,
                   int w_dt, const int64_t* pos, int64_t T_, int k, void* out, int64_t ldo, int64_t D,
                   hipStream_t st) {
  const bool vec = D % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && sstride % 8 == 0 && aligned(x, 16) &&
                   aligned(out, 16);
  const dim3 grid((unsigned)T_), block(256);
#define MLS_COMBINE(WT)                                                                                   \
  hipLaunchKernelGGL((moe_combine_kernel<T, WT, OT>), grid, block, 0, st, (const T*)x, ldx, x_rows, splits, \
                     sstride, (const WT*)w, pos, k, (OT*)out, ldo, D, vec)
  if (w_dt == MLS_F32) MLS_COMBINE(float);
  else if (w_dt == MLS_F16) MLS_COMBINE(_Float16);
  else if (w_dt == MLS_F64) MLS_COMBINE(double);
  else MLS_COMBINE(__bf16);
#undef MLS_COMBINE
  return check_launch("mls_moe_combine");
}

template <typename T>
int launch_combine_out(int out_dt, const void* x, int64_t ldx, int64_t x_rows, int splits, int64_t sstride,
                       const void* w, int w_dt, const int64_t* pos, int64_t T_, int k, void* out, int64_t ldo,
                       int64_t D, hipStream_t st) {
  if (out_dt == MLS_F32) return launch_combine<T, float>(x, ldx, x_rows, splits, sstride, w, w_dt, pos, T_, k, out, ldo, D, st);
  if (out_dt == MLS_F16) return launch_combine<T, _Float16>(x, ldx, x_rows, splits, sstride, w, w_dt, pos, T_, k, out, ldo, D, st);
  return launch_combine<T, __bf16>(x, ldx, x_rows, splits, sstride, w, w_dt, pos, T_, k, out, ldo, D, st);
}

}  // namespace

}  // namespace mls

using namespace mls;

extern "C" int mls_moe_combine(const void* x, int x_dt, int64_t ldx, int64_t x_rows, int splits,
                               int64_t split_stride, const void* w, int w_dt, const int64_t* pos, int64_t T, int k,
                               void* out, int out_dt, int64_t ldo, int64_t D, mls_stream_t stream) {
  const char* fn = "mls_moe_combine";
  if (T < 0 || D < 0 || k < 1 || x_rows < 0 || splits < 1)
    return fail(MLS_ERR_ARG, "%s: bad sizes T=%lld k=%d D=%lld splits=%d", fn, (long long)T, k, (long long)D,
                splits);
  // fp64 rows (accumulated in fp64, fp64 output) or 16/32-bit rows (fp32 accumulation, any
  // 16/32-bit output); weights of any of the four dtypes
  const bool x64 = x_dt == MLS_F64;
  if ((!x64 && !is_float_dt(x_dt)) || (!is_float_dt(w_dt) && w_dt != MLS_F64) ||
      (x64 ? out_dt != MLS_F64 : !is_float_dt(out_dt)))
    return fail(MLS_ERR_ARG, "%s: bad dtype (x %d, w %d, out %d; fp64 rows need an fp64 output)", fn, x_dt, w_dt,
                out_dt);
  if (T == 0 || D == 0) return MLS_OK;
  if (!pos || !out || !w || (x_rows > 0 && !x)) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (ldx < D || ldo < D || (splits > 1 && split_stride < x_rows * ldx))
    return fail(MLS_ERR_ARG, "%s: bad leading dimension or split stride", fn);
  if (T > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "%s: T too large", fn);
  hipStream_t st = (hipStream_t)stream;
  const int64_t ss = splits > 1 ? split_stride : 0;
  if (x64) return launch_combine<double, double>(x, ldx, x_rows, splits, ss, w, w_dt, pos, T, k, out, ldo, D, st);
  if (x_dt == MLS_F32) return launch_combine_out<float>(out_dt, x, ldx, x_rows, splits, ss, w, w_dt, pos, T, k, out, ldo, D, st);
  if (x_dt == MLS_F16) return launch_combine_out<_Float16>(out_dt, x, ldx, x_rows, splits, ss, w, w_dt, pos, T, k, out, ldo, D, st);
  return launch_combine_out<__bf16>(out_dt, x, ldx, x_rows, splits, ss, w, w_dt, pos, T, k, out, ldo, D, st);
}
