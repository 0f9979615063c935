// Weighted combine of the expert outputs of a routed MoE layer, atomic-free: one
// block per token row t, out[t][:] = sum_k w[t][k] * x[pos[t][k]][:], accumulated in
// fp32 and rounded once. Each output row is owned by one block, so no atomics.
// A position outside [0, x_rows) contributes nothing (it is never dereferenced).
// HBM-bound: k rows read, one row written; 16-byte vector accesses when the rows allow.
#include "common.h"

namespace mls {

namespace {

template <typename T, typename WT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const T* __restrict__ x, int64_t ldx,
                                                          const WT* __restrict__ w,
                                                          const int64_t* __restrict__ pos, int k,
                                                          int64_t x_rows, T* __restrict__ out, int64_t ldo, int64_t D,
                                                          bool vec) {
  const int64_t t = blockIdx.x;
  if (vec) {
    // 8 elements (16 bytes of 16-bit data, or two float4 of fp32) per thread and step
    constexpr int V = 8;
    for (int64_t d = (int64_t)threadIdx.x * V; d < D; d += (int64_t)blockDim.x * V) {
      float acc[V] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < k; ++s) {
        const int64_t r = pos[t * k + s];
        if (r < 0 || r >= x_rows) continue;
        const float ws = to_f32(w[t * k + s]);
        const T* src = x + r * ldx + d;
        T v[V];
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<uint4*>(v) = *reinterpret_cast<const uint4*>(src);
        } else {
          *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(src);
          *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(src + 4);
        }
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = fmaf(ws, to_f32(v[i]), acc[i]);
      }
      T o[V];
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = from_f32<T>(acc[i]);
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint4*>(out + t * ldo + d) = *reinterpret_cast<const uint4*>(o);
      } else {
        *reinterpret_cast<float4*>(out + t * ldo + d) = *reinterpret_cast<const float4*>(o);
        *reinterpret_cast<float4*>(out + t * ldo + d + 4) = *reinterpret_cast<const float4*>(o + 4);
      }
    }
  } else {
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
      float acc = 0.f;
      for (int s = 0; s < k; ++s) {
        const int64_t r = pos[t * k + s];
        if (r >= 0 && r < x_rows) acc = fmaf(to_f32(w[t * k + s]), to_f32(x[r * ldx + d]), acc);
      }
      out[t * ldo + d] = from_f32<T>(acc);
    }
  }
}

template <typename T>
int launch_combine(const void* x, int64_t ldx, int64_t x_rows, const void* w, int w_dt, const int64_t* pos,
                   int64_t T_, int k, void* out, int64_t ldo, int64_t D, hipStream_t st) {
  const bool vec = D % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && aligned(x, 16) && aligned(out, 16);
  const dim3 grid((unsigned)T_), block(256);
#define MLS_COMBINE(WT)                                                                              \
  hipLaunchKernelGGL((moe_combine_kernel<T, WT>), grid, block, 0, st, (const T*)x, ldx, (const WT*)w, \
                     pos, k, x_rows, (T*)out, ldo, D, vec)
  if (w_dt == MLS_F32) MLS_COMBINE(float);
  else if (w_dt == MLS_F16) MLS_COMBINE(_Float16);
  else MLS_COMBINE(__bf16);
#undef MLS_COMBINE
  return check_launch("mls_moe_combine");
}

}  // namespace

}  // namespace mls

using namespace mls;

extern "C" int mls_moe_combine(const void* x, int x_dt, int64_t ldx, int64_t x_rows, const void* w, int w_dt,
                               const int64_t* pos, int64_t T, int k, void* out, int64_t ldo,
                               int64_t D, mls_stream_t stream) {
  const char* fn = "mls_moe_combine";
  if (T < 0 || D < 0 || k < 1 || x_rows < 0) return fail(MLS_ERR_ARG, "%s: bad sizes T=%lld k=%d D=%lld", fn, (long long)T, k, (long long)D);
  if (!is_float_dt(x_dt) || !is_float_dt(w_dt)) return fail(MLS_ERR_ARG, "%s: bad dtype", fn);
  if (T == 0 || D == 0) return MLS_OK;
  if (!pos || !out || !w || (x_rows > 0 && !x)) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (ldx < D || ldo < D) return fail(MLS_ERR_ARG, "%s: bad leading dimension", fn);
  if (T > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "%s: T too large", fn);
  hipStream_t st = (hipStream_t)stream;
  if (x_dt == MLS_F32) return launch_combine<float>(x, ldx, x_rows, w, w_dt, pos, T, k, out, ldo, D, st);
  if (x_dt == MLS_F16) return launch_combine<_Float16>(x, ldx, x_rows, w, w_dt, pos, T, k, out, ldo, D, st);
  return launch_combine<__bf16>(x, ldx, x_rows, w, w_dt, pos, T, k, out, ldo, D, st);
}
