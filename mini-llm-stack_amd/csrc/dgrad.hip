// INT8 input gradient dx[M][K] = sum_n (dy[m][n] * s[n]) * wq[n][k]
// (kernels/dequant_matmul.py:103-132): the transpose-side GEMM of the INT8
// straight-through estimator. Reduction over N, which is the slow axis of wq.
//
// Block tile 64 (m) x 64 (k), 256 threads, each computing a 4 x 4 patch with
// fp32 FMAs from LDS tiles of 32 n: dy*s is formed in fp32 (the reference
// rounds it to dy's dtype first; fp32 is closer to the dequantize-then-fp32
// oracle) and int8 weights are exact in fp32.
#include "common.h"

namespace mls {

template <typename T>
__global__ __launch_bounds__(256) void int8_dgrad_kernel(const T* __restrict__ dy, int64_t lddy,
                                                         const int8_t* __restrict__ w, int64_t ldw,
                                                         const void* __restrict__ s, int s_dt,
                                                         T* __restrict__ dx, int64_t lddx, int M,
                                                         int N, int K) {
  constexpr int TMB = 64, TKB = 64, TNB = 32;
  __shared__ float ys[TNB][TMB + 1];  // [n][m]
  __shared__ float ws[TNB][TKB + 1];  // [n][k]
  const int m0 = blockIdx.y * TMB, k0 = blockIdx.x * TKB;
  const int tid = threadIdx.x, tm = tid / 16, tk = tid % 16;
  float acc[4][4] = {};
  for (int n0 = 0; n0 < N; n0 += TNB) {
    for (int e = tid; e < TNB * TMB; e += 256) {
      const int nn = e % TNB, mm = e / TNB;
      const int m = m0 + mm, n = n0 + nn;
      float v = 0.0f;
      if (m < M && n < N) {
        const float sn = s_dt == MLS_F16 ? (float)((const _Float16*)s)[n] : ((const float*)s)[n];
        v = to_f32(dy[(int64_t)m * lddy + n]) * sn;
      }
      ys[nn][mm] = v;
    }
    for (int e = tid; e < TNB * TKB; e += 256) {
      const int kk = e % TKB, nn = e / TKB;
      const int k = k0 + kk, n = n0 + nn;
      ws[nn][kk] = (k < K && n < N) ? (float)w[(int64_t)n * ldw + k] : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int nn = 0; nn < TNB; ++nn) {
      float yv[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) yv[i] = ys[nn][tm * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = ws[nn][tk * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(yv[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + tm * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + tk * 4 + j;
      if (k < K) dx[(int64_t)m * lddx + k] = from_f32<T>(acc[i][j]);
    }
  }
}

}  // namespace mls

using namespace mls;

extern "C" int mls_int8_dgrad(const void* dy, int dy_dt, int64_t lddy, const int8_t* w, int64_t ldw,
                              const void* s, int s_dt, void* dx, int dx_dt, int64_t lddx, int64_t M,
                              int64_t N, int64_t K, mls_stream_t stream) {
  if (M < 0 || N < 0 || K < 0) return fail(MLS_ERR_ARG, "mls_int8_dgrad: negative size");
  if (!is_float_dt(dy_dt) || dx_dt != dy_dt)
    return fail(MLS_ERR_ARG, "mls_int8_dgrad: dy/dx dtypes %d/%d (must match)", dy_dt, dx_dt);
  if (s_dt != MLS_F32 && s_dt != MLS_F16)
    return fail(MLS_ERR_ARG, "mls_int8_dgrad: scale dtype %d (f32 or f16)", s_dt);
  if (M == 0 || K == 0) return MLS_OK;
  if (!dy || !w || !s || !dx) return fail(MLS_ERR_ARG, "mls_int8_dgrad: null pointer");
  if (lddy < N || ldw < K || lddx < K)
    return fail(MLS_ERR_ARG, "mls_int8_dgrad: bad leading dimension");
  if (M > 0x7FFFFFFF || N > 0x7FFFFFFF || K > 0x7FFFFFFF || cdiv(M, 64) > 65535)
    return fail(MLS_ERR_UNSUPPORTED, "mls_int8_dgrad: shape too large");
  const dim3 grid((unsigned)cdiv(K, 64), (unsigned)cdiv(M, 64));
  hipStream_t st = (hipStream_t)stream;
  if (dy_dt == MLS_F32)
    hipLaunchKernelGGL(int8_dgrad_kernel<float>, grid, dim3(256), 0, st, (const float*)dy, lddy, w,
                       ldw, s, s_dt, (float*)dx, lddx, (int)M, (int)N, (int)K);
  else if (dy_dt == MLS_F16)
    hipLaunchKernelGGL(int8_dgrad_kernel<_Float16>, grid, dim3(256), 0, st, (const _Float16*)dy,
                       lddy, w, ldw, s, s_dt, (_Float16*)dx, lddx, (int)M, (int)N, (int)K);
  else
    hipLaunchKernelGGL(int8_dgrad_kernel<__bf16>, grid, dim3(256), 0, st, (const __bf16*)dy, lddy,
                       w, ldw, s, s_dt, (__bf16*)dx, lddx, (int)M, (int)N, (int)K);
  return check_launch("mls_int8_dgrad");
}
