// fp32 activations for the 16-bit matrix cores: every fp32 x becomes two bf16 values,
//   hi = x with the low 16 bits of its encoding cleared (exact in bf16; truncation never
//        overflows to infinity),
//   lo = bf16(x - hi) (x - hi is exact in fp32 and below 2^-7 |x|, so lo keeps x to about
//        2^-16 of its magnitude; the rounding of lo is the only error of the split),
// and a weight-only GEMM of x becomes one of hi plus one of lo, both on the bf16 MFMA with
// fp32 accumulation (INT8 values and INT4 v - 8 are exact in bf16). Non-finite x: hi = x
// (a NaN kept a NaN), lo = 0, so an inf or NaN reaches the output as fp32 arithmetic would
// carry it (split_f32, mfma16.h; shared with the fp32 INT8 STE gradient in dgrad.hip).
//
// The split rows are a [split_rows(M)][K] bf16 matrix (mfma16.h): row R holds part
// (R >> 4) & 1 (0 hi, 1 lo) of row m = 16 (R >> 5) + (R & 15) of x, rows for m >= M are
// zero. One thread per 8 consecutive k of one row m writes both of its split rows.
#include "mfma16.h"

namespace mls {

namespace {

template <bool VEC>
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ x, int64_t ldx, int M, int K,
                                                         __bf16* __restrict__ x2, int Mp) {
  const int64_t pieces = K / 8;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= pieces * Mp) return;
  const int m = (int)(t / pieces), k0 = (int)(t % pieces) * 8;
  float v[8];
  if (m < M) {
    if constexpr (VEC) {
      const float4 a = *reinterpret_cast<const float4*>(x + (int64_t)m * ldx + k0);
      const float4 b = *reinterpret_cast<const float4*>(x + (int64_t)m * ldx + k0 + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = x[(int64_t)m * ldx + k0 + e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  }
  uint32_t h[4], l[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float h0, l0, h1, l1;
    split_f32(v[2 * q], h0, l0);
    split_f32(v[2 * q + 1], h1, l1);
    h[q] = pack2_bits((__bf16)h0, (__bf16)h1);  // exact: hi has no bits below bf16's
    l[q] = pack2_bits((__bf16)l0, (__bf16)l1);  // round to nearest even
  }
  *reinterpret_cast<uint4*>(x2 + (int64_t)split_row(m, 0) * K + k0) = make_uint4(h[0], h[1], h[2], h[3]);
  *reinterpret_cast<uint4*>(x2 + (int64_t)split_row(m, 1) * K + k0) = make_uint4(l[0], l[1], l[2], l[3]);
}

}  // namespace

int launch_split_rows(const float* x, int64_t ldx, int64_t M, int64_t K, void* x2, hipStream_t st) {
  if (K % 8 != 0 || !aligned(x2, 16)) return MLS_ERR_UNSUPPORTED;
  const int64_t Mp = cdiv(M, 16) * 16;
  const int64_t threads = Mp * (K / 8);
  if (Mp > 0x3FFFFFFF || K > 0x3FFFFFFF || cdiv(threads, 256) > 0x7FFFFFFF) return MLS_ERR_UNSUPPORTED;
  const bool vec = aligned(x, 16) && ldx % 4 == 0;
  const dim3 grid((unsigned)cdiv(threads, 256));
  if (vec)
    hipLaunchKernelGGL(split_rows_kernel<true>, grid, dim3(256), 0, st, x, ldx, (int)M, (int)K, (__bf16*)x2, (int)Mp);
  else
    hipLaunchKernelGGL(split_rows_kernel<false>, grid, dim3(256), 0, st, x, ldx, (int)M, (int)K, (__bf16*)x2, (int)Mp);
  return check_launch("split rows");
}

}  // namespace mls
