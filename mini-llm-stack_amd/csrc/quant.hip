// Load-time weight quantizers for device tensors (serve/quantize.py:18-36):
// symmetric INT8 per output row and INT4 per group along K, packed two nibbles
// per byte (even k in the low nibble, stored value = q + 8). IEEE fp32
// division and round-half-to-even, so the codes match the reference's CPU path.
#include "common.h"

namespace mls {

// One 256-thread block per row n.
__global__ __launch_bounds__(256) void quant_int8_kernel(const float* __restrict__ w, int64_t K,
                                                         int64_t ldw, int8_t* __restrict__ wq,
                                                         int64_t ldq, float* __restrict__ scale) {
  const int64_t n = blockIdx.x;
  const float* row = w + n * ldw;
  float amax = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) amax = fmaxf(amax, fabsf(row[k]));
  amax = wave_max(amax);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(amax / 127.0f, 1e-8f);
  if (threadIdx.x == 0) scale[n] = s;
  int8_t* qrow = wq + n * ldq;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
    const float q = fminf(fmaxf(__builtin_rintf(row[k] / s), -127.0f), 127.0f);
    qrow[k] = (int8_t)(int)q;
  }
}

// One thread per (row, group).
__global__ void quant_int4_kernel(const float* __restrict__ w, int64_t N, int64_t K, int64_t ldw,
                                  int group, uint8_t* __restrict__ packed, int64_t ldp,
                                  float* __restrict__ scale) {
  const int64_t G = K / group;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * G) return;
  const int64_t n = t / G, g = t - n * G;
  const float* src = w + n * ldw + g * group;
  float amax = 0.0f;
  for (int i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(src[i]));
  const float s = fmaxf(amax / 7.0f, 1e-8f);
  scale[n * G + g] = s;
  uint8_t* dst = packed + n * ldp + g * (group / 2);
  for (int i = 0; i < group; i += 2) {
    const float q0 = fminf(fmaxf(__builtin_rintf(src[i] / s), -8.0f), 7.0f) + 8.0f;
    const float q1 = fminf(fmaxf(__builtin_rintf(src[i + 1] / s), -8.0f), 7.0f) + 8.0f;
    dst[i / 2] = (uint8_t)((unsigned)q0 | ((unsigned)q1 << 4));
  }
}

}  // namespace mls

using namespace mls;

extern "C" int mls_quantize_int8(const float* w, int64_t N, int64_t K, int64_t ldw, int8_t* wq,
                                 int64_t ldq, float* scale, mls_stream_t stream) {
  if (N < 0 || K < 1) return fail(MLS_ERR_ARG, "mls_quantize_int8: bad shape N=%lld K=%lld",
                                  (long long)N, (long long)K);
  if (N == 0) return MLS_OK;
  if (!w || !wq || !scale) return fail(MLS_ERR_ARG, "mls_quantize_int8: null pointer");
  if (ldw < K || ldq < K) return fail(MLS_ERR_ARG, "mls_quantize_int8: bad leading dimension");
  if (N > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "mls_quantize_int8: N too large");
  hipLaunchKernelGGL(quant_int8_kernel, dim3((unsigned)N), dim3(256), 0, (hipStream_t)stream, w, K,
                     ldw, wq, ldq, scale);
  return check_launch("mls_quantize_int8");
}

extern "C" int mls_quantize_int4(const float* w, int64_t N, int64_t K, int64_t ldw, int group,
                                 uint8_t* packed, int64_t ldp, float* scale, mls_stream_t stream) {
  if (N < 0 || K < 1 || group < 1)
    return fail(MLS_ERR_ARG, "mls_quantize_int4: bad shape N=%lld K=%lld group=%d", (long long)N,
                (long long)K, group);
  if (K % group != 0) return fail(MLS_ERR_ARG, "mls_quantize_int4: K %% group != 0");
  if (group % 2 != 0) return fail(MLS_ERR_ARG, "mls_quantize_int4: group must be even");
  if (N == 0) return MLS_OK;
  if (!w || !packed || !scale) return fail(MLS_ERR_ARG, "mls_quantize_int4: null pointer");
  if (ldw < K || ldp < K / 2) return fail(MLS_ERR_ARG, "mls_quantize_int4: bad leading dimension");
  const int64_t work = N * (K / group);
  hipLaunchKernelGGL(quant_int4_kernel, dim3((unsigned)cdiv(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, w, N, K, ldw, group, packed, ldp, scale);
  return check_launch("mls_quantize_int4");
}
