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

// INT8, vector path: one 256-thread block per row, 4 consecutive k per lane and step
// (16-byte loads, 4-byte stores); the row is read twice (amax, then codes), the
// second time from L2.
__global__ __launch_bounds__(256) void quant_int8_vec_kernel(const float* __restrict__ w, int64_t K,
                                                             int64_t ldw, int8_t* __restrict__ wq,
                                                             int64_t ldq, float* __restrict__ scale) {
  const int64_t n = blockIdx.x;
  const float4* row = reinterpret_cast<const float4*>(w + n * ldw);
  const int64_t K4 = K / 4;
  float amax = 0.0f;
  for (int64_t k = threadIdx.x; k < K4; k += blockDim.x) {
    const float4 v = row[k];
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  amax = wave_max(amax);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(amax / 127.0f, 1e-8f);
  if (threadIdx.x == 0) scale[n] = s;
  uint32_t* qrow = reinterpret_cast<uint32_t*>(wq + n * ldq);
  for (int64_t k = threadIdx.x; k < K4; k += blockDim.x) {
    const float4 v = row[k];
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint32_t o = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float q = fminf(fmaxf(__builtin_rintf(e[i] / s), -127.0f), 127.0f);
      o |= ((uint32_t)(int)q & 0xFFu) << (8 * i);
    }
    qrow[k] = o;
  }
}

// INT4, vector path for power-of-two groups of 8 .. 512: one wavefront per (row, span of
// 512 k), 8 consecutive k per lane (two 16-byte loads, one 4-byte store of 8 nibbles);
// a group is GL = group / 8 adjacent lanes, whose amax meets by DPP moves.
template <int GL>
__global__ __launch_bounds__(256) void quant_int4_vec_kernel(const float* __restrict__ w, int64_t N, int64_t K,
                                                             int64_t ldw, uint8_t* __restrict__ packed,
                                                             int64_t ldp, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t spans = (K + 511) / 512;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= N * spans) return;
  const int64_t n = wid / spans;
  const int64_t k0 = (wid - n * spans) * 512 + lane * 8;
  const bool on = k0 < K;  // K % 8 == 0, and a group never straddles the span end
  float e[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (on) {
    const float4* src = reinterpret_cast<const float4*>(w + n * ldw + k0);
    const float4 a = src[0], b = src[1];
    e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w;
    e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(e[i]));
  amax = lane_group_max<GL>(amax);
  if (!on) return;
  const float s = fmaxf(amax / 7.0f, 1e-8f);
  const int64_t G = K / (8 * GL);
  if ((lane & (GL - 1)) == 0) scale[n * G + k0 / (8 * GL)] = s;
  uint32_t o = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q = fminf(fmaxf(__builtin_rintf(e[i] / s), -8.0f), 7.0f) + 8.0f;
    o |= (uint32_t)q << (4 * i);  // k0 + i: even i in the low nibble of byte i / 2
  }
  *reinterpret_cast<uint32_t*>(packed + n * ldp + k0 / 2) = o;
}

// Generic INT4 path: one thread per (row, group).
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
  if (K % 4 == 0 && ldw % 4 == 0 && ldq % 4 == 0 && aligned(w, 16) && aligned(wq, 4))
    hipLaunchKernelGGL(quant_int8_vec_kernel, dim3((unsigned)N), dim3(256), 0, (hipStream_t)stream, w, K,
                       ldw, wq, ldq, scale);
  else
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
  const bool pow2 = group >= 8 && group <= 512 && (group & (group - 1)) == 0;
  if (pow2 && ldw % 4 == 0 && ldp % 4 == 0 && aligned(w, 16) && aligned(packed, 4)) {
    const int64_t waves = N * cdiv(K, 512);
    if (cdiv(waves, 4) > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "mls_quantize_int4: too large");
    const dim3 grid((unsigned)cdiv(waves, 4)), block(256);
    hipStream_t st = (hipStream_t)stream;
#define MLS_Q4(GL) hipLaunchKernelGGL(quant_int4_vec_kernel<GL>, grid, block, 0, st, w, N, K, ldw, packed, ldp, scale)
    switch (group / 8) {
      case 1: MLS_Q4(1); break;
      case 2: MLS_Q4(2); break;
      case 4: MLS_Q4(4); break;
      case 8: MLS_Q4(8); break;
      case 16: MLS_Q4(16); break;
      case 32: MLS_Q4(32); break;
      default: MLS_Q4(64); break;
    }
#undef MLS_Q4
    return check_launch("mls_quantize_int4");
  }
  const int64_t work = N * (K / group);
  hipLaunchKernelGGL(quant_int4_kernel, dim3((unsigned)cdiv(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, w, N, K, ldw, group, packed, ldp, scale);
  return check_launch("mls_quantize_int4");
}
