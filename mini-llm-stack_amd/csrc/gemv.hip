// Decode-shaped weight-only GEMM (small M): the HBM-bound family.
//
// Each wavefront owns R output columns n (weight rows) over the whole K. Lane l
// owns 16-byte weight chunks c = l + 64 j (j < CPL) of every one of its rows, so
// one load instruction covers 1 KiB of a row contiguously, and all R*CPL loads
// of a lane are issued before any arithmetic. The lane's slice of x (the same
// k range for every row) is loaded once and kept in registers, already laid out
// for the dot products, then reused across the R rows.
//
// Dequantization is folded into the dot products: a 16-byte INT4 chunk (32 k)
// lies inside one scale group, so  sum_k x_k (v_k - 8) s_g = s_g (sum_k x_k v'_k
// - off * sum_k x_k)  where v'_k = v_k + bias is produced by OR-ing the nibble into
// the mantissa of a 16-bit float constant (bf16 128.0 / fp16 1024.0): one
// v_and_or per two weights and one v_dot2 per two products. fp32 activations use
// exact byte->float converts and FMAs. INT8 uses u = q ^ 0x80 = q + 128 bytes.
// Each lane's partial sums are reduced across the wavefront at the end.
#include "wq.h"

namespace mls {

__device__ __forceinline__ float load_scale(const void* s, int s_dt, int64_t i) {
  return s_dt == MLS_F16 ? (float)((const _Float16*)s)[i] : ((const float*)s)[i];
}

template <typename AT> struct Half16;

template <> struct Half16<__bf16> {
  static constexpr uint32_t MAGIC4 = 0x43004300u;  // bf16 128.0 in both halves
  static constexpr float OFF4 = 136.0f;            // 128 + 8
  static constexpr uint32_t ONE2 = 0x3F803F80u;    // bf16 (1.0, 1.0)
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  // exact for the integers 0..255 this is used on
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <> struct Half16<_Float16> {
  static constexpr uint32_t MAGIC4 = 0x64006400u;  // fp16 1024.0 in both halves
  static constexpr float OFF4 = 1032.0f;           // 1024 + 8
  static constexpr uint32_t ONE2 = 0x3C003C00u;    // fp16 (1.0, 1.0)
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  }
};

__device__ __forceinline__ float ub0(uint32_t v) { return (float)(v & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t v) { return (float)(v >> 24); }

template <int WBITS, typename AT>
struct XSlot {
  static constexpr bool F32 = sizeof(AT) == 4;
  static constexpr int KC = WBITS == 4 ? 32 : 16;    // k per 16-byte weight chunk
  static constexpr int NV = F32 ? KC : KC / 2;       // registers per chunk of x
};

// Loads the lane's x values for chunk c of row m (zeros when out of range) into
// xr[NV] in the layout the dot products expect, and returns their sum.
template <int WBITS, typename AT>
__device__ __forceinline__ float load_x_chunk(const AT* __restrict__ xrow, bool valid, int c,
                                              uint32_t* xr) {
  using S = XSlot<WBITS, AT>;
  constexpr int KC = S::KC;
  if constexpr (S::F32) {
    float sum = 0.0f;
    if (valid) {
      const float4* src = reinterpret_cast<const float4*>(xrow + (int64_t)c * KC);
#pragma unroll
      for (int q = 0; q < KC / 4; ++q) {
        const float4 v = src[q];
        xr[4 * q + 0] = __float_as_uint(v.x);
        xr[4 * q + 1] = __float_as_uint(v.y);
        xr[4 * q + 2] = __float_as_uint(v.z);
        xr[4 * q + 3] = __float_as_uint(v.w);
        sum += (v.x + v.y) + (v.z + v.w);
      }
    } else {
#pragma unroll
      for (int q = 0; q < KC; ++q) xr[q] = 0u;
    }
    return sum;
  } else {
    using H = Half16<AT>;
    uint32_t d[KC / 2];
    if (valid) {
      const uint4* src = reinterpret_cast<const uint4*>(xrow + (int64_t)c * KC);
#pragma unroll
      for (int q = 0; q < KC / 8; ++q) {
        const uint4 v = src[q];
        d[4 * q + 0] = v.x;
        d[4 * q + 1] = v.y;
        d[4 * q + 2] = v.z;
        d[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < KC / 2; ++q) d[q] = 0u;
    }
    if constexpr (WBITS == 4) {
      // sub-block b holds k 8b..8b+7 as pairs (x0,x1)(x2,x3)(x4,x5)(x6,x7); the
      // nibble unpack yields weights for (k0,k4)(k1,k5)(k2,k6)(k3,k7).
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        xr[4 * b + 0] = __builtin_amdgcn_perm(d[4 * b + 2], d[4 * b + 0], 0x05040100u);
        xr[4 * b + 1] = __builtin_amdgcn_perm(d[4 * b + 2], d[4 * b + 0], 0x07060302u);
        xr[4 * b + 2] = __builtin_amdgcn_perm(d[4 * b + 3], d[4 * b + 1], 0x05040100u);
        xr[4 * b + 3] = __builtin_amdgcn_perm(d[4 * b + 3], d[4 * b + 1], 0x07060302u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < KC / 2; ++q) xr[q] = d[q];
    }
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < S::NV; ++q) sum = H::dot2(xr[q], H::ONE2, sum);
    return sum;
  }
}

// sum_k x_k * u_k over one 16-byte weight chunk, where u_k is the biased code
// (INT4: nibble + bias of the 16-bit path, or the raw nibble for fp32; INT8: q + 128).
template <int WBITS, typename AT>
__device__ __forceinline__ float chunk_dot(const uint4 wq, const uint32_t* xr) {
  using S = XSlot<WBITS, AT>;
  const uint32_t q[4] = {wq.x, wq.y, wq.z, wq.w};
  float acc = 0.0f;
  if constexpr (WBITS == 4) {
    if constexpr (S::F32) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t lo = q[b] & 0x0F0F0F0Fu, hi = (q[b] >> 4) & 0x0F0F0F0Fu;
        const float* x = reinterpret_cast<const float*>(xr) + 8 * b;
        acc = fmaf(ub0(lo), x[0], acc);
        acc = fmaf(ub0(hi), x[1], acc);
        acc = fmaf(ub1(lo), x[2], acc);
        acc = fmaf(ub1(hi), x[3], acc);
        acc = fmaf(ub2(lo), x[4], acc);
        acc = fmaf(ub2(hi), x[5], acc);
        acc = fmaf(ub3(lo), x[6], acc);
        acc = fmaf(ub3(hi), x[7], acc);
      }
    } else {
      using H = Half16<AT>;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t p0 = (q[b] & 0x000F000Fu) | H::MAGIC4;
        const uint32_t p1 = ((q[b] >> 4) & 0x000F000Fu) | H::MAGIC4;
        const uint32_t p2 = ((q[b] >> 8) & 0x000F000Fu) | H::MAGIC4;
        const uint32_t p3 = ((q[b] >> 12) & 0x000F000Fu) | H::MAGIC4;
        acc = H::dot2(p0, xr[4 * b + 0], acc);
        acc = H::dot2(p1, xr[4 * b + 1], acc);
        acc = H::dot2(p2, xr[4 * b + 2], acc);
        acc = H::dot2(p3, xr[4 * b + 3], acc);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t u = q[t] ^ 0x80808080u;  // signed int8 -> q + 128
      if constexpr (S::F32) {
        const float* x = reinterpret_cast<const float*>(xr) + 4 * t;
        acc = fmaf(ub0(u), x[0], acc);
        acc = fmaf(ub1(u), x[1], acc);
        acc = fmaf(ub2(u), x[2], acc);
        acc = fmaf(ub3(u), x[3], acc);
      } else {
        using H = Half16<AT>;
        acc = H::dot2(H::pack2(ub0(u), ub1(u)), xr[2 * t + 0], acc);
        acc = H::dot2(H::pack2(ub2(u), ub3(u)), xr[2 * t + 1], acc);
      }
    }
  }
  return acc;
}

template <int WBITS, typename AT>
constexpr float code_offset() {
  if constexpr (WBITS == 8) return 128.0f;
  else if constexpr (sizeof(AT) == 4) return 8.0f;
  else return Half16<AT>::OFF4;
}

template <int WBITS, typename AT, int MT, int CPL, int R>
__global__ __launch_bounds__(256) void gemv_wq_kernel(
    const AT* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ w, int64_t ldw,
    const void* __restrict__ s, int s_dt, int64_t ld_sn, int64_t ld_sg, int group,
    AT* __restrict__ y, int64_t ldy, int M, int N, int K) {
  using S = XSlot<WBITS, AT>;
  constexpr int KC = S::KC, NV = S::NV;
  constexpr float OFF = code_offset<WBITS, AT>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunks = K / KC;
  const int m0 = blockIdx.y * MT;
  const int n0 = (blockIdx.x * 4 + wave) * R;

  // 1. every weight chunk (and INT4 group scale) of this lane, issued up front
  uint4 wv[R][CPL];
  float sc[R][CPL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = n0 + r;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      const bool ok = n < N && c < nchunks;
      wv[r][j] = ok ? reinterpret_cast<const uint4*>(w + (int64_t)n * ldw)[c] : make_uint4(0, 0, 0, 0);
      if constexpr (WBITS == 4)
        sc[r][j] = ok ? load_scale(s, s_dt, (int64_t)n * ld_sn + (int64_t)((c * KC) / group) * ld_sg)
                      : 0.0f;
    }
  }

  // 2. the lane's x slice for MT rows
  uint32_t xr[MT][CPL][NV];
  float osx[MT][CPL];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const int m = m0 + mi;
    const AT* xrow = x + (int64_t)(m < M ? m : 0) * ldx;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      osx[mi][j] = OFF * load_x_chunk<WBITS, AT>(xrow, m < M && c < nchunks, c, xr[mi][j]);
    }
  }

  // 3. dot products
  float part[MT][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) part[mi][r] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) {
        const float d = chunk_dot<WBITS, AT>(wv[r][j], xr[mi][j]) - osx[mi][j];
        if constexpr (WBITS == 4) part[mi][r] = fmaf(sc[r][j], d, part[mi][r]);
        else part[mi][r] += d;
      }
    }
  }

  // 4. reduce across the wavefront and store
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = n0 + r;
    float sn = 1.0f;
    if constexpr (WBITS == 8) sn = n < N ? load_scale(s, s_dt, n) : 0.0f;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      const float v = wave_sum(part[mi][r]);
      const int m = m0 + mi;
      if (lane == 0 && n < N && m < M) y[(int64_t)m * ldy + n] = from_f32<AT>(v * sn);
    }
  }
}

template <int WBITS, typename AT, int MT, int CPL>
static void launch_one(const WqArgs& p) {
  constexpr int R = CPL >= 8 ? 1 : 8 / CPL;
  const dim3 grid((unsigned)cdiv(p.N, 4 * R), (unsigned)cdiv(p.M, MT));
  hipLaunchKernelGGL((gemv_wq_kernel<WBITS, AT, MT, CPL, R>), grid, dim3(256), 0, p.stream,
                     (const AT*)p.a, p.lda, p.w, p.ldw, p.s, p.s_dt, p.ld_sn, p.ld_sg, p.group,
                     (AT*)p.c, p.ldc, (int)p.M, (int)p.N, (int)p.K);
}

// Picks MT (rows of x per block) for a given CPL so that the x slice fits in
// 128 registers: MT * CPL * NV <= 128.
template <int WBITS, typename AT, int CPL>
static int dispatch_mt(const WqArgs& p) {
  constexpr int NV = XSlot<WBITS, AT>::NV;
  constexpr int MAXMT = 128 / (CPL * NV);
  if constexpr (MAXMT < 1) {
    return MLS_ERR_UNSUPPORTED;
  } else {
    if (p.M == 1 || MAXMT < 2) launch_one<WBITS, AT, 1, CPL>(p);
    else if (p.M == 2 || MAXMT < 4) launch_one<WBITS, AT, (MAXMT >= 2 ? 2 : 1), CPL>(p);
    else launch_one<WBITS, AT, (MAXMT >= 4 ? 4 : 1), CPL>(p);
    return MLS_OK;
  }
}

template <int WBITS, typename AT>
static int dispatch_cpl(const WqArgs& p) {
  constexpr int KC = XSlot<WBITS, AT>::KC;
  const int64_t cpl = cdiv(p.K / KC, 64);
  if (cpl <= 1) return dispatch_mt<WBITS, AT, 1>(p);
  if (cpl <= 2) return dispatch_mt<WBITS, AT, 2>(p);
  if (cpl <= 4) return dispatch_mt<WBITS, AT, 4>(p);
  if (cpl <= 8) return dispatch_mt<WBITS, AT, 8>(p);
  if (cpl <= 16) return dispatch_mt<WBITS, AT, 16>(p);
  return MLS_ERR_UNSUPPORTED;
}

int launch_gemv_wq(int wbits, const WqArgs& p) {
  const int KC = wbits == 4 ? 32 : 16;
  const int esz = dt_size(p.a_dt);
  if (p.K % KC != 0) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && (p.group % KC != 0)) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || (p.lda * esz) % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (p.N > 0x7FFFFFFF / 2 || p.M > 4 * 65535) return MLS_ERR_UNSUPPORTED;  // grid.y = M / MT
  if (wbits == 4) {
    if (p.a_dt == MLS_F32) return dispatch_cpl<4, float>(p);
    if (p.a_dt == MLS_F16) return dispatch_cpl<4, _Float16>(p);
    return dispatch_cpl<4, __bf16>(p);
  }
  if (p.a_dt == MLS_F32) return dispatch_cpl<8, float>(p);
  if (p.a_dt == MLS_F16) return dispatch_cpl<8, _Float16>(p);
  return dispatch_cpl<8, __bf16>(p);
}

// ------------------------------------------------------------------ generic path

template <int WBITS, typename AT>
__global__ void gemm_wq_generic_kernel(const AT* __restrict__ x, int64_t ldx,
                                       const uint8_t* __restrict__ w, int64_t ldw,
                                       const void* __restrict__ s, int s_dt, int64_t ld_sn,
                                       int64_t ld_sg, int group, AT* __restrict__ y, int64_t ldy,
                                       int64_t M, int64_t N, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * N) return;
  const int64_t m = t / N, n = t - m * N;
  const AT* xr = x + m * ldx;
  const uint8_t* wr = w + n * ldw;
  float acc = 0.0f;
  if constexpr (WBITS == 8) {
    for (int64_t k = 0; k < K; ++k) acc = fmaf(to_f32(xr[k]), (float)(int8_t)wr[k], acc);
    acc *= load_scale(s, s_dt, n);
  } else {
    for (int64_t k = 0; k < K; ++k) {
      const uint32_t byte = wr[k >> 1];
      const uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 15u);
      const float wk = ((float)nib - 8.0f) * load_scale(s, s_dt, n * ld_sn + (k / group) * ld_sg);
      acc = fmaf(to_f32(xr[k]), wk, acc);
    }
  }
  y[m * ldy + n] = from_f32<AT>(acc);
}

int launch_gemm_wq_generic(int wbits, const WqArgs& p) {
  const int64_t work = p.M * p.N;
  const dim3 grid((unsigned)cdiv(work, 256));
#define MLS_GENERIC(WB, T)                                                                        \
  hipLaunchKernelGGL((gemm_wq_generic_kernel<WB, T>), grid, dim3(256), 0, p.stream,              \
                     (const T*)p.a, p.lda, p.w, p.ldw, p.s, p.s_dt, p.ld_sn, p.ld_sg, p.group,    \
                     (T*)p.c, p.ldc, p.M, p.N, p.K)
  if (wbits == 4) {
    if (p.a_dt == MLS_F32) MLS_GENERIC(4, float);
    else if (p.a_dt == MLS_F16) MLS_GENERIC(4, _Float16);
    else MLS_GENERIC(4, __bf16);
  } else {
    if (p.a_dt == MLS_F32) MLS_GENERIC(8, float);
    else if (p.a_dt == MLS_F16) MLS_GENERIC(8, _Float16);
    else MLS_GENERIC(8, __bf16);
  }
#undef MLS_GENERIC
  return MLS_OK;
}

}  // namespace mls
