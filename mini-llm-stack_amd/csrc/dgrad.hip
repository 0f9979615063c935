// INT8 input gradient dx[M][K] = sum_n (dy[m][n] * s[n]) * wq[n][k]
// (kernels/dequant_matmul.py:103-132): the transpose-side GEMM of the INT8
// straight-through estimator. Reduction over N, which is the slow axis of wq.
//
// Two routes:
//  - matrix cores (mls_int8_dgrad_ws, 16-bit dy): the reference's own arithmetic, the
//    product (dy * s) rounded to dy's dtype (dequant_matmul.py:128) times the int8 weights
//    (exact in bf16 / fp16) on the 16-bit MFMA with fp32 accumulation. Three launches on
//    the caller's stream into a caller workspace: (1) ys = dy * s in dy's dtype, columns
//    padded with zeros to Np = N rounded up to 64, and a vector of K ones; (2) wt = wq^T
//    [K][Np] (mls_transpose_u8; its padding columns stay unwritten, and multiply only the
//    zeros of ys); (3) the INT8 weight-only GEMM dx = ys wt^T with unit row scales
//    (mls_int8_gemm), whose reduction axis is now contiguous in both operands.
//  - matrix cores with fp32 dy (M > 16): ys = dy * s in fp32, split into bf16 hi and lo rows
//    (mfma16.h), the same transpose, and the split-row GEMM adding both parts in fp32.
//  - VALU (mls_int8_dgrad, and fp32 dy with M <= 16): block tile 64 (m) x 64 (k), 256 threads, each
//    computing a 4 x 4 patch with fp32 FMAs from LDS tiles of 32 n, dy * s formed in fp32
//    (closer to the dequantize-then-fp32 oracle than the reference's rounding).
#include <algorithm>

#include "mfma16.h"

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

// ys[m][n] = T(dy[m][n] * s[n]) for n < N, 0 for N <= n < Np; ones[k] = 1 for k < K.
// One thread per 8 consecutive n of a row, consecutive threads on consecutive 16-byte
// pieces of a row (VEC: one 16-byte load of dy, 16- or 32-byte loads of the scales).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void dgrad_scale_kernel(const T* __restrict__ dy, int64_t lddy,
                                                          const void* __restrict__ s, int s_dt,
                                                          T* __restrict__ ys, int64_t Np, float* __restrict__ ones,
                                                          int M, int N, int K) {
  // 2-D grid: x over a row's 8-element pieces (the first row of blocks also writes the K
  // ones, grid-stride), y over rows (grid-stride)
  const int64_t per_row = Np / 8;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.y == 0)
    for (int64_t i = c; i < K; i += (int64_t)gridDim.x * 256) ones[i] = 1.0f;
  if (c >= per_row) return;
  const int n0 = (int)c * 8;
  // this thread's 8 scales (0 past N), once for all its rows
  float sv[8];
  if (VEC && n0 + 8 <= N) {
    if (s_dt == MLS_F16) {
      const uint4 h = *reinterpret_cast<const uint4*>((const _Float16*)s + n0);
      const _Float16* hv = reinterpret_cast<const _Float16*>(&h);
#pragma unroll
      for (int e = 0; e < 8; ++e) sv[e] = (float)hv[e];
    } else {
      const float4 a = *reinterpret_cast<const float4*>((const float*)s + n0);
      const float4 b = *reinterpret_cast<const float4*>((const float*)s + n0 + 4);
      sv[0] = a.x; sv[1] = a.y; sv[2] = a.z; sv[3] = a.w;
      sv[4] = b.x; sv[5] = b.y; sv[6] = b.z; sv[7] = b.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      sv[e] = n0 + e < N ? (s_dt == MLS_F16 ? (float)((const _Float16*)s)[n0 + e] : ((const float*)s)[n0 + e]) : 0.0f;
  }
  const int64_t ystep = gridDim.y;
  int64_t m = blockIdx.y;
  if (VEC && n0 + 8 <= N) {
    // RB rows at a time, every load issued before the first use: RB 16-byte loads in
    // flight per thread instead of one
    constexpr int RB = 4;
    for (; m + (RB - 1) * ystep < M; m += RB * ystep) {
      uint4 d[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) d[r] = *reinterpret_cast<const uint4*>(dy + (m + r * ystep) * lddy + n0);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const T* dv = reinterpret_cast<const T*>(&d[r]);
        uint32_t o[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
          o[h] = pack2_bits(from_f32<T>(to_f32(dv[2 * h]) * sv[2 * h]), from_f32<T>(to_f32(dv[2 * h + 1]) * sv[2 * h + 1]));
        *reinterpret_cast<uint4*>(ys + (m + r * ystep) * Np + n0) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  for (; m < M; m += ystep) {
    float v[8];
    if (VEC && n0 + 8 <= N) {  // one 16-byte load (rows 16-byte aligned: checked on the host)
      const uint4 d = *reinterpret_cast<const uint4*>(dy + m * lddy + n0);
      const T* dv = reinterpret_cast<const T*>(&d);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f32(dv[e]) * sv[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = n0 + e < N ? to_f32(dy[m * lddy + n0 + e]) * sv[e] : 0.0f;
    }
    uint32_t o[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) o[h] = pack2_bits(from_f32<T>(v[2 * h]), from_f32<T>(v[2 * h + 1]));
    *reinterpret_cast<uint4*>(ys + m * Np + n0) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// fp32 dy: the split rows (mfma16.h) of ys = dy * s, formed in fp32 (.to(dy.dtype) rounds
// nothing for fp32 dy, dequant_matmul.py:128): row m's hi and lo parts go to split rows
// split_row(m, 0 / 1), columns N .. Np - 1 and rows M .. Mp - 1 are zero. One thread per
// 8 consecutive n of one row; the first row of blocks also writes the K ones.
template <bool VEC>
__global__ __launch_bounds__(256) void dgrad_scale_split_kernel(const float* __restrict__ dy, int64_t lddy,
                                                                const void* __restrict__ s, int s_dt,
                                                                __bf16* __restrict__ ys, int64_t Np,
                                                                float* __restrict__ ones, int M, int Mp, int N,
                                                                int K) {
  const int64_t per_row = Np / 8;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.y == 0)
    for (int64_t i = c; i < K; i += (int64_t)gridDim.x * 256) ones[i] = 1.0f;
  if (c >= per_row) return;
  const int n0 = (int)c * 8;
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    sv[e] = n0 + e < N ? (s_dt == MLS_F16 ? (float)((const _Float16*)s)[n0 + e] : ((const float*)s)[n0 + e]) : 0.0f;
  for (int64_t m = blockIdx.y; m < Mp; m += gridDim.y) {
    float v[8];
    if (m >= M) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    } else if (VEC && n0 + 8 <= N) {
      const float4 a = *reinterpret_cast<const float4*>(dy + m * lddy + n0);
      const float4 b = *reinterpret_cast<const float4*>(dy + m * lddy + n0 + 4);
      v[0] = a.x * sv[0]; v[1] = a.y * sv[1]; v[2] = a.z * sv[2]; v[3] = a.w * sv[3];
      v[4] = b.x * sv[4]; v[5] = b.y * sv[5]; v[6] = b.z * sv[6]; v[7] = b.w * sv[7];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = n0 + e < N ? dy[m * lddy + n0 + e] * sv[e] : 0.0f;
    }
    uint32_t h[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float hv[2], lv[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) split_f32(v[2 * q + e], hv[e], lv[e]);
      h[q] = pack2_bits((__bf16)hv[0], (__bf16)hv[1]);
      l[q] = pack2_bits((__bf16)lv[0], (__bf16)lv[1]);
    }
    *reinterpret_cast<uint4*>(ys + (int64_t)split_row((int)m, 0) * Np + n0) = make_uint4(h[0], h[1], h[2], h[3]);
    *reinterpret_cast<uint4*>(ys + (int64_t)split_row((int)m, 1) * Np + n0) = make_uint4(l[0], l[1], l[2], l[3]);
  }
}

// Workspace layout of the matrix-core route (each part 256-byte aligned): ys (16-bit dy:
// M rows; fp32 dy: split_rows(M) bf16 rows), W_q^T, the ones.
struct DgradWs {
  int64_t Np, ys_off, wt_off, ones_off, bytes;
};
DgradWs dgrad_ws(int64_t M, int64_t N, int64_t K, int dy_dt) {
  DgradWs w;
  w.Np = cdiv(N, 64) * 64;
  const auto up = [](int64_t b) { return cdiv(b, 256) * 256; };
  w.ys_off = 0;
  w.wt_off = up((dy_dt == MLS_F32 ? split_rows(M) : M) * w.Np * 2);
  w.ones_off = w.wt_off + up(K * w.Np);
  w.bytes = w.ones_off + up(K * 4);
  return w;
}

// Shapes the matrix-core route takes: 16-bit dy, or fp32 dy with M > 16 (split rows), and
// the INT8 GEMM's 32-bit tile offsets.
bool dgrad_mfma_ok(int dy_dt, int64_t M, int64_t N, int64_t K) {
  static const bool split_env = env_int("MLS_SPLIT", 1) != 0;
  if (dy_dt == MLS_F32) {
    if (!split_env || M <= 16) return false;
  } else if (dy_dt != MLS_BF16 && dy_dt != MLS_F16) {
    return false;
  }
  const int64_t Np = cdiv(N, 64) * 64, rows = dy_dt == MLS_F32 ? split_rows(M) : M;
  return rows <= 0x3FFFFFFF && K <= 0x3FFFFFFF && Np * 2 * 256 < (1ll << 31) && rows * (Np / 8) < (1ll << 40);
}

}  // namespace mls

using namespace mls;

extern "C" int64_t mls_int8_dgrad_workspace(int64_t M, int64_t N, int64_t K, int dy_dt) {
  if (M <= 0 || N <= 0 || K <= 0 || !dgrad_mfma_ok(dy_dt, M, N, K)) return 0;
  return dgrad_ws(M, N, K, dy_dt).bytes;
}

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

extern "C" int mls_int8_dgrad_ws(const void* dy, int dy_dt, int64_t lddy, const int8_t* w, int64_t ldw,
                                 const void* s, int s_dt, void* dx, int dx_dt, int64_t lddx, int64_t M,
                                 int64_t N, int64_t K, void* workspace, int64_t ws_bytes,
                                 mls_stream_t stream) {
  const int64_t need = mls_int8_dgrad_workspace(M, N, K, dy_dt);
  // nothing to do, or the VALU route (fp32 dy with M <= 16, or an output the split GEMM's
  // 8-byte stores cannot take): no workspace needed
  if (need == 0 || (dy_dt == MLS_F32 && !aligned(dx, 8)))
    return mls_int8_dgrad(dy, dy_dt, lddy, w, ldw, s, s_dt, dx, dx_dt, lddx, M, N, K, stream);
  if (dx_dt != dy_dt)
    return fail(MLS_ERR_ARG, "mls_int8_dgrad_ws: dy/dx dtypes %d/%d (must match)", dy_dt, dx_dt);
  if (s_dt != MLS_F32 && s_dt != MLS_F16)
    return fail(MLS_ERR_ARG, "mls_int8_dgrad_ws: scale dtype %d (f32 or f16)", s_dt);
  if (!dy || !w || !s || !dx) return fail(MLS_ERR_ARG, "mls_int8_dgrad_ws: null pointer");
  if (lddy < N || ldw < K || lddx < K) return fail(MLS_ERR_ARG, "mls_int8_dgrad_ws: bad leading dimension");
  if (!workspace || ws_bytes < need || !aligned(workspace, 256))
    return fail(MLS_ERR_ARG, "mls_int8_dgrad_ws: workspace of %lld bytes at %p (need %lld, 256-byte aligned)",
                (long long)ws_bytes, workspace, (long long)need);
  const DgradWs L = dgrad_ws(M, N, K, dy_dt);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  void* ys = ws + L.ys_off;
  uint8_t* wt = ws + L.wt_off;
  float* ones = reinterpret_cast<float*>(ws + L.ones_off);
  hipStream_t st = (hipStream_t)stream;
  const int64_t gx = cdiv(L.Np / 8, 256);
  if (gx > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "mls_int8_dgrad_ws: shape too large");
  // about 8 rows per thread: the scales are loaded once for all of them
  const dim3 grid((unsigned)gx, (unsigned)std::min<int64_t>(cdiv(M, 8), 65535));
  // 16-byte accesses when dy's rows and the scale vector are 16-byte aligned
  const bool vec = aligned(dy, 16) && lddy % 8 == 0 && aligned(s, 16);
  if (dy_dt == MLS_F32) {
    const int64_t Mp = split_rows(M) / 2;
    const dim3 g2((unsigned)gx, (unsigned)std::min<int64_t>(cdiv(Mp, 8), 65535));
    const bool v4 = aligned(dy, 16) && lddy % 4 == 0;
    auto k = v4 ? dgrad_scale_split_kernel<true> : dgrad_scale_split_kernel<false>;
    hipLaunchKernelGGL(k, g2, dim3(256), 0, st, (const float*)dy, lddy, s, s_dt, (__bf16*)ys, L.Np, ones, (int)M,
                       (int)Mp, (int)N, (int)K);
    int rc = check_launch("mls_int8_dgrad_ws (scale, split rows)");
    if (rc != MLS_OK) return rc;
    rc = mls_transpose_u8(reinterpret_cast<const uint8_t*>(w), N, K, ldw, wt, L.Np, stream);
    if (rc != MLS_OK) return rc;
    WqArgs q{ys, MLS_BF16, L.Np, wt, L.Np, ones, MLS_F32, 1, 0, 0, dx, lddx, split_rows(M), K, L.Np, st};
    rc = launch_split_gemm(8, q, M);
    if (rc == MLS_ERR_UNSUPPORTED) return fail(MLS_ERR_HIP, "mls_int8_dgrad_ws: no split GEMM took the rows");
    if (rc != MLS_OK) return rc;
    return check_launch("mls_int8_dgrad_ws (split GEMM)");
  }
  if (dy_dt == MLS_F16) {
    auto k = vec ? dgrad_scale_kernel<_Float16, true> : dgrad_scale_kernel<_Float16, false>;
    hipLaunchKernelGGL(k, grid, dim3(256), 0, st, (const _Float16*)dy, lddy, s, s_dt, (_Float16*)ys, L.Np, ones,
                       (int)M, (int)N, (int)K);
  } else {
    auto k = vec ? dgrad_scale_kernel<__bf16, true> : dgrad_scale_kernel<__bf16, false>;
    hipLaunchKernelGGL(k, grid, dim3(256), 0, st, (const __bf16*)dy, lddy, s, s_dt, (__bf16*)ys, L.Np, ones,
                       (int)M, (int)N, (int)K);
  }
  int rc = check_launch("mls_int8_dgrad_ws (scale)");
  if (rc != MLS_OK) return rc;
  rc = mls_transpose_u8(reinterpret_cast<const uint8_t*>(w), N, K, ldw, wt, L.Np, stream);
  if (rc != MLS_OK) return rc;
  return mls_int8_gemm(ys, dy_dt, L.Np, reinterpret_cast<const int8_t*>(wt), L.Np, ones, MLS_F32, dx, dx_dt,
                       lddx, M, K, L.Np, stream);
}
