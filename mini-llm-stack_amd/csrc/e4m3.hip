// FP8 codec kernels. OCP E4M3 ("fn"): decode (reference semantics: NaN -> 0),
// dequantize (NaN stays NaN, times a scale) and the saturating encoder used by
// quantize_e4m3. Written from the OCP OFP8 definition: 1 sign, 4 exponent bits
// (bias 7), 3 mantissa bits, no infinities, S.1111.111 = NaN, max finite 448.
// E5M2: the encoder of FP8 training's gradients (train/fp8.py:50-52), from the OCP
// definition: 1 sign, 5 exponent bits (bias 15), 2 mantissa bits, infinities and NaNs
// at exponent 31, max finite 57344.
#include "common.h"

namespace mls {

// Exact value of an e4m3 byte. nan_to_zero selects the reference kernel's
// decode (kernels/fp8_matmul.py:37-47), which maps the NaN patterns to (signed) 0.
__device__ __forceinline__ float e4m3_value(uint32_t b, bool nan_to_zero) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float mag;
  if (e == 0) mag = (float)m * 0x1p-9f;                        // subnormal: m/8 * 2^-6
  else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));  // (1 + m/8) * 2^(e-7)
  if (e == 15u && m == 7u) mag = nan_to_zero ? 0.0f : __uint_as_float(0x7FC00000u);
  return (b & 0x80u) ? -mag : mag;
}

// The encoders below are straight-line (selects, no branches): the data decides between
// the subnormal and normal grids per element, and lanes of one wavefront disagree.

// e4m3 code of a finite magnitude 0 <= a <= 448, round to nearest, ties to even.
__device__ __forceinline__ uint32_t e4m3_code_of_mag(float a) {
  const uint32_t u = __float_as_uint(a);
  // a < 2^-6: the subnormal grid has step 2^-9 (code 8 is 2^-6)
  const uint32_t sub = (uint32_t)__builtin_rintf(a * 512.0f);
  // a >= 2^-6 (fp32 exponent field >= 121): round the fp32 pattern to its top 3 mantissa
  // bits, ties to even (add half - 1 plus the kept bit), and rebias the exponent
  // (127 -> 7); a carry out of the mantissa bumps the exponent.
  const uint32_t nrm = ((u + 0x7FFFFu + ((u >> 20) & 1u)) >> 20) - (120u << 3);
  return u < 0x3C800000u ? sub : nrm;
}

// Saturating encode of q (already divided by the scale): NaN -> 0x7F | sign,
// otherwise clamp |q| to 448 and round.
__device__ __forceinline__ uint32_t e4m3_encode(float q) {
  const uint32_t sign = (__float_as_uint(q) >> 24) & 0x80u;
  const uint32_t code = e4m3_code_of_mag(fminf(fabsf(q), 448.0f));
  return (__builtin_isnan(q) ? 0x7Fu : code) | sign;
}

// e5m2 code of a finite magnitude 0 <= a <= 57344, round to nearest, ties to even.
// e5m2: 1 sign, 5 exponent bits (bias 15), 2 mantissa bits; subnormals m/4 * 2^-14.
__device__ __forceinline__ uint32_t e5m2_code_of_mag(float a) {
  const uint32_t u = __float_as_uint(a);
  // a < 2^-14: the subnormal grid has step 2^-16 (code 4 is 2^-14)
  const uint32_t sub = (uint32_t)__builtin_rintf(a * 65536.0f);
  // a >= 2^-14 (fp32 exponent field >= 113): round to the top 2 mantissa bits, ties to
  // even, and rebias the exponent (127 -> 15); a mantissa carry bumps the exponent.
  const uint32_t nrm = ((u + 0xFFFFFu + ((u >> 21) & 1u)) >> 21) - (112u << 2);
  return u < 0x38800000u ? sub : nrm;
}

// The reference's e5m2 quantization of q (already divided by the scale): clamp to
// +-57344 (the largest finite e5m2), round; NaN -> 0x7F | sign.
__device__ __forceinline__ uint32_t e5m2_encode(float q) {
  const uint32_t sign = (__float_as_uint(q) >> 24) & 0x80u;
  const uint32_t code = e5m2_code_of_mag(fminf(fabsf(q), 57344.0f));
  return (__builtin_isnan(q) ? 0x7Fu : code) | sign;
}

// vec: bits/out are 16-byte aligned, so the bulk is read 16 bytes per thread.
__global__ void e4m3_decode_kernel(const uint8_t* __restrict__ bits, float* __restrict__ out,
                                   int64_t n, bool vec) {
  const int64_t nvec = vec ? n / 16 : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t v = tid; v < nvec; v += stride) {
    const uint4 w = reinterpret_cast<const uint4*>(bits)[v];
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float4* o = reinterpret_cast<float4*>(out + v * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 f;
      f.x = e4m3_value(words[q] & 0xFFu, true);
      f.y = e4m3_value((words[q] >> 8) & 0xFFu, true);
      f.z = e4m3_value((words[q] >> 16) & 0xFFu, true);
      f.w = e4m3_value(words[q] >> 24, true);
      o[q] = f;
    }
  }
  for (int64_t i = nvec * 16 + tid; i < n; i += stride) out[i] = e4m3_value(bits[i], true);
}

__global__ void e4m3_dequant_kernel(const uint8_t* __restrict__ bits, int64_t rows, int64_t cols,
                                    int64_t ldb, float scale, const float* __restrict__ sp,
                                    int64_t sstride, float* __restrict__ out, int64_t ldo) {
  const int64_t total = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / cols, c = i - r * cols;
    const float s = sp ? sp[r * sstride] : scale;
    out[r * ldo + c] = e4m3_value(bits[r * ldb + c], false) * s;
  }
}

template <typename T, bool E5M2>
__global__ void fp8_encode_kernel(const T* __restrict__ x, int64_t rows, int64_t cols, int64_t ldx,
                                  float scale, const float* __restrict__ sp, int64_t sstride,
                                  uint8_t* __restrict__ out, int64_t ldo) {
  const int64_t total = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / cols, c = i - r * cols;
    const float s = sp ? sp[r * sstride] : scale;
    const float q = to_f32(x[r * ldx + c]) / s;
    out[r * ldo + c] = (uint8_t)(E5M2 ? e5m2_encode(q) : e4m3_encode(q));
  }
}

// Vector path (cols % 4 == 0, 16-byte aligned rows for fp32, 8-byte for 16-bit inputs,
// 4-byte aligned output rows): 4 consecutive elements of one row per thread and step.
template <typename T, bool E5M2>
__global__ void fp8_encode_vec_kernel(const T* __restrict__ x, int64_t rows, int64_t cols, int64_t ldx,
                                      float scale, const float* __restrict__ sp, int64_t sstride,
                                      uint8_t* __restrict__ out, int64_t ldo) {
  const int64_t c4 = cols / 4, total = rows * c4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / c4, c = (i - r * c4) * 4;
    const float s = sp ? sp[r * sstride] : scale;
    float v[4];
    if constexpr (sizeof(T) == 4) {
      const float4 f = *reinterpret_cast<const float4*>(x + r * ldx + c);
      v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
      const uint2 h = *reinterpret_cast<const uint2*>(x + r * ldx + c);
      const T* e = reinterpret_cast<const T*>(&h);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = to_f32(e[k]);
    }
    uint32_t o = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) o |= (E5M2 ? e5m2_encode(v[k] / s) : e4m3_encode(v[k] / s)) << (8 * k);
    *reinterpret_cast<uint32_t*>(out + r * ldo + c) = o;
  }
}

// fp8 encode (e5m2 or e4m3) with a transposed copy: out[r][c] = out_t[c][r] = fp8(x[r][c] / s[r]).
// A 256-thread block encodes a 64 x 64 tile: each thread 16 consecutive elements of one
// row (written as one 16-byte store), the bytes also go to an LDS tile padded by 4 bytes
// per row, and after the barrier each thread writes 16 consecutive bytes of one row of
// the transpose. vec: full tile, 16-byte aligned input rows and output rows.
template <typename T, bool E5M2>
__global__ __launch_bounds__(256) void fp8_encode_t_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                            int64_t ldx, float scale, const float* __restrict__ sp,
                                                            int64_t sstride, uint8_t* __restrict__ out, int64_t ldo,
                                                            uint8_t* __restrict__ out_t, int64_t ldt,
                                                            int64_t col_tiles, bool vec) {
  constexpr int TS = 64, P = TS + 4;
  __shared__ uint8_t tile[TS * P];
  const int64_t bt = blockIdx.x;
  const int64_t r0 = (bt / col_tiles) * TS, c0 = (bt % col_tiles) * TS;
  const int tid = threadIdx.x;
  const int lr = tid >> 2, lc = (tid & 3) * 16;
  const int64_t r = r0 + lr;
  const bool full = vec && r0 + TS <= rows && c0 + TS <= cols;
  uint8_t b[16];
  if (full) {
    const float s = sp ? sp[r * sstride] : scale;
    float v[16];
    const T* src = x + r * ldx + c0 + lc;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = reinterpret_cast<const float4*>(src)[q];
        v[4 * q + 0] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint4 h = reinterpret_cast<const uint4*>(src)[q];
        const T* e = reinterpret_cast<const T*>(&h);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[8 * q + k] = to_f32(e[k]);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) b[i] = (uint8_t)(E5M2 ? e5m2_encode(v[i] / s) : e4m3_encode(v[i] / s));
    *reinterpret_cast<uint4*>(out + r * ldo + c0 + lc) = *reinterpret_cast<const uint4*>(b);
  } else {
    const float s = r < rows ? (sp ? sp[r * sstride] : scale) : 1.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t c = c0 + lc + i;
      b[i] = 0;
      if (r < rows && c < cols) {
        const float q = to_f32(x[r * ldx + c]) / s;
        b[i] = (uint8_t)(E5M2 ? e5m2_encode(q) : e4m3_encode(q));
        out[r * ldo + c] = b[i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) tile[lr * P + lc + i] = b[i];
  __syncthreads();
  // row c0 + lr of the transpose holds source column c0 + lr, bytes of source rows r0 + lc ..
  const int64_t dr = c0 + lr;
  if (full) {
    uint8_t t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = tile[(lc + i) * P + lr];
    *reinterpret_cast<uint4*>(out_t + dr * ldt + r0 + lc) = *reinterpret_cast<const uint4*>(t);
  } else if (dr < cols) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t dc = r0 + lc + i;
      if (dc < rows) out_t[dr * ldt + dc] = tile[(lc + i) * P + lr];
    }
  }
}

static int grid_for(int64_t work, int block) {
  int64_t g = cdiv(work, block);
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

}  // namespace mls

using namespace mls;

extern "C" int mls_e4m3_decode(const uint8_t* bits, float* out, int64_t n, mls_stream_t stream) {
  if (n < 0) return fail(MLS_ERR_ARG, "mls_e4m3_decode: n=%lld < 0", (long long)n);
  if (n == 0) return MLS_OK;
  if (!bits || !out) return fail(MLS_ERR_ARG, "mls_e4m3_decode: null pointer");
  const bool vec = aligned(bits, 16) && aligned(out, 16);
  const int block = 256;
  hipLaunchKernelGGL(e4m3_decode_kernel, dim3(grid_for(vec ? n / 16 + 1 : n, block)), dim3(block),
                     0, (hipStream_t)stream, bits, out, n, vec);
  return check_launch("mls_e4m3_decode");
}

extern "C" int mls_e4m3_dequantize(const uint8_t* bits, int64_t rows, int64_t cols, int64_t ldb,
                                   float scale, const float* scale_ptr, int64_t scale_stride,
                                   float* out, int64_t ldo, mls_stream_t stream) {
  if (rows < 0 || cols < 0) return fail(MLS_ERR_ARG, "mls_e4m3_dequantize: negative size");
  if (rows == 0 || cols == 0) return MLS_OK;
  if (!bits || !out) return fail(MLS_ERR_ARG, "mls_e4m3_dequantize: null pointer");
  if (ldb < cols || ldo < cols || scale_stride < 0)
    return fail(MLS_ERR_ARG, "mls_e4m3_dequantize: bad leading dimension or scale stride");
  const int block = 256;
  hipLaunchKernelGGL(e4m3_dequant_kernel, dim3(grid_for(rows * cols, block)), dim3(block), 0,
                     (hipStream_t)stream, bits, rows, cols, ldb, scale, scale_ptr, scale_stride,
                     out, ldo);
  return check_launch("mls_e4m3_dequantize");
}

template <bool E5M2>
static int fp8_encode(const char* fn, const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                      float scale, const float* scale_ptr, int64_t scale_stride, uint8_t* out, int64_t ldo,
                      mls_stream_t stream) {
  if (rows < 0 || cols < 0) return fail(MLS_ERR_ARG, "%s: negative size", fn);
  if (rows == 0 || cols == 0) return MLS_OK;
  if (!x || !out) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (!is_float_dt(x_dt)) return fail(MLS_ERR_ARG, "%s: bad x dtype %d", fn, x_dt);
  if (ldx < cols || ldo < cols || scale_stride < 0)
    return fail(MLS_ERR_ARG, "%s: bad leading dimension or scale stride", fn);
  const int block = 256;
  hipStream_t st = (hipStream_t)stream;
  const int xsz = dt_size(x_dt);
  if (cols % 4 == 0 && aligned(x, 4 * xsz) && (ldx * xsz) % (4 * xsz) == 0 && aligned(out, 4) && ldo % 4 == 0) {
    const dim3 grid(grid_for(rows * (cols / 4), block));
    if (x_dt == MLS_F32)
      hipLaunchKernelGGL((fp8_encode_vec_kernel<float, E5M2>), grid, dim3(block), 0, st, (const float*)x, rows,
                         cols, ldx, scale, scale_ptr, scale_stride, out, ldo);
    else if (x_dt == MLS_F16)
      hipLaunchKernelGGL((fp8_encode_vec_kernel<_Float16, E5M2>), grid, dim3(block), 0, st, (const _Float16*)x,
                         rows, cols, ldx, scale, scale_ptr, scale_stride, out, ldo);
    else
      hipLaunchKernelGGL((fp8_encode_vec_kernel<__bf16, E5M2>), grid, dim3(block), 0, st, (const __bf16*)x,
                         rows, cols, ldx, scale, scale_ptr, scale_stride, out, ldo);
    return check_launch(fn);
  }
  const dim3 grid(grid_for(rows * cols, block));
  if (x_dt == MLS_F32)
    hipLaunchKernelGGL((fp8_encode_kernel<float, E5M2>), grid, dim3(block), 0, st, (const float*)x, rows,
                       cols, ldx, scale, scale_ptr, scale_stride, out, ldo);
  else if (x_dt == MLS_F16)
    hipLaunchKernelGGL((fp8_encode_kernel<_Float16, E5M2>), grid, dim3(block), 0, st, (const _Float16*)x,
                       rows, cols, ldx, scale, scale_ptr, scale_stride, out, ldo);
  else
    hipLaunchKernelGGL((fp8_encode_kernel<__bf16, E5M2>), grid, dim3(block), 0, st, (const __bf16*)x, rows,
                       cols, ldx, scale, scale_ptr, scale_stride, out, ldo);
  return check_launch(fn);
}

extern "C" int mls_e4m3_encode(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                               float scale, const float* scale_ptr, int64_t scale_stride,
                               uint8_t* out, int64_t ldo, mls_stream_t stream) {
  return fp8_encode<false>("mls_e4m3_encode", x, x_dt, rows, cols, ldx, scale, scale_ptr, scale_stride, out,
                           ldo, stream);
}

extern "C" int mls_e5m2_encode(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                               float scale, const float* scale_ptr, int64_t scale_stride,
                               uint8_t* out, int64_t ldo, mls_stream_t stream) {
  return fp8_encode<true>("mls_e5m2_encode", x, x_dt, rows, cols, ldx, scale, scale_ptr, scale_stride, out,
                          ldo, stream);
}

template <bool E5M2>
static int fp8_encode_t(const char* fn, const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                        float scale, const float* scale_ptr, int64_t scale_stride, uint8_t* out, int64_t ldo,
                        uint8_t* out_t, int64_t ldt, mls_stream_t stream) {
  if (rows < 0 || cols < 0) return fail(MLS_ERR_ARG, "%s: negative size", fn);
  if (rows == 0 || cols == 0) return MLS_OK;
  if (!x || !out || !out_t) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (!is_float_dt(x_dt)) return fail(MLS_ERR_ARG, "%s: bad x dtype %d", fn, x_dt);
  if (ldx < cols || ldo < cols || ldt < rows || scale_stride < 0)
    return fail(MLS_ERR_ARG, "%s: bad leading dimension or scale stride", fn);
  const int64_t rt = cdiv(rows, 64), ct = cdiv(cols, 64);
  if (rt * ct > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "%s: too large", fn);
  const int xsz = dt_size(x_dt);
  const bool vec = aligned(x, 16) && (ldx * xsz) % 16 == 0 && aligned(out, 16) && ldo % 16 == 0 &&
                   aligned(out_t, 16) && ldt % 16 == 0;
  const dim3 grid((unsigned)(rt * ct));
  hipStream_t st = (hipStream_t)stream;
  if (x_dt == MLS_F32)
    hipLaunchKernelGGL((fp8_encode_t_kernel<float, E5M2>), grid, dim3(256), 0, st, (const float*)x, rows, cols, ldx,
                       scale, scale_ptr, scale_stride, out, ldo, out_t, ldt, ct, vec);
  else if (x_dt == MLS_F16)
    hipLaunchKernelGGL((fp8_encode_t_kernel<_Float16, E5M2>), grid, dim3(256), 0, st, (const _Float16*)x, rows, cols,
                       ldx, scale, scale_ptr, scale_stride, out, ldo, out_t, ldt, ct, vec);
  else
    hipLaunchKernelGGL((fp8_encode_t_kernel<__bf16, E5M2>), grid, dim3(256), 0, st, (const __bf16*)x, rows, cols,
                       ldx, scale, scale_ptr, scale_stride, out, ldo, out_t, ldt, ct, vec);
  return check_launch(fn);
}

extern "C" int mls_e5m2_encode_t(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                                 float scale, const float* scale_ptr, int64_t scale_stride,
                                 uint8_t* out, int64_t ldo, uint8_t* out_t, int64_t ldt, mls_stream_t stream) {
  return fp8_encode_t<true>("mls_e5m2_encode_t", x, x_dt, rows, cols, ldx, scale, scale_ptr, scale_stride, out, ldo,
                            out_t, ldt, stream);
}

extern "C" int mls_e4m3_encode_t(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                                 float scale, const float* scale_ptr, int64_t scale_stride,
                                 uint8_t* out, int64_t ldo, uint8_t* out_t, int64_t ldt, mls_stream_t stream) {
  return fp8_encode_t<false>("mls_e4m3_encode_t", x, x_dt, rows, cols, ldx, scale, scale_ptr, scale_stride, out, ldo,
                             out_t, ldt, stream);
}
