// Byte transpose dst[c][r] = src[r][c]: the materialised .t() of fp8 operands in FP8
// training's backward (train/fp8.py:92-94), which the K-contiguous GEMMs need.
//
// HBM-bound: each byte read once and written once. A 256-thread block moves a 64 x 64
// tile through LDS: each thread reads 16 consecutive bytes of one source row (one
// 16-byte load) and writes 16 consecutive bytes of one destination row, so both
// sides are coalesced. The LDS tile is padded by 4 bytes per row, which spreads a
// column walk over the 32 banks. Partial tiles at the edges take byte accesses.
#include "common.h"

namespace mls {

namespace {

__global__ __launch_bounds__(256) void transpose_u8_kernel(const uint8_t* __restrict__ src, int64_t rows,
                                                           int64_t cols, int64_t lds,
                                                           uint8_t* __restrict__ dst, int64_t ldd,
                                                           int64_t col_tiles, bool vec) {
  constexpr int T = 64, P = T + 4;
  __shared__ uint8_t tile[T * P];
  const int64_t bt = blockIdx.x;
  const int64_t r0 = (bt / col_tiles) * T, c0 = (bt % col_tiles) * T;
  const int tid = threadIdx.x;
  const int lr = tid >> 2, lc = (tid & 3) * 16;  // 64 rows x 4 sixteen-byte pieces
  const int64_t r = r0 + lr;
  const bool full = vec && r0 + T <= rows && c0 + T <= cols;
  if (full) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + r * lds + c0 + lc);
    const uint8_t* b = reinterpret_cast<const uint8_t*>(&v);
#pragma unroll
    for (int i = 0; i < 16; ++i) tile[lr * P + lc + i] = b[i];
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t c = c0 + lc + i;
      tile[lr * P + lc + i] = (r < rows && c < cols) ? src[r * lds + c] : 0;
    }
  }
  __syncthreads();
  // destination row c0 + lr holds source column c0 + lr, bytes for source rows r0 + lc ..
  const int64_t dr = c0 + lr;
  if (full) {
    uint8_t b[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) b[i] = tile[(lc + i) * P + lr];
    *reinterpret_cast<uint4*>(dst + dr * ldd + r0 + lc) = *reinterpret_cast<const uint4*>(b);
  } else if (dr < cols) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t dc = r0 + lc + i;
      if (dc < rows) dst[dr * ldd + dc] = tile[(lc + i) * P + lr];
    }
  }
}

}  // namespace

}  // namespace mls

using namespace mls;

extern "C" int mls_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, int64_t lds, uint8_t* dst,
                                int64_t ldd, mls_stream_t stream) {
  const char* fn = "mls_transpose_u8";
  if (rows < 0 || cols < 0) return fail(MLS_ERR_ARG, "%s: negative size", fn);
  if (rows == 0 || cols == 0) return MLS_OK;
  if (!src || !dst) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (lds < cols || ldd < rows) return fail(MLS_ERR_ARG, "%s: bad leading dimension", fn);
  const int64_t rt = cdiv(rows, 64), ct = cdiv(cols, 64);
  if (rt * ct > 0x7FFFFFFF) return fail(MLS_ERR_UNSUPPORTED, "%s: too large", fn);
  const bool vec = aligned(src, 16) && aligned(dst, 16) && lds % 16 == 0 && ldd % 16 == 0;
  hipLaunchKernelGGL(transpose_u8_kernel, dim3((unsigned)(rt * ct)), dim3(256), 0, (hipStream_t)stream, src,
                     rows, cols, lds, dst, ldd, ct, vec);
  return check_launch(fn);
}
