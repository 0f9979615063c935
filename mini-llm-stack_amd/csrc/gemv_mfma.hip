// Entry points of the skinny MFMA GEMM (gemv_mfma.h) and its INT4 kernels.
#include "gemv_mfma.h"

namespace mls {

// Shape checks shared by the 16-bit and the split-x launches.
static bool gemv_mfma_fits(int wbits, const WqArgs& p) {
  if (p.M < 1 || p.M > 16) return false;
  // INT4 steps of 128 k (groups a multiple of 128) or of 64 k (other multiples of 64)
  const bool s64 = wbits == 4 && p.group % 128 != 0;
  const int KB = wbits == 4 && !s64 ? 128 : 64;
  if (p.K % KB != 0) return false;
  if (wbits == 4 && p.group % 64 != 0) return false;
  if (!aligned(p.a, 16) || (p.lda * 2) % 16 != 0) return false;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0) return false;
  // 32-bit buffer offsets: 32 rows of x and a 32-row weight tile
  // (and the past-the-end x offset 0x7FFFFFF0 added to an x offset must not wrap)
  if (32 * p.lda * 2 >= (1ll << 31) || 32 * p.ldw >= (1ll << 31)) return false;
  return p.N <= 0x7FFFFFFF - 32 && p.K <= 0x3FFFFFFF;
}

int launch_gemv_mfma_split(int wbits, const WqArgs& q) {
  if (q.a_dt != MLS_BF16 || !gemv_mfma_fits(wbits, q)) return MLS_ERR_UNSUPPORTED;
  const bool s64 = wbits == 4 && q.group % 128 != 0;
  if (wbits == 4 && s64) return launch_st<4, __bf16, true, true>(q);
  if (wbits == 4) return launch_st<4, __bf16, false, true>(q);
  return launch_gemv_mfma_split_int8(q);
}

// fp32 x with 2 <= M <= 16: the split-x kernel reading the fp32 rows and splitting them in
// registers (XF), so no split pass runs. MLS_SKINNY_F32=0: the split pass and the split-row
// kernel instead (A/B runs).
int launch_gemv_mfma_f32(int wbits, const WqArgs& p) {
  static const bool on = env_int("MLS_SKINNY_F32", 1) != 0;
  if (!on || p.a_dt != MLS_F32 || p.M < 2 || p.M > 16) return MLS_ERR_UNSUPPORTED;
  const bool s64 = wbits == 4 && p.group % 128 != 0;
  const int KB = wbits == 4 && !s64 ? 128 : 64;
  if (p.K % KB != 0 || (wbits == 4 && p.group % 64 != 0)) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || p.lda % 4 != 0 || !aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.c, 16)) return MLS_ERR_UNSUPPORTED;
  // 32-bit buffer offsets: 16 rows of fp32 x and a 32-row weight tile (and the past-the-end
  // x offset 0x7FFFFFF0 added to an x offset must not wrap)
  if (16 * p.lda * 4 >= (1ll << 30) || 32 * p.ldw >= (1ll << 31)) return MLS_ERR_UNSUPPORTED;
  if (p.N > 0x7FFFFFFF - 32 || p.K > 0x3FFFFFFF) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && s64) return launch_st<4, __bf16, true, true, true>(p);
  if (wbits == 4) return launch_st<4, __bf16, false, true, true>(p);
  return launch_gemv_mfma_f32_int8(p);
}

int launch_gemv_mfma(int wbits, const WqArgs& p) {
  static const bool enabled = [] {
    const char* v = getenv("MLS_GEMV_MFMA");
    return !(v && v[0] == '0' && v[1] == 0);
  }();
  if (!enabled) return MLS_ERR_UNSUPPORTED;
  if (p.a_dt != MLS_BF16 && p.a_dt != MLS_F16) return MLS_ERR_UNSUPPORTED;
  if (p.M < 1 || p.M > 16) return MLS_ERR_UNSUPPORTED;
  // INT4 steps of 128 k (groups a multiple of 128) or of 64 k (other multiples of 64)
  const bool s64 = wbits == 4 && p.group % 128 != 0;
  const int KB = wbits == 4 && !s64 ? 128 : 64;
  if (p.K % KB != 0) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && p.group % 64 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.a, 16) || (p.lda * 2) % 16 != 0) return MLS_ERR_UNSUPPORTED;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0) return MLS_ERR_UNSUPPORTED;
  // 32-bit buffer offsets: 16 rows of x and a 32-row weight tile
  // (and the past-the-end x offset 0x7FFFFFF0 added to an x offset must not wrap)
  if (16 * p.lda * 2 >= (1ll << 31) || 32 * p.ldw >= (1ll << 31)) return MLS_ERR_UNSUPPORTED;
  if (p.N > 0x7FFFFFFF - 32 || p.K > 0x3FFFFFFF) return MLS_ERR_UNSUPPORTED;
  if (wbits == 4 && s64) return p.a_dt == MLS_BF16 ? launch_st<4, __bf16, true>(p) : launch_st<4, _Float16, true>(p);
  if (wbits == 4) return p.a_dt == MLS_BF16 ? launch_st<4, __bf16>(p) : launch_st<4, _Float16>(p);
  return launch_gemv_mfma_int8(p);
}

}  // namespace mls
