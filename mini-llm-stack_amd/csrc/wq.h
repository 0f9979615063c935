// Internal launchers of the weight-only (INT8 / INT4) GEMM family.
#pragma once

#include "common.h"

namespace mls {

// Arguments of one weight-only GEMM c[M][N] = a[M][K] . dequant(w)[N][K]^T.
struct WqArgs {
  const void* a;
  int a_dt;
  int64_t lda;
  const uint8_t* w;  // int8 [N][ldw] or packed int4 [N][ldw]
  int64_t ldw;
  const void* s;
  int s_dt;
  int64_t ld_sn, ld_sg;  // scale strides (INT8: ld_sn = 1, ld_sg = 0)
  int group;             // INT4 group (INT8: 0)
  void* c;
  int64_t ldc;
  int64_t M, N, K;
  hipStream_t stream;
};

// VALU decode GEMV for small M (x kept in registers). Returns MLS_ERR_UNSUPPORTED
// when the shape or alignment is outside its fast path.
int launch_gemv_wq(int wbits, const WqArgs& p);

// M = 2 with 16-bit activations on the M = 1 GEMV's layout (x of both rows in LDS, each
// weight chunk widened once for both). MLS_ERR_UNSUPPORTED outside its fast path.
int launch_gemv_rows(int wbits, const WqArgs& p);

// MFMA skinny GEMM for M <= 16 and 16-bit activations (weights read once for all M).
// MLS_ERR_UNSUPPORTED outside its fast path.
int launch_gemv_mfma(int wbits, const WqArgs& p);
// The same for fp32 x, 2 <= M <= 16: x read in fp32 and split into bf16 hi + lo parts in
// registers; fp32 output. MLS_ERR_UNSUPPORTED outside its fast path.
int launch_gemv_mfma_f32(int wbits, const WqArgs& p);

// Small / medium GEMM for 16-bit activations (MFMA operands straight into registers, K
// split over a block's wavefronts). MLS_ERR_UNSUPPORTED outside its fast path.
int launch_gemm_small(int wbits, const WqArgs& p);

// MFMA tiled GEMM for 16-bit activations. MLS_ERR_UNSUPPORTED outside its fast path.
int launch_gemm_wq_mfma(int wbits, const WqArgs& p);

// Any shape, any dtype: one thread per output element.
int launch_gemm_wq_generic(int wbits, const WqArgs& p);

// fp32 activations on the 16-bit matrix cores (split.hip, mfma16.h): p.a holds p.M split
// rows (bf16 hi and lo parts of m_out rows of x, p.M = split_rows(m_out)); the output is
// fp32 [m_out][ldc]. MLS_ERR_UNSUPPORTED outside the kernels' fast paths.
int launch_gemm_small_split(int wbits, const WqArgs& p, int64_t m_out);
// The skinny MFMA GEMV on split rows of M <= 16 rows of x (hi parts in rows 0..15, lo parts
// in rows 16..31 of p.a; p.M = the rows of x), fp32 output.
int launch_gemv_mfma_split(int wbits, const WqArgs& p);
int launch_gemm_wq_mfma_split(int wbits, const WqArgs& p, int64_t m_out);
// x fp32 [M][ldx] -> split rows [split_rows(M)][K] bf16 (zeros for rows past M).
int launch_split_rows(const float* x, int64_t ldx, int64_t M, int64_t K, void* x2, hipStream_t st);
// The GEMM of split rows q.a ([q.M][q.lda] bf16, q.M = split_rows(m_out)) into fp32 q.c:
// the medium GEMM where the engine would have few tiles, else the engine.
int launch_split_gemm(int wbits, const WqArgs& q, int64_t m_out);

// Per-expert INT4 GEMM over expert-sorted row segments (MFMA).
struct GroupedArgs {
  WqArgs base;            // base.M = total rows; base.w/base.s point at expert 0
  const int32_t* seg_off; // device [E+1]
  int E;
  int64_t w_estride;      // bytes between experts' packed weights
  int64_t s_estride;      // elements between experts' scales
  const int32_t* a_rows = nullptr;  // device [M_total]: sorted row m is row a_rows[m] of a
  int64_t a_src_rows = 0;           // rows of a when a_rows is set
};
int launch_grouped_int4(const GroupedArgs& p);
// The gate/up pair of a SwiGLU expert MLP over expert-sorted segments: base.w / base.s
// are the gate matrices, wu / su the up matrices (same strides); base.c receives
// silu(a Wg^T) * (a Wu^T).
int launch_grouped_gate_up(const GroupedArgs& p, const uint8_t* wu, const void* su);
// `splits` fp32 partial products over equal K ranges: partial + s * sstride holds
// a[rows] . dequant(w)[:, K range s]^T, [M_total][ldp].
int launch_grouped_int4_partial(const GroupedArgs& p, int splits, float* partial, int64_t ldp, int64_t sstride);
// K splits that give a grouped GEMM with few column tiles two blocks per CU (1: none).
int grouped_splits(int64_t M, int E, int64_t N, int64_t K, int group);

// e4m3 x e4m3 GEMM arguments (scales: pointer with a row stride, or the scalar).
struct Fp8Args {
  const uint8_t* a;
  int64_t lda;
  const uint8_t* b;
  int64_t ldb;
  float sa;
  const float* sap;
  int64_t sas;
  float sb;
  const float* sbp;
  int64_t sbs;
  void* c;
  int c_dt;
  int64_t ldc;
  int64_t M, N, K;
  hipStream_t stream;
  bool a_e5m2;  // A holds e5m2 bytes (B is always e4m3 here)
};

// Exact fp8 GEMM (A e4m3 or e5m2, B e4m3): operands widened to bf16 on the way into
// LDS, bf16 MFMA.
int launch_fp8_exact(const Fp8Args& f);

}  // namespace mls
