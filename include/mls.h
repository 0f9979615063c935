/*
 * mls.h — C ABI of libmls_hip.so, the gfx950 (MI355X) quantized-linear library.
 *
 * Plain C: raw device pointers, element strides, sizes and a HIP stream. No
 * torch types cross this boundary. Every entry point validates its arguments on
 * the host before any HIP call and returns MLS_OK (0) or a negative MLS_ERR_*
 * code; mls_last_error() then holds a message (thread-local).
 *
 * Ownership: the caller allocates every buffer (inputs, outputs and any
 * workspace). The library never allocates, frees or synchronises on these
 * paths; all work is enqueued on `stream` (a hipStream_t; NULL = the default
 * stream of the current device).
 *
 * Layouts (all row-major, unit inner stride, leading dimensions in ELEMENTS):
 *   activations  a[M][K]           lda >= K
 *   INT8 weights w[N][K] int8      ldw >= K        scale s[N]
 *   INT4 weights w[N][K/2] uint8   ldw >= K/2      scale s[N][K/group] with
 *                (even k -> low nibble, value = nibble - 8)     strides ld_sn, ld_sg
 *   e4m3 bytes   OCP FP8 E4M3 ("fn": bias 7, no inf, max 448, NaN = S.1111.111)
 *
 * dtype codes: MLS_F32, MLS_F16, MLS_BF16 (MLS_F64 only where an entry point says so).
 */
#ifndef MLS_H
#define MLS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mls_stream_t; /* identical to hipStream_t */

enum { MLS_F32 = 0, MLS_F16 = 1, MLS_BF16 = 2,
       MLS_F64 = 3 /* only where an entry point says so (mls_moe_combine) */ };
enum {
  MLS_OK = 0,
  MLS_ERR_ARG = -1,         /* invalid argument (shape, stride, dtype, null, alignment) */
  MLS_ERR_UNSUPPORTED = -2, /* valid but outside what the library implements */
  MLS_ERR_HIP = -3          /* a HIP runtime call failed */
};

#define MLS_ABI_VERSION 7

/* No reference counterpart: version of this ABI (MLS_ABI_VERSION). */
int mls_abi_version(void);

/* No reference counterpart: message for the last failing call on this thread. */
const char* mls_last_error(void);

/* ---------------------------------------------------------------- e4m3 codec */

/* Replaces _decode_e4m3_kernel + decode_e4m3 (kernels/fp8_matmul.py:37-47, 84-100):
 * out[i] = value of e4m3 byte bits[i] as fp32; the NaN patterns 0x7F/0xFF decode
 * to 0 (fp8_matmul.py:46). Bit-exact. */
int mls_e4m3_decode(const uint8_t* bits, float* out, int64_t n, mls_stream_t stream);

/* Replaces dequantize_e4m3 (kernels/fp8_matmul.py:109-110): out[r][c] =
 * value(bits[r][c]) * scale_r, where NaN patterns stay NaN (torch's float8 view
 * semantics) and scale_r = scale_ptr ? scale_ptr[r * scale_stride] : scale.
 * The multiply is one fp32 rounding, as in the reference. */
int mls_e4m3_dequantize(const uint8_t* bits, int64_t rows, int64_t cols, int64_t ldb,
                        float scale, const float* scale_ptr, int64_t scale_stride,
                        float* out, int64_t ldo, mls_stream_t stream);

/* Replaces quantize_e4m3 (kernels/fp8_matmul.py:103-106): q = x / scale_r
 * (IEEE fp32 division), clamped to [-448, 448], then rounded to the nearest e4m3
 * value, ties to even. x is f32/f16/bf16 (x_dt). NaN inputs give 0x7F|sign.
 * scale_r as for mls_e4m3_dequantize. Bit-exact against the reference's CPU path. */
int mls_e4m3_encode(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                    float scale, const float* scale_ptr, int64_t scale_stride,
                    uint8_t* out, int64_t ldo, mls_stream_t stream);

/* Replaces _quant_e5m2 (train/fp8.py:50-52): q = x / scale_r (IEEE fp32 division),
 * clamped to [-57344, 57344], rounded to the nearest e5m2 value, ties to even; NaN
 * inputs give 0x7F|sign (torch's float8_e5m2 cast). Arguments as for
 * mls_e4m3_encode. Bit-exact against the reference's CPU path. */
int mls_e5m2_encode(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                    float scale, const float* scale_ptr, int64_t scale_stride,
                    uint8_t* out, int64_t ldo, mls_stream_t stream);

/* mls_e5m2_encode that also writes the transposed bytes: out[r][c] and
 * out_t[c][r] = e5m2(x[r][c] / scale[r]) (same rounding as mls_e5m2_encode).
 * FP8 training's backward needs the e5m2 gradient in both layouts: dy for
 * dx = dy W and dy^T for dw = dy^T x (train/fp8.py:88-94); one pass replaces an
 * encode and a transpose. ldt >= rows. */
int mls_e5m2_encode_t(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                      float scale, const float* scale_ptr, int64_t scale_stride,
                      uint8_t* out, int64_t ldo, uint8_t* out_t, int64_t ldt, mls_stream_t stream);

/* mls_e4m3_encode that also writes the transposed bytes (same rounding): with
 * FP8Linear's kernels, the forward encodes x and W once into both layouts and keeps
 * the transposes for the backward (train/fp8.py:68-69, 88-94), which needs x^T and
 * W^T only. ldt >= rows. */
int mls_e4m3_encode_t(const void* x, int x_dt, int64_t rows, int64_t cols, int64_t ldx,
                      float scale, const float* scale_ptr, int64_t scale_stride,
                      uint8_t* out, int64_t ldo, uint8_t* out_t, int64_t ldt, mls_stream_t stream);

/* No single reference counterpart: the byte transpose behind the .t() of fp8
 * operands in FP8 training's backward (train/fp8.py:92-94), which the K-contiguous
 * GEMM needs materialised: dst[c][r] = src[r][c] for r < rows, c < cols. */
int mls_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, int64_t lds,
                     uint8_t* dst, int64_t ldd, mls_stream_t stream);

/* ---------------------------------------------------------------- quantizers */

/* Replaces quantize_int8 (serve/quantize.py:18-21) for device tensors:
 * scale[n] = max(max_k |w[n][k]| / 127, 1e-8); wq = clamp(rint(w / scale), -127, 127).
 * fp32 in, IEEE division, round half to even. Bit-exact. */
int mls_quantize_int8(const float* w, int64_t N, int64_t K, int64_t ldw,
                      int8_t* wq, int64_t ldq, float* scale, mls_stream_t stream);

/* Replaces quantize_int4 (serve/quantize.py:28-36) for device tensors: per group of
 * `group` along K, scale = max(amax / 7, 1e-8); q = clamp(rint(w / scale), -8, 7) + 8;
 * packed[n][j] = q[n][2j] | q[n][2j+1] << 4. scale is [N][K/group] contiguous.
 * Requires K % group == 0 and K even. Bit-exact. */
int mls_quantize_int4(const float* w, int64_t N, int64_t K, int64_t ldw, int group,
                      uint8_t* packed, int64_t ldp, float* scale, mls_stream_t stream);

/* ---------------------------------------------------------------- GEMMs */

/* Replaces _int8_matmul_kernel + int8_matmul (kernels/dequant_matmul.py:39-66, 140-152):
 * c[m][n] = s[n] * sum_k a[m][k] * w[n][k], fp32 accumulation, one rounding to c_dt.
 * a_dt = c_dt in {F32, F16, BF16}; s_dt in {F32, F16}. Any M, N, K >= 1. */
int mls_int8_gemm(const void* a, int a_dt, int64_t lda,
                  const int8_t* w, int64_t ldw,
                  const void* s, int s_dt,
                  void* c, int c_dt, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, mls_stream_t stream);

/* Replaces _int4_matmul_kernel + int4_matmul (kernels/dequant_matmul.py:69-100, 170-185):
 * c[m][n] = sum_k a[m][k] * (nib(w, n, k) - 8) * s[n * ld_sn + (k / group) * ld_sg].
 * Requires K % group == 0 (the reference's assert, :175). fp32 accumulation. */
int mls_int4_gemm(const void* a, int a_dt, int64_t lda,
                  const uint8_t* w, int64_t ldw,
                  const void* s, int s_dt, int64_t ld_sn, int64_t ld_sg, int group,
                  void* c, int c_dt, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, mls_stream_t stream);

/* The same two GEMMs (kernels/dequant_matmul.py:39-100, 140-185) with a caller workspace,
 * for fp32 activations on the matrix cores: with a_dt = F32 and M >= 2 (and K % 64 == 0,
 * 16-byte aligned weight rows, a 16-byte aligned c, INT4 groups a multiple of 64) x is
 * split into bf16 hi and lo parts (hi = x truncated to bf16, lo = bf16(x - hi): x to about
 * 2^-16 of its magnitude) in the workspace, and both are multiplied on the bf16 MFMA with
 * fp32 accumulation and added in fp32; every other call runs as mls_int8_gemm /
 * mls_int4_gemm and ignores the workspace. mls_wq_gemm_workspace(wbits, M, N, K, a_dt,
 * group) gives the bytes (256-byte aligned workspace; 0: none used). */
int64_t mls_wq_gemm_workspace(int wbits, int64_t M, int64_t N, int64_t K, int a_dt, int group);
int mls_int8_gemm_ws(const void* a, int a_dt, int64_t lda,
                     const int8_t* w, int64_t ldw,
                     const void* s, int s_dt,
                     void* c, int c_dt, int64_t ldc,
                     int64_t M, int64_t N, int64_t K,
                     void* workspace, int64_t ws_bytes, mls_stream_t stream);
int mls_int4_gemm_ws(const void* a, int a_dt, int64_t lda,
                     const uint8_t* w, int64_t ldw,
                     const void* s, int s_dt, int64_t ld_sn, int64_t ld_sg, int group,
                     void* c, int c_dt, int64_t ldc,
                     int64_t M, int64_t N, int64_t K,
                     void* workspace, int64_t ws_bytes, mls_stream_t stream);

/* Replaces _int8_dgrad_kernel + int8_dgrad (kernels/dequant_matmul.py:103-132, 155-167):
 * dx[m][k] = sum_n dy[m][n] * s[n] * w[n][k] (the input gradient of y = x W^T). */
int mls_int8_dgrad(const void* dy, int dy_dt, int64_t lddy,
                   const int8_t* w, int64_t ldw,
                   const void* s, int s_dt,
                   void* dx, int dx_dt, int64_t lddx,
                   int64_t M, int64_t N, int64_t K, mls_stream_t stream);

/* The same input gradient on the matrix cores, with the reference's arithmetic
 * (kernels/dequant_matmul.py:127-128): ys = (dy * s) rounded to dy's dtype, times the int8
 * weights on the 16-bit MFMA, fp32 accumulation; fp32 dy with M > 16: ys in fp32 as bf16
 * hi + lo parts (as mls_int8_gemm_ws), both multiplied and added in fp32. Needs a caller
 * workspace of mls_int8_dgrad_workspace(M, N, K, dy_dt) bytes, 256-byte aligned (the scaled
 * dy, the transposed weights and a vector of ones); 0 means this shape takes mls_int8_dgrad's
 * route (fp32 dy with M <= 16), for which workspace may be null. Runs on `stream`, three
 * launches. */
int64_t mls_int8_dgrad_workspace(int64_t M, int64_t N, int64_t K, int dy_dt);
int mls_int8_dgrad_ws(const void* dy, int dy_dt, int64_t lddy,
                      const int8_t* w, int64_t ldw,
                      const void* s, int s_dt,
                      void* dx, int dx_dt, int64_t lddx,
                      int64_t M, int64_t N, int64_t K,
                      void* workspace, int64_t ws_bytes, mls_stream_t stream);

/* Replaces _fp8_matmul_kernel + fp8_matmul (kernels/fp8_matmul.py:50-81, 113-128):
 * c[m][n] = (sum_k e4m3(a[m][k]) * e4m3(b[n][k])) * sa_m * sb_n, fp32 accumulation.
 * sa_m = sa_ptr ? sa_ptr[m * sa_stride] : sa, likewise sb_n: per-tensor (the
 * reference) or per-row scales. c_dt any of F32/F16/BF16.
 * flags = 0 (exact): operands widened to bf16 and multiplied on the bf16 MFMA,
 *   whose accumulation matches an fp32 GEMM of the decoded operands.
 * flags = MLS_FP8_NATIVE: e4m3 bytes straight into the gfx950 fp8 MFMA (twice the
 *   peak rate); that instruction truncates each product of a group of 8 toward zero
 *   at 2^-13 of the group's largest before adding them, so outlier-heavy rows differ
 *   from the fp32 result.
 * NaN operand bytes propagate NaN on the MFMA paths (the reference decodes them
 * to 0; quantize_e4m3 never produces them).
 * flags |= MLS_FP8_A_E5M2: a holds e5m2 bytes (b stays e4m3): the gradient operand of
 *   FP8 training's backward GEMMs (train/fp8.py:80-95: dx = dy W, dw = dy^T x with dy
 *   in e5m2), on the same datapaths (e5m2 widens to bf16 exactly; the native path
 *   selects the MFMA's bf8 operand format). */
#define MLS_FP8_NATIVE 1
#define MLS_FP8_A_E5M2 2
int mls_fp8_gemm(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb,
                 float sa, const float* sa_ptr, int64_t sa_stride,
                 float sb, const float* sb_ptr, int64_t sb_stride,
                 void* c, int c_dt, int64_t ldc,
                 int64_t M, int64_t N, int64_t K, int flags, mls_stream_t stream);

/* Replaces the per-expert segment loop of moe_dispatch_combine
 * (kernels/moe_routing.py:145-151) that calls int4_matmul once per expert through
 * QuantLinear (serve/quantize.py:110-114): one launch over all experts.
 * Rows seg_off[e] .. seg_off[e+1]-1 of a (expert-sorted, M_total rows) multiply
 * expert e's packed weights w + e*w_estride (bytes) with scales s + e*s_estride
 * (elements). seg_off is a DEVICE int32 array of E+1 non-decreasing offsets with
 * seg_off[0] = 0 and seg_off[E] = M_total; it is read on the device (no host sync).
 * Each segment is clamped to [0, M_total) on the device: offsets that break the
 * contract give wrong rows, never an access outside a or c.
 * a_dt = c_dt in {F16, BF16}. */
int mls_int4_grouped_gemm(const void* a, int a_dt, int64_t lda,
                          const int32_t* seg_off, int E, int64_t M_total,
                          const uint8_t* w, int64_t w_estride, int64_t ldw,
                          const void* s, int s_dt, int64_t s_estride,
                          int64_t ld_sn, int64_t ld_sg, int group,
                          void* c, int c_dt, int64_t ldc,
                          int64_t N, int64_t K, mls_stream_t stream);

/* mls_int4_grouped_gemm with the dispatch gather fused into the activation load
 * (replaces gather_rows, kernels/moe_routing.py:89-97 + 144, in front of the per-expert
 * loop): sorted row m of the product reads row a_rows[m] of a, a [a_src_rows][lda];
 * a_rows int32 [M_total] on the device (the token of each sorted slot, sort_by_expert's
 * token_of_slot). A row index outside [0, a_src_rows) reads zeros. */
int mls_int4_grouped_gemm_rows(const void* a, int a_dt, int64_t lda,
                               const int32_t* a_rows, int64_t a_src_rows,
                               const int32_t* seg_off, int E, int64_t M_total,
                               const uint8_t* w, int64_t w_estride, int64_t ldw,
                               const void* s, int s_dt, int64_t s_estride,
                               int64_t ld_sn, int64_t ld_sg, int group,
                               void* c, int c_dt, int64_t ldc,
                               int64_t N, int64_t K, mls_stream_t stream);

/* ---------------------------------------------------------------- MoE expert MLP */

/* The gate/up half of the quantized SwiGLU expert MLP (train/model.py:127-135,
 * SwiGLU.forward: w_down(silu(w_gate(x)) * w_up(x)), with w_gate / w_up swapped for
 * INT4 QuantLinear by serve/quantize.py:110-114) for every expert in one launch:
 * h[r] = silu(a[r] . dequant(wg_e)^T) * (a[r] . dequant(wu_e)^T) for the rows r of
 * expert e's segment, fp32 accumulation, one rounding to h_dt (= a_dt, F16 or BF16).
 * The reference runs this as two QuantLinear calls per expert plus elementwise ops
 * (moe_routing.py:145-151 loop); here the 2 x H intermediate never reaches memory.
 * Layouts and seg_off as for mls_int4_grouped_gemm; the up matrices/scales share the
 * gate's strides. */
int mls_int4_grouped_gate_up(const void* a, int a_dt, int64_t lda,
                             const int32_t* seg_off, int E, int64_t M_total,
                             const uint8_t* wg, const uint8_t* wu, int64_t w_estride, int64_t ldw,
                             const void* sg, const void* su, int s_dt, int64_t s_estride,
                             int64_t ld_sn, int64_t ld_sg, int group,
                             void* h, int h_dt, int64_t ldh,
                             int64_t H, int64_t K, mls_stream_t stream);

/* mls_int4_grouped_gate_up with the dispatch gather fused into the activation load, as
 * mls_int4_grouped_gemm_rows (gather_rows, kernels/moe_routing.py:89-97 + 144). */
int mls_int4_grouped_gate_up_rows(const void* a, int a_dt, int64_t lda,
                                  const int32_t* a_rows, int64_t a_src_rows,
                                  const int32_t* seg_off, int E, int64_t M_total,
                                  const uint8_t* wg, const uint8_t* wu,
                                  int64_t w_estride, int64_t ldw,
                                  const void* sg, const void* su, int s_dt,
                                  int64_t s_estride, int64_t ld_sn, int64_t ld_sg, int group,
                                  void* h, int h_dt, int64_t ldh,
                                  int64_t H, int64_t K, mls_stream_t stream);

/* Replaces _combine_rows_kernel + combine_rows (kernels/moe_routing.py:52-76, 100-113):
 * out[t][d] = sum_{s<k} w[t][s] * X(pos[t][s], d), fp32 accumulation, one rounding; one block
 * per output row, no atomics. x_dt MLS_F64 (the reference's ACC64, moe_routing.py:58-72,
 * 112): accumulated in fp64, and out_dt must be MLS_F64; w_dt may be any of the four. x: x_dt [x_rows][ldx]; X(r, d) = x[r][d], or with splits > 1
 * the sum of the `splits` partial products x[p * split_stride + r * ldx + d] of a K-split
 * GEMM (mls_int4_grouped_gemm_partial). out: out_dt [T][ldo]; w: w_dt [T][k]; pos: int64
 * [T][k]; a position outside [0, x_rows) contributes nothing. */
int mls_moe_combine(const void* x, int x_dt, int64_t ldx, int64_t x_rows, int splits, int64_t split_stride,
                    const void* w, int w_dt, const int64_t* pos, int64_t T, int k,
                    void* out, int out_dt, int64_t ldo, int64_t D, mls_stream_t stream);

/* No single reference counterpart: the down projection of the INT4 expert MLP
 * (train/model.py:135 per expert, kernels/moe_routing.py:145-151) as `splits` fp32
 * partial products over equal K ranges, partial[p][r][n] at partial + p * split_stride +
 * r * ldp + n, for mls_moe_combine to sum: a narrow output (few column tiles) then still
 * spreads over two blocks per CU. Arguments otherwise as mls_int4_grouped_gemm; needs
 * K / splits a multiple of 64 and of the group (MLS_ERR_UNSUPPORTED otherwise).
 * mls_int4_grouped_splits returns the split count this build uses for a shape (1: no
 * split). */
int mls_int4_grouped_splits(int64_t M_total, int E, int64_t N, int64_t K, int group);
int mls_int4_grouped_gemm_partial(const void* a, int a_dt, int64_t lda, const int32_t* seg_off,
                                  int E, int64_t M_total, const uint8_t* w, int64_t w_estride, int64_t ldw,
                                  const void* s, int s_dt, int64_t s_estride, int64_t ld_sn, int64_t ld_sg,
                                  int group, int splits, float* partial, int64_t ldp, int64_t split_stride,
                                  int64_t N, int64_t K, mls_stream_t stream);

/* Replaces _paged_attn_kernel + paged_attention_decode (kernels/paged_attention.py:33-118):
 * out[s][h][:] = softmax_j(scale * q[s][h] . K_j) V_j over the context_lens[s] tokens of
 * sequence s, token j at row j % block_size of block block_tables[s][j / block_size].
 * q, out: [n_seqs][H][D] (strides q_ss/q_sh, o_ss/o_sh; unit stride in D), q_dt (out too);
 * pools: [num_blocks][H][block_size][D] of kv_dt, strides kv_sb/kv_sh/kv_st shared by K and
 * V, unit stride in D. Tokens at or past the context length weigh 0; a block id outside
 * [0, num_blocks) is skipped; a zero context gives zeros. The workspace (fp32) must hold
 * mls_paged_attention_workspace(n_seqs, H, D, max_blocks) floats (0: none needed). */
int64_t mls_paged_attention_workspace(int64_t n_seqs, int64_t H, int64_t D, int64_t max_blocks);
int mls_paged_attention_decode(const void* q, int q_dt, int64_t q_ss, int64_t q_sh,
                               const void* k_pool, const void* v_pool, int kv_dt,
                               int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t num_blocks,
                               const int32_t* block_tables, int64_t bt_ss, int64_t max_blocks,
                               const int32_t* context_lens,
                               void* out, int64_t o_ss, int64_t o_sh,
                               int64_t n_seqs, int64_t H, int64_t D, int64_t block_size, float scale,
                               float* workspace, int64_t workspace_floats, mls_stream_t stream);

/* No reference counterpart. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * decode as mls_paged_attention_decode with the context-split workspace taken from a
 * static device array of MLS_PAGED_SCRATCH_FLOATS floats (8 MiB per GPU, held until the
 * process ends) instead of a caller buffer. Allocates and frees nothing. A call whose
 * split needs more than the array (mls_paged_attention_workspace > the maximum; never
 * for head dims up to 254) returns MLS_ERR_ARG. All calls on one GPU share its array:
 * calls that overlap on one GPU (two streams, two host threads) race. */
#define MLS_PAGED_SCRATCH_FLOATS (2 * 1024 * 1024)
int mls_paged_attention_decode_noalloc(const void* q, int q_dt, int64_t q_ss, int64_t q_sh,
                                       const void* k_pool, const void* v_pool, int kv_dt,
                                       int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t num_blocks,
                                       const int32_t* block_tables, int64_t bt_ss, int64_t max_blocks,
                                       const int32_t* context_lens,
                                       void* out, int64_t o_ss, int64_t o_sh,
                                       int64_t n_seqs, int64_t H, int64_t D, int64_t block_size, float scale,
                                       mls_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MLS_H */
