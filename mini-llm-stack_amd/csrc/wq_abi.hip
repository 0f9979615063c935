// C-ABI entry points of the weight-only GEMMs: argument validation on the host,
// then dispatch by shape: the VALU decode GEMV for small M (and fp32
// activations), the MFMA tiled GEMM for larger M with 16-bit activations, and a
// one-thread-per-output kernel for shapes neither fast path covers.
#include "mfma16.h"
#include "wq.h"

using namespace mls;

namespace {

int validate(const char* fn, int wbits, const WqArgs& p, int c_dt) {
  if (p.M < 0 || p.N < 0 || p.K < 0)
    return fail(MLS_ERR_ARG, "%s: negative size M=%lld N=%lld K=%lld", fn, (long long)p.M,
                (long long)p.N, (long long)p.K);
  if (!is_float_dt(p.a_dt)) return fail(MLS_ERR_ARG, "%s: bad activation dtype %d", fn, p.a_dt);
  if (c_dt != p.a_dt)
    return fail(MLS_ERR_ARG, "%s: output dtype %d must equal activation dtype %d", fn, c_dt, p.a_dt);
  if (p.s_dt != MLS_F32 && p.s_dt != MLS_F16)
    return fail(MLS_ERR_ARG, "%s: scale dtype %d (f32 or f16)", fn, p.s_dt);
  if (wbits == 4) {
    if (p.group < 1) return fail(MLS_ERR_ARG, "%s: group %d < 1", fn, p.group);
    if (p.K % p.group != 0 || p.K % 2 != 0)
      return fail(MLS_ERR_ARG, "%s: K=%lld must be even and a multiple of group %d", fn,
                  (long long)p.K, p.group);
    if (p.ld_sn < 0 || p.ld_sg < 0) return fail(MLS_ERR_ARG, "%s: negative scale stride", fn);
  }
  if (p.M == 0 || p.N == 0) return MLS_OK;
  if (!p.a || !p.w || !p.s || !p.c) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  const int64_t wcols = wbits == 4 ? p.K / 2 : p.K;
  if (p.lda < p.K || p.ldw < wcols || p.ldc < p.N)
    return fail(MLS_ERR_ARG, "%s: bad leading dimension (lda=%lld ldw=%lld ldc=%lld)", fn,
                (long long)p.lda, (long long)p.ldw, (long long)p.ldc);
  // M * N / 256 must fit 31 bits; compared by division (M, N > 0 here), as the product of
  // two valid int64 sizes can overflow
  if (p.M > (int64_t)0x7FFFFFFF * 256 / p.N) return fail(MLS_ERR_UNSUPPORTED, "%s: M*N too large", fn);
  return MLS_OK;
}

// Whether a GEMM with 16-bit activations goes to the register-operand medium GEMM rather
// than the LDS-tiled engine: the engine's 128 x 256 tiles need about 256 blocks to fill
// the GPU, which a short or narrow problem does not give (2048 x 2048 at M = 128: 8
// blocks). M <= 16 stays on the skinny GEMV, which measured faster there. MLS_SMALL = 0 / 1
// forces it off / on for 2 <= M (sweeps).
bool use_small(const WqArgs& p) {
  static const int env = env_int("MLS_SMALL", -1);
  if (p.a_dt == MLS_F32 || p.M < 2) return false;
  if (env >= 0) return env != 0;
  if (p.M <= 16) return false;
  return p.M <= 256 && cdiv(p.M, 128) * cdiv(p.N, 256) < 128;
}

int run(const char* fn, int wbits, const WqArgs& p) {
  if (p.M == 0 || p.N == 0) return MLS_OK;
  int rc = MLS_ERR_UNSUPPORTED;
  if (p.K > 0) {
    if (use_small(p)) rc = launch_gemm_small(wbits, p);
    const bool small_m = p.a_dt == MLS_F32 || p.M <= 16;
    if (rc != MLS_ERR_UNSUPPORTED) {
    } else if (small_m) {
      // M = 2 on the M = 1 GEMV's layout (INT4 -4%, INT8 -18% against the MFMA skinny kernel
      // at K = N = 4096); MLS_GEMV_M2=0 keeps M = 2 on the skinny kernel (A/B sweeps)
      static const bool rows_env = env_int("MLS_GEMV_M2", 1) != 0;
      if (rows_env && p.M == 2) rc = launch_gemv_rows(wbits, p);
      if (rc == MLS_ERR_UNSUPPORTED && p.M >= 2 && p.a_dt != MLS_F32) rc = launch_gemv_mfma(wbits, p);
      if (rc == MLS_ERR_UNSUPPORTED && p.M >= 2 && p.a_dt == MLS_F32) rc = launch_gemv_mfma_f32(wbits, p);
      if (rc == MLS_ERR_UNSUPPORTED) rc = launch_gemv_wq(wbits, p);
    } else {
      rc = launch_gemm_wq_mfma(wbits, p);
      if (rc == MLS_ERR_UNSUPPORTED) rc = launch_gemv_wq(wbits, p);
    }
  }
  if (rc == MLS_ERR_UNSUPPORTED) rc = launch_gemm_wq_generic(wbits, p);
  if (rc != MLS_OK) return rc;
  return check_launch(fn);
}

// fp32 activations with M >= 2 on the 16-bit matrix cores (split.hip): x is split into
// bf16 hi and lo rows in the workspace, then the skinny GEMV (M <= 16), the medium GEMM
// (few engine tiles) or the engine multiplies both and adds them. Taken only where the engine is
// sure to accept the split rows, so the split pass never runs for nothing.
// 2 <= M <= 16 takes the skinny MFMA GEMV on the split rows (each x MFMA once per part).
bool split_ok(int wbits, const WqArgs& p) {
  static const bool enabled = env_int("MLS_SPLIT", 1) != 0;  // 0: the VALU GEMV (A/B runs)
  if (!enabled || p.a_dt != MLS_F32 || p.M < 2 || p.M > 0x3FFFFFFF || p.K < 64 || p.K % 64 != 0) return false;
  if (!aligned(p.w, 16) || p.ldw % 16 != 0 || !aligned(p.c, 16)) return false;
  if (wbits == 4 && p.group % 64 != 0) return false;
  if (p.M <= 16 && wbits == 4 && p.group % 128 == 0 && p.K % 128 != 0) return false;  // (K % group == 0 anyway)
  const int64_t m2 = split_rows(p.M);
  return m2 <= 0x3FFFFFFF && p.N <= 0x3FFFFFFF && p.K <= 0x3FFFFFFF && p.K * 2 * 256 < (1ll << 31) &&
         p.ldw * 256 < (1ll << 31) && p.ld_sn <= 0x7FFFFFFF && p.ld_sg <= 0x7FFFFFFF;
}

int64_t split_ws_bytes(const WqArgs& p) { return split_rows(p.M) * p.K * 2; }

int run_split(const char* fn, int wbits, const WqArgs& p, void* ws) {
  int rc = launch_split_rows(static_cast<const float*>(p.a), p.lda, p.M, p.K, ws, p.stream);
  if (rc != MLS_OK) return rc;
  WqArgs q = p;
  q.a = ws;
  q.a_dt = MLS_BF16;
  q.lda = p.K;
  q.M = split_rows(p.M);
  if (p.M <= 16) {
    q.M = p.M;  // the skinny kernel reads the M hi rows and, 16 rows down, the M lo rows
    rc = launch_gemv_mfma_split(wbits, q);
  } else {
    rc = launch_split_gemm(wbits, q, p.M);
  }
  if (rc == MLS_ERR_UNSUPPORTED) return fail(MLS_ERR_HIP, "%s: split rows written but no split GEMM took them", fn);
  if (rc != MLS_OK) return rc;
  return check_launch(fn);
}

int run_ws(const char* fn, int wbits, const WqArgs& p, void* ws, int64_t ws_bytes) {
  if (p.M >= 2 && p.M <= 16 && p.N > 0 && p.a_dt == MLS_F32) {
    // fp32 x, 2 <= M <= 16: the skinny kernel splits x itself (no split pass, no workspace)
    const int rc = launch_gemv_mfma_f32(wbits, p);
    if (rc != MLS_ERR_UNSUPPORTED) return rc == MLS_OK ? check_launch(fn) : rc;
  }
  if (p.M == 0 || p.N == 0 || !split_ok(wbits, p)) return run(fn, wbits, p);
  const int64_t need = split_ws_bytes(p);
  if (!ws || ws_bytes < need || !aligned(ws, 256))
    return fail(MLS_ERR_ARG, "%s: workspace of %lld bytes at %p (need %lld, 256-byte aligned)", fn,
                (long long)ws_bytes, ws, (long long)need);
  return run_split(fn, wbits, p, ws);
}

}  // namespace

namespace mls {

// The medium GEMM where the engine would have few tiles (as use_small, on the split rows),
// else the engine.
int launch_split_gemm(int wbits, const WqArgs& q, int64_t m_out) {
  const int64_t eng_bm = wbits == 8 && q.M >= 256 ? 256 : 128;
  int rc = MLS_ERR_UNSUPPORTED;
  if (q.M <= 512 && cdiv(q.M, eng_bm) * cdiv(q.N, 256) < 128) rc = launch_gemm_small_split(wbits, q, m_out);
  if (rc == MLS_ERR_UNSUPPORTED) rc = launch_gemm_wq_mfma_split(wbits, q, m_out);
  return rc;
}

}  // namespace mls

extern "C" int64_t mls_wq_gemm_workspace(int wbits, int64_t M, int64_t N, int64_t K, int a_dt, int group) {
  if ((wbits != 4 && wbits != 8) || M <= 0 || N <= 0 || K <= 0) return 0;
  // the checks of split_ok that do not depend on pointers or strides (those can only turn
  // the split off, and then no workspace is used)
  WqArgs p{};
  p.a_dt = a_dt; p.M = M; p.N = N; p.K = K; p.group = wbits == 4 ? group : 0;
  if (a_dt != MLS_F32 || M < 2 || K < 64 || K % 64 != 0 || (wbits == 4 && (group < 1 || group % 64 != 0))) return 0;
  if (M > 0x3FFFFFFF || split_rows(M) > 0x3FFFFFFF || N > 0x3FFFFFFF || K > 0x3FFFFFFF || K * 2 * 256 >= (1ll << 31))
    return 0;
  return split_ws_bytes(p);
}

extern "C" int mls_int8_gemm_ws(const void* a, int a_dt, int64_t lda, const int8_t* w, int64_t ldw, const void* s,
                                int s_dt, void* c, int c_dt, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                void* workspace, int64_t ws_bytes, mls_stream_t stream) {
  WqArgs p{a, a_dt, lda, reinterpret_cast<const uint8_t*>(w), ldw, s, s_dt, 1, 0, 0,
           c, ldc, M, N, K, (hipStream_t)stream};
  int rc = validate("mls_int8_gemm_ws", 8, p, c_dt);
  if (rc != MLS_OK) return rc;
  return run_ws("mls_int8_gemm_ws", 8, p, workspace, ws_bytes);
}

extern "C" int mls_int4_gemm_ws(const void* a, int a_dt, int64_t lda, const uint8_t* w, int64_t ldw, const void* s,
                                int s_dt, int64_t ld_sn, int64_t ld_sg, int group, void* c, int c_dt, int64_t ldc,
                                int64_t M, int64_t N, int64_t K, void* workspace, int64_t ws_bytes,
                                mls_stream_t stream) {
  WqArgs p{a, a_dt, lda, w, ldw, s, s_dt, ld_sn, ld_sg, group, c, ldc, M, N, K, (hipStream_t)stream};
  int rc = validate("mls_int4_gemm_ws", 4, p, c_dt);
  if (rc != MLS_OK) return rc;
  return run_ws("mls_int4_gemm_ws", 4, p, workspace, ws_bytes);
}

extern "C" int mls_int8_gemm(const void* a, int a_dt, int64_t lda, const int8_t* w, int64_t ldw,
                             const void* s, int s_dt, void* c, int c_dt, int64_t ldc, int64_t M,
                             int64_t N, int64_t K, mls_stream_t stream) {
  WqArgs p{a, a_dt, lda, reinterpret_cast<const uint8_t*>(w), ldw, s, s_dt, 1, 0, 0,
           c, ldc, M, N, K, (hipStream_t)stream};
  int rc = validate("mls_int8_gemm", 8, p, c_dt);
  if (rc != MLS_OK) return rc;
  return run("mls_int8_gemm", 8, p);
}

extern "C" int mls_int4_gemm(const void* a, int a_dt, int64_t lda, const uint8_t* w, int64_t ldw,
                             const void* s, int s_dt, int64_t ld_sn, int64_t ld_sg, int group,
                             void* c, int c_dt, int64_t ldc, int64_t M, int64_t N, int64_t K,
                             mls_stream_t stream) {
  WqArgs p{a, a_dt, lda, w, ldw, s, s_dt, ld_sn, ld_sg, group, c, ldc, M, N, K,
           (hipStream_t)stream};
  int rc = validate("mls_int4_gemm", 4, p, c_dt);
  if (rc != MLS_OK) return rc;
  return run("mls_int4_gemm", 4, p);
}

namespace {

int grouped_gemm(const char* fn, const void* a, int a_dt, int64_t lda, const int32_t* a_rows,
                 int64_t a_src_rows, const int32_t* seg_off, int E, int64_t M_total, const uint8_t* w,
                 int64_t w_estride, int64_t ldw, const void* s, int s_dt, int64_t s_estride, int64_t ld_sn,
                 int64_t ld_sg, int group, void* c, int c_dt, int64_t ldc, int64_t N, int64_t K,
                 mls_stream_t stream) {
  GroupedArgs g{{a, a_dt, lda, w, ldw, s, s_dt, ld_sn, ld_sg, group, c, ldc, M_total, N, K,
                 (hipStream_t)stream},
                seg_off, E, w_estride, s_estride, a_rows, a_src_rows};
  int rc = validate(fn, 4, g.base, c_dt);
  if (rc != MLS_OK) return rc;
  if (E < 1) return fail(MLS_ERR_ARG, "%s: E=%d < 1", fn, E);
  if (K < 1) return fail(MLS_ERR_ARG, "%s: K=%lld must be positive", fn, (long long)K);
  if (w_estride < 0 || s_estride < 0) return fail(MLS_ERR_ARG, "%s: negative expert stride", fn);
  if (a_rows && a_src_rows < 1) return fail(MLS_ERR_ARG, "%s: a_src_rows=%lld < 1", fn, (long long)a_src_rows);
  if (M_total == 0 || N == 0) return MLS_OK;
  if (!seg_off) return fail(MLS_ERR_ARG, "%s: null seg_off", fn);
  if (a_dt != MLS_F16 && a_dt != MLS_BF16)
    return fail(MLS_ERR_UNSUPPORTED, "%s: activations must be f16 or bf16", fn);
  rc = launch_grouped_int4(g);
  if (rc == MLS_ERR_UNSUPPORTED)
    return fail(MLS_ERR_UNSUPPORTED,
                "%s: needs K %% 64 == 0, group %% 32 == 0, 16-byte aligned rows (and a gathered a under 1 GiB)",
                fn);
  return rc;
}

int grouped_gate_up(const char* fn, const void* a, int a_dt, int64_t lda, const int32_t* a_rows,
                    int64_t a_src_rows, const int32_t* seg_off, int E, int64_t M_total, const uint8_t* wg,
                    const uint8_t* wu, int64_t w_estride, int64_t ldw, const void* sg, const void* su, int s_dt,
                    int64_t s_estride, int64_t ld_sn, int64_t ld_sg, int group, void* h, int h_dt, int64_t ldh,
                    int64_t H, int64_t K, mls_stream_t stream) {
  GroupedArgs g{{a, a_dt, lda, wg, ldw, sg, s_dt, ld_sn, ld_sg, group, h, ldh, M_total, H, K,
                 (hipStream_t)stream},
                seg_off, E, w_estride, s_estride, a_rows, a_src_rows};
  int rc = validate(fn, 4, g.base, h_dt);
  if (rc != MLS_OK) return rc;
  if (E < 1) return fail(MLS_ERR_ARG, "%s: E=%d < 1", fn, E);
  if (K < 1) return fail(MLS_ERR_ARG, "%s: K=%lld must be positive", fn, (long long)K);
  if (w_estride < 0 || s_estride < 0) return fail(MLS_ERR_ARG, "%s: negative expert stride", fn);
  if (a_rows && a_src_rows < 1) return fail(MLS_ERR_ARG, "%s: a_src_rows=%lld < 1", fn, (long long)a_src_rows);
  if (M_total == 0 || H == 0) return MLS_OK;
  if (!seg_off || !wu || !su) return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (a_dt != MLS_F16 && a_dt != MLS_BF16)
    return fail(MLS_ERR_UNSUPPORTED, "%s: activations must be f16 or bf16", fn);
  rc = launch_grouped_gate_up(g, wu, su);
  if (rc == MLS_ERR_UNSUPPORTED)
    return fail(MLS_ERR_UNSUPPORTED,
                "%s: needs K %% 64 == 0, group %% 32 == 0, 16-byte aligned rows (and a gathered a under 1 GiB)",
                fn);
  return rc;
}

}  // namespace

extern "C" int mls_int4_grouped_gemm(const void* a, int a_dt, int64_t lda, const int32_t* seg_off,
                                     int E, int64_t M_total, const uint8_t* w, int64_t w_estride,
                                     int64_t ldw, const void* s, int s_dt, int64_t s_estride,
                                     int64_t ld_sn, int64_t ld_sg, int group, void* c, int c_dt,
                                     int64_t ldc, int64_t N, int64_t K, mls_stream_t stream) {
  return grouped_gemm("mls_int4_grouped_gemm", a, a_dt, lda, nullptr, 0, seg_off, E, M_total, w, w_estride, ldw,
                      s, s_dt, s_estride, ld_sn, ld_sg, group, c, c_dt, ldc, N, K, stream);
}

extern "C" int mls_int4_grouped_gemm_rows(const void* a, int a_dt, int64_t lda, const int32_t* a_rows,
                                          int64_t a_src_rows, const int32_t* seg_off, int E, int64_t M_total,
                                          const uint8_t* w, int64_t w_estride, int64_t ldw, const void* s,
                                          int s_dt, int64_t s_estride, int64_t ld_sn, int64_t ld_sg, int group,
                                          void* c, int c_dt, int64_t ldc, int64_t N, int64_t K,
                                          mls_stream_t stream) {
  const char* fn = "mls_int4_grouped_gemm_rows";
  if (!a_rows) return fail(MLS_ERR_ARG, "%s: null a_rows", fn);
  return grouped_gemm(fn, a, a_dt, lda, a_rows, a_src_rows, seg_off, E, M_total, w, w_estride, ldw, s, s_dt,
                      s_estride, ld_sn, ld_sg, group, c, c_dt, ldc, N, K, stream);
}

extern "C" int mls_int4_grouped_gate_up(const void* a, int a_dt, int64_t lda, const int32_t* seg_off,
                                        int E, int64_t M_total, const uint8_t* wg, const uint8_t* wu,
                                        int64_t w_estride, int64_t ldw, const void* sg, const void* su,
                                        int s_dt, int64_t s_estride, int64_t ld_sn, int64_t ld_sg,
                                        int group, void* h, int h_dt, int64_t ldh, int64_t H, int64_t K,
                                        mls_stream_t stream) {
  return grouped_gate_up("mls_int4_grouped_gate_up", a, a_dt, lda, nullptr, 0, seg_off, E, M_total, wg, wu,
                         w_estride, ldw, sg, su, s_dt, s_estride, ld_sn, ld_sg, group, h, h_dt, ldh, H, K, stream);
}

extern "C" int mls_int4_grouped_gate_up_rows(const void* a, int a_dt, int64_t lda, const int32_t* a_rows,
                                             int64_t a_src_rows, const int32_t* seg_off, int E, int64_t M_total,
                                             const uint8_t* wg, const uint8_t* wu, int64_t w_estride,
                                             int64_t ldw, const void* sg, const void* su, int s_dt,
                                             int64_t s_estride, int64_t ld_sn, int64_t ld_sg, int group, void* h,
                                             int h_dt, int64_t ldh, int64_t H, int64_t K, mls_stream_t stream) {
  const char* fn = "mls_int4_grouped_gate_up_rows";
  if (!a_rows) return fail(MLS_ERR_ARG, "%s: null a_rows", fn);
  return grouped_gate_up(fn, a, a_dt, lda, a_rows, a_src_rows, seg_off, E, M_total, wg, wu, w_estride, ldw, sg,
                         su, s_dt, s_estride, ld_sn, ld_sg, group, h, h_dt, ldh, H, K, stream);
}

extern "C" int mls_int4_grouped_splits(int64_t M_total, int E, int64_t N, int64_t K, int group) {
  return grouped_splits(M_total, E, N, K, group);
}

extern "C" int mls_int4_grouped_gemm_partial(const void* a, int a_dt, int64_t lda, const int32_t* seg_off,
                                             int E, int64_t M_total, const uint8_t* w, int64_t w_estride,
                                             int64_t ldw, const void* s, int s_dt, int64_t s_estride,
                                             int64_t ld_sn, int64_t ld_sg, int group, int splits, float* partial,
                                             int64_t ldp, int64_t split_stride, int64_t N, int64_t K,
                                             mls_stream_t stream) {
  const char* fn = "mls_int4_grouped_gemm_partial";
  GroupedArgs g{{a, a_dt, lda, w, ldw, s, s_dt, ld_sn, ld_sg, group, partial, ldp, M_total, N, K,
                 (hipStream_t)stream},
                seg_off, E, w_estride, s_estride};
  int rc = validate(fn, 4, g.base, a_dt);
  if (rc != MLS_OK) return rc;
  if (E < 1) return fail(MLS_ERR_ARG, "%s: E=%d < 1", fn, E);
  if (K < 1) return fail(MLS_ERR_ARG, "%s: K=%lld must be positive", fn, (long long)K);
  if (splits < 1 || splits > 64) return fail(MLS_ERR_ARG, "%s: splits=%d", fn, splits);
  if (w_estride < 0 || s_estride < 0 || split_stride < M_total * ldp)
    return fail(MLS_ERR_ARG, "%s: bad expert or split stride", fn);
  if (M_total == 0 || N == 0) return MLS_OK;
  if (!seg_off) return fail(MLS_ERR_ARG, "%s: null seg_off", fn);
  rc = launch_grouped_int4_partial(g, splits, partial, ldp, split_stride);
  if (rc == MLS_ERR_UNSUPPORTED)
    return fail(MLS_ERR_UNSUPPORTED,
                "%s: needs 16-bit activations, K / splits a multiple of 64 and of the group, 16-byte aligned "
                "rows", fn);
  return rc;
}
