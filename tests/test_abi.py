"""The C-ABI library: it loads, exports every symbol include/mls.h declares, and
rejects invalid arguments on the host before any HIP call (these calls pass null
device pointers, so they never reach the GPU)."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT

import kernels

HEADER = ROOT / "include" / "mls.h"
NULL = None


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(mls_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_boundary():
    syms = declared_symbols()
    assert len(syms) == len(set(syms)) == 30
    assert set(syms) == set(kernels.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(kernels.LIB_PATH))
    for s in declared_symbols():
        assert hasattr(lib, s), s


def test_abi_version_and_error_string():
    lib = kernels.load_library()
    assert lib.mls_abi_version() == kernels.ABI_VERSION == 7
    assert isinstance(lib.mls_last_error(), bytes)


def _err(rc):
    return rc, kernels.lib().mls_last_error().decode()


@pytest.mark.parametrize("bad", ["neg_m", "null", "dtype", "out_dtype", "scale_dtype", "lda"])
def test_int8_gemm_rejects(bad):
    L = kernels.load_library()
    a = dict(a=1, adt=kernels.MLS_BF16, lda=64, w=1, ldw=64, s=1, sdt=kernels.MLS_F32, c=1,
             cdt=kernels.MLS_BF16, ldc=32, M=4, N=32, K=64)
    if bad == "neg_m":
        a["M"] = -1
    elif bad == "null":
        a["a"] = NULL
    elif bad == "dtype":
        a["adt"] = a["cdt"] = 7
    elif bad == "out_dtype":
        a["cdt"] = kernels.MLS_F32
    elif bad == "scale_dtype":
        a["sdt"] = kernels.MLS_BF16
    elif bad == "lda":
        a["lda"] = 10
    rc, msg = _err(L.mls_int8_gemm(a["a"], a["adt"], a["lda"], a["w"], a["ldw"], a["s"], a["sdt"],
                                   a["c"], a["cdt"], a["ldc"], a["M"], a["N"], a["K"], NULL))
    assert rc == kernels.MLS_ERR_ARG and "mls_int8_gemm" in msg


def test_int4_gemm_rejects_group_mismatch():
    L = kernels.load_library()
    rc, msg = _err(L.mls_int4_gemm(1, kernels.MLS_F32, 96, 1, 48, 1, kernels.MLS_F32, 3, 1, 64,
                                   1, kernels.MLS_F32, 8, 2, 8, 96, NULL))
    assert rc == kernels.MLS_ERR_ARG and "group" in msg
    rc, _ = _err(L.mls_int4_gemm(1, kernels.MLS_F32, 96, 1, 48, 1, kernels.MLS_F32, 3, 1, 0,
                                 1, kernels.MLS_F32, 8, 2, 8, 96, NULL))
    assert rc == kernels.MLS_ERR_ARG


def test_zero_sized_calls_are_noops():
    L = kernels.load_library()
    assert L.mls_int8_gemm(NULL, 0, 0, NULL, 0, NULL, 0, NULL, 0, 0, 0, 5, 5, NULL) == 0
    assert L.mls_e4m3_decode(NULL, NULL, 0, NULL) == 0
    assert L.mls_fp8_gemm(NULL, 0, NULL, 0, 1.0, NULL, 0, 1.0, NULL, 0, NULL, 0, 0, 0, 0, 8, 0, NULL) == 0


def test_fp8_and_codec_reject():
    L = kernels.load_library()
    assert L.mls_fp8_gemm(1, 64, 1, 64, 1.0, NULL, 0, 1.0, NULL, 0, 1, 9, 8, 4, 8, 64, 0, NULL) == \
        kernels.MLS_ERR_ARG
    assert L.mls_fp8_gemm(1, 32, 1, 64, 1.0, NULL, 0, 1.0, NULL, 0, 1, 0, 8, 4, 8, 64, 0, NULL) == \
        kernels.MLS_ERR_ARG
    assert L.mls_fp8_gemm(1, 64, 1, 64, 1.0, NULL, 0, 1.0, NULL, 0, 1, 0, 8, 4, 8, 64, 4, NULL) == \
        kernels.MLS_ERR_ARG
    assert L.mls_e4m3_decode(1, 1, -3, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_e4m3_encode(1, 5, 2, 2, 2, 1.0, NULL, 0, 1, 2, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_quantize_int4(1, 4, 30, 30, 4, 1, 15, 1, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_int8_dgrad(1, 0, 8, 1, 8, 1, 0, 1, 1, 8, 2, 8, 8, NULL) == kernels.MLS_ERR_ARG


def test_grouped_rejects():
    L = kernels.load_library()
    # E = 0
    assert L.mls_int4_grouped_gemm(1, kernels.MLS_BF16, 64, 1, 0, 8, 1, 0, 32, 1, 0, 0, 2, 1, 32,
                                   1, kernels.MLS_BF16, 16, 16, 64, NULL) == kernels.MLS_ERR_ARG
    # fp32 activations are outside the grouped kernel
    assert L.mls_int4_grouped_gemm(1, kernels.MLS_F32, 64, 1, 2, 8, 1, 0, 32, 1, 0, 0, 2, 1, 32,
                                   1, kernels.MLS_F32, 16, 16, 64, NULL) == kernels.MLS_ERR_UNSUPPORTED


def test_grouped_reject_empty_k():
    """K = 0 passes the K % 64 and K % group checks; the grouped kernels would then read
    scales before the buffer, so the host rejects it first (all three entry points)."""
    L = kernels.load_library()
    bf = kernels.MLS_BF16
    rc, msg = _err(L.mls_int4_grouped_gemm(1, bf, 64, 1, 2, 8, 1, 0, 32, 1, kernels.MLS_F16, 0, 2, 1, 32,
                                           1, bf, 16, 16, 0, NULL))
    assert rc == kernels.MLS_ERR_ARG and "K=0" in msg
    rc, msg = _err(L.mls_int4_grouped_gate_up(1, bf, 64, 1, 2, 8, 1, 1, 0, 32, 1, 1, kernels.MLS_F16, 0, 2, 1,
                                              32, 1, bf, 16, 16, 0, NULL))
    assert rc == kernels.MLS_ERR_ARG and "K=0" in msg
    rc, msg = _err(L.mls_int4_grouped_gemm_partial(1, bf, 64, 1, 2, 8, 1, 0, 32, 1, kernels.MLS_F16, 0, 2, 1,
                                                   32, 1, 1, 16, 128, 16, 0, NULL))
    assert rc == kernels.MLS_ERR_ARG and "K=0" in msg


def test_dgrad_workspace_and_rejects():
    """The matrix-core dgrad's workspace: scaled dy [M][Np] 16-bit (fp32 dy: its bf16 hi and
    lo rows, 32 per 16 rows of dy) + transposed weights [K][Np] bytes + K fp32 ones, Np = N
    rounded up to 64, each part 256-byte aligned; 0 for fp32 dy with M <= 16 (the VALU
    route). A short or misaligned workspace is rejected on the host."""
    L = kernels.load_library()
    bf = kernels.MLS_BF16
    M, N, K = 40, 100, 72
    Np = 128
    up = lambda b: -(-b // 256) * 256
    assert L.mls_int8_dgrad_workspace(M, N, K, bf) == up(M * Np * 2) + up(K * Np) + up(K * 4)
    assert L.mls_int8_dgrad_workspace(M, N, K, kernels.MLS_F16) == up(M * Np * 2) + up(K * Np) + up(K * 4)
    assert L.mls_int8_dgrad_workspace(M, N, K, kernels.MLS_F32) == up(96 * Np * 2) + up(K * Np) + up(K * 4)
    assert L.mls_int8_dgrad_workspace(16, N, K, kernels.MLS_F32) == 0
    assert L.mls_int8_dgrad_workspace(0, N, K, bf) == 0
    need = L.mls_int8_dgrad_workspace(M, N, K, bf)
    args = (1, bf, N, 1, K, 1, kernels.MLS_F32, 1, bf, K, M, N, K)
    rc, msg = _err(L.mls_int8_dgrad_ws(*args, 256, need - 1, NULL))
    assert rc == kernels.MLS_ERR_ARG and "workspace" in msg
    rc, msg = _err(L.mls_int8_dgrad_ws(*args, 256 + 16, need, NULL))
    assert rc == kernels.MLS_ERR_ARG and "aligned" in msg
    rc, msg = _err(L.mls_int8_dgrad_ws(*args, NULL, need, NULL))
    assert rc == kernels.MLS_ERR_ARG
    rc, msg = _err(L.mls_int8_dgrad_ws(1, bf, N, 1, K, 1, kernels.MLS_F32, 1, kernels.MLS_F16, K, M, N, K,
                                       256, need, NULL))
    assert rc == kernels.MLS_ERR_ARG and "dtypes" in msg


def test_gate_up_and_combine_reject():
    L = kernels.load_library()
    bf = kernels.MLS_BF16
    # null up matrix
    assert L.mls_int4_grouped_gate_up(1, bf, 64, 1, 2, 8, 1, NULL, 0, 32, 1, 1, 0, 2, 1, 1, 32,
                                      1, bf, 16, 16, 64, NULL) == kernels.MLS_ERR_ARG
    # fp32 activations
    assert L.mls_int4_grouped_gate_up(1, kernels.MLS_F32, 64, 1, 2, 8, 1, 1, 0, 32, 1, 1, 0, 2, 1, 1,
                                      32, 1, kernels.MLS_F32, 16, 16, 64, NULL) == kernels.MLS_ERR_UNSUPPORTED
    # output dtype differs from the activations
    assert L.mls_int4_grouped_gate_up(1, bf, 64, 1, 2, 8, 1, 1, 0, 32, 1, 1, 0, 2, 1, 1, 32,
                                      1, kernels.MLS_F16, 16, 16, 64, NULL) == kernels.MLS_ERR_ARG
    # empty problems are no-ops
    assert L.mls_int4_grouped_gate_up(NULL, bf, 64, NULL, 2, 0, NULL, NULL, 0, 32, NULL, NULL, 0, 2, 1, 1,
                                      32, NULL, bf, 16, 16, 64, NULL) == 0
    # combine: k < 1, ldo < D, null pos, splits < 1, overlapping splits, empty
    assert L.mls_moe_combine(1, bf, 8, 4, 1, 0, 1, bf, 1, 2, 0, 1, bf, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(1, bf, 8, 4, 1, 0, 1, bf, 1, 2, 2, 1, bf, 4, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(1, bf, 8, 4, 1, 0, 1, bf, NULL, 2, 2, 1, bf, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(1, bf, 8, 4, 0, 0, 1, bf, 1, 2, 2, 1, bf, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(1, bf, 8, 4, 2, 16, 1, bf, 1, 2, 2, 1, bf, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(NULL, bf, 8, 0, 1, 0, NULL, bf, NULL, 0, 2, NULL, bf, 8, 8, NULL) == 0
    # fp64 rows need an fp64 output, and an fp64 output needs fp64 rows; unknown codes fail
    f64, f32 = kernels.MLS_F64, kernels.MLS_F32
    assert L.mls_moe_combine(1, f64, 8, 4, 1, 0, 1, f64, 1, 2, 2, 1, f32, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(1, f32, 8, 4, 1, 0, 1, f64, 1, 2, 2, 1, f64, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(1, 4, 8, 4, 1, 0, 1, f32, 1, 2, 2, 1, f32, 8, 8, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_moe_combine(NULL, f64, 8, 0, 1, 0, NULL, f64, NULL, 0, 2, NULL, f64, 8, 8, NULL) == 0
    # split count: the down projection of config E's expert MLP splits K in 4; a wide output does not
    assert L.mls_int4_grouped_splits(1024, 8, 4096, 14336, 128) == 4
    assert L.mls_int4_grouped_splits(1024, 8, 14336, 4096, 128) == 1


def test_fp8_train_entry_points_reject():
    L = kernels.load_library()
    # unknown flag bit
    assert L.mls_fp8_gemm(1, 64, 1, 64, 1.0, NULL, 0, 1.0, NULL, 0, 1, 0, 8, 4, 8, 64, 8, NULL) == \
        kernels.MLS_ERR_ARG
    assert L.mls_e5m2_encode(1, 5, 2, 2, 2, 1.0, NULL, 0, 1, 2, NULL) == kernels.MLS_ERR_ARG
    assert L.mls_e5m2_encode(1, 0, 2, 4, 2, 1.0, NULL, 0, 1, 4, NULL) == kernels.MLS_ERR_ARG   # ldx < cols
    assert L.mls_e5m2_encode_t(1, 0, 4, 8, 8, 1.0, NULL, 0, 1, 8, 1, 3, NULL) == kernels.MLS_ERR_ARG  # ldt < rows
    assert L.mls_e5m2_encode_t(1, 0, 4, 8, 8, 1.0, NULL, 0, 1, 8, NULL, 4, NULL) == kernels.MLS_ERR_ARG  # no out_t
    assert L.mls_e5m2_encode_t(NULL, 0, 0, 8, 8, 1.0, NULL, 0, NULL, 8, NULL, 0, NULL) == 0
    assert L.mls_e4m3_encode_t(1, 0, 4, 8, 8, 1.0, NULL, 0, 1, 8, 1, 3, NULL) == kernels.MLS_ERR_ARG  # ldt < rows
    assert L.mls_e4m3_encode_t(1, 7, 4, 8, 8, 1.0, NULL, 0, 1, 8, 1, 4, NULL) == kernels.MLS_ERR_ARG  # x dtype
    assert L.mls_transpose_u8(1, 4, 8, 4, 1, 4, NULL) == kernels.MLS_ERR_ARG                  # lds < cols
    assert L.mls_transpose_u8(1, 4, 8, 8, 1, 3, NULL) == kernels.MLS_ERR_ARG                  # ldd < rows
    assert L.mls_transpose_u8(NULL, 0, 8, 8, NULL, 0, NULL) == 0


def test_paged_attention_rejects_and_sizes_workspace():
    L = kernels.load_library()
    f32 = kernels.MLS_F32
    # no workspace needed for many (sequence, head) pairs; a split needs n*H*s*(D+2)
    assert L.mls_paged_attention_workspace(128, 32, 128, 128) == 0
    w = L.mls_paged_attention_workspace(1, 2, 64, 313)
    assert w > 0 and w % (2 * 66) == 0
    args = dict(q=1, qdt=f32, qss=64, qsh=32, k=1, v=1, kvdt=f32, sb=512, sh=256, st=32, nb=4, bt=1, btss=2,
                mb=2, ctx=1, out=1, oss=64, osh=32, n=1, H=2, D=32, bs=8, scale=1.0, ws=NULL, wsn=0)

    def call(**kw):
        a = dict(args, **kw)
        return L.mls_paged_attention_decode(a["q"], a["qdt"], a["qss"], a["qsh"], a["k"], a["v"], a["kvdt"],
                                            a["sb"], a["sh"], a["st"], a["nb"], a["bt"], a["btss"], a["mb"],
                                            a["ctx"], a["out"], a["oss"], a["osh"], a["n"], a["H"], a["D"],
                                            a["bs"], a["scale"], a["ws"], a["wsn"], NULL)

    assert call(bs=0) == kernels.MLS_ERR_ARG
    assert call(qdt=9) == kernels.MLS_ERR_ARG
    assert call(ctx=NULL) == kernels.MLS_ERR_ARG
    assert call(st=16) == kernels.MLS_ERR_ARG                 # row stride below D
    assert call(btss=1) == kernels.MLS_ERR_ARG                # table rows overlap
    assert call(n=0) == 0
