"""gfx950 (MI355X) quantized-linear kernels behind the reference's ``kernels`` API.

The reference's package of the same name selects the Triton interpreter when no
GPU is present (kernels/__init__.py:12-15). Here there is no interpreter and no
Triton: every kernel entry point calls the hand-written HIP library
``libmls_hip.so`` (C ABI in include/mls.h) through ctypes, on HIP device tensors
only. The library is bound on first use; if it is missing, or a CPU tensor
reaches a kernel entry point, the call raises instead of computing elsewhere.

Overlay. This package replaces only the reference's quantized-linear modules
(dequant_matmul, fp8_matmul, moe_routing, paged_attention). Its search path is
extended over every ``kernels`` directory on ``sys.path`` (pkgutil.extend_path),
so with this directory first and a reference checkout after it, the reference's
other modules (attention_fwd, attention_bwd, autograd_ops, moe_backward,
fusion_compiler) import from the checkout and bind this package's GEMMs. Both
roots must be on ``sys.path`` before the first ``import kernels``.
"""

from __future__ import annotations

import ctypes
import os
import pkgutil
from pathlib import Path

__path__ = pkgutil.extend_path(__path__, __name__)

import torch  # noqa: E402

# The reference's own Triton modules that this package does not replace read the
# interpreter switch set by the package import on a machine without a GPU
# (reference kernels/__init__.py:12-13); it is kept so that they behave as before.
# Nothing in this package uses Triton.
if not torch.cuda.is_available():
    os.environ.setdefault("TRITON_INTERPRET", "1")

# The reference exposes whether it runs interpreted (kernels/__init__.py:15).
# This implementation only ever runs compiled gfx950 code.
INTERPRETER = False

ABI_VERSION = 7
LIB_PATH = Path(os.environ.get("MLS_LIB") or
                Path(__file__).resolve().parent.parent / "libmls_hip.so")

MLS_F32, MLS_F16, MLS_BF16 = 0, 1, 2
MLS_F64 = 3  # mls_moe_combine only
MLS_OK, MLS_ERR_ARG, MLS_ERR_UNSUPPORTED, MLS_ERR_HIP = 0, -1, -2, -3
MLS_FP8_NATIVE = 1
MLS_FP8_A_E5M2 = 2

_LIB = None

_P, _I, _I64, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# argument types of every exported entry point, in include/mls.h order
SIGNATURES = {
    "mls_abi_version": ([], _I),
    "mls_last_error": ([], ctypes.c_char_p),
    "mls_e4m3_decode": ([_P, _P, _I64, _P], _I),
    "mls_e4m3_dequantize": ([_P, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _P], _I),
    "mls_e4m3_encode": ([_P, _I, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _P], _I),
    "mls_e5m2_encode": ([_P, _I, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _P], _I),
    "mls_e5m2_encode_t": ([_P, _I, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _P, _I64, _P], _I),
    "mls_e4m3_encode_t": ([_P, _I, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _P, _I64, _P], _I),
    "mls_transpose_u8": ([_P, _I64, _I64, _I64, _P, _I64, _P], _I),
    "mls_quantize_int8": ([_P, _I64, _I64, _I64, _P, _I64, _P, _P], _I),
    "mls_quantize_int4": ([_P, _I64, _I64, _I64, _I, _P, _I64, _P, _P], _I),
    "mls_int8_gemm": ([_P, _I, _I64, _P, _I64, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P], _I),
    "mls_int4_gemm": ([_P, _I, _I64, _P, _I64, _P, _I, _I64, _I64, _I, _P, _I, _I64,
                       _I64, _I64, _I64, _P], _I),
    "mls_wq_gemm_workspace": ([_I, _I64, _I64, _I64, _I, _I], _I64),
    "mls_int8_gemm_ws": ([_P, _I, _I64, _P, _I64, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "mls_int4_gemm_ws": ([_P, _I, _I64, _P, _I64, _P, _I, _I64, _I64, _I, _P, _I, _I64,
                          _I64, _I64, _I64, _P, _I64, _P], _I),
    "mls_int8_dgrad": ([_P, _I, _I64, _P, _I64, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P], _I),
    "mls_int8_dgrad_workspace": ([_I64, _I64, _I64, _I], _I64),
    "mls_int8_dgrad_ws": ([_P, _I, _I64, _P, _I64, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P],
                          _I),
    "mls_fp8_gemm": ([_P, _I64, _P, _I64, _F, _P, _I64, _F, _P, _I64, _P, _I, _I64,
                      _I64, _I64, _I64, _I, _P], _I),
    "mls_int4_grouped_gemm": ([_P, _I, _I64, _P, _I, _I64, _P, _I64, _I64, _P, _I, _I64,
                               _I64, _I64, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "mls_int4_grouped_gate_up": ([_P, _I, _I64, _P, _I, _I64, _P, _P, _I64, _I64, _P, _P, _I,
                                  _I64, _I64, _I64, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "mls_int4_grouped_gemm_rows": ([_P, _I, _I64, _P, _I64, _P, _I, _I64, _P, _I64, _I64, _P, _I, _I64,
                                    _I64, _I64, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "mls_int4_grouped_gate_up_rows": ([_P, _I, _I64, _P, _I64, _P, _I, _I64, _P, _P, _I64, _I64, _P, _P, _I,
                                       _I64, _I64, _I64, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "mls_moe_combine": ([_P, _I, _I64, _I64, _I, _I64, _P, _I, _P, _I64, _I, _P, _I, _I64, _I64, _P], _I),
    "mls_int4_grouped_splits": ([_I64, _I, _I64, _I64, _I], _I),
    "mls_int4_grouped_gemm_partial": ([_P, _I, _I64, _P, _I, _I64, _P, _I64, _I64, _P, _I, _I64, _I64, _I64,
                                       _I, _I, _P, _I64, _I64, _I64, _I64, _P], _I),
    "mls_paged_attention_workspace": ([_I64, _I64, _I64, _I64], _I64),
    "mls_paged_attention_decode": ([_P, _I, _I64, _I64, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _I64,
                                    _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I64, _P], _I),
    "mls_paged_attention_decode_noalloc": ([_P, _I, _I64, _I64, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64,
                                            _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P], _I),
}


class HipKernelError(RuntimeError):
    """A HIP kernel entry point returned an error status."""


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Binds libmls_hip.so (once). torch is imported first so that the library
    resolves the HIP runtime torch already loaded: one runtime per process, and
    torch's streams are valid in the library."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    import torch  # noqa: F401  (loads torch's libamdhip64 before ours binds to it)
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `python mini-llm-stack_amd/csrc/build.py` (the HIP kernels have no fallback)")
    lib = ctypes.CDLL(str(p))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res
    if lib.mls_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {lib.mls_abi_version()} != {ABI_VERSION}")
    if path is None:
        _LIB = lib
    return lib


def lib() -> ctypes.CDLL:
    return _LIB if _LIB is not None else load_library()


def check(rc: int, what: str) -> None:
    if rc == MLS_OK:
        return
    msg = lib().mls_last_error().decode(errors="replace")
    if rc == MLS_ERR_ARG:
        raise ValueError(f"{what}: {msg}")
    if rc == MLS_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise HipKernelError(f"{what}: {msg}")
