"""The Python drop-in: this package placed ahead of a reference checkout on sys.path.

The build provides only the quantized-linear modules (kernels.dequant_matmul,
kernels.fp8_matmul, kernels.moe_routing, kernels.paged_attention, serve.quantize,
train.fp8). The reference's engine, model and autograd modules import each other
through the same package names (reference serve/engine.py:30-31, 95, 142;
train/model.py:110-114, 167-171; kernels/autograd_ops.py:15-19, 129), so with the
build first on the path they must still resolve from the checkout and bind the
build's GEMMs.

The checkout here is a stub tree written into tmp_path (module names and import
lines shaped like the reference's; the reference itself is not read or run). Each
case runs in a fresh interpreter because this process already imported `kernels`.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
import textwrap

from conftest import PKG

STUBS = {
    # the checkout's package inits never run: the build's come first and extend the path
    "kernels/__init__.py": "raise RuntimeError('checkout kernels/__init__ ran')\n",
    "serve/__init__.py": "raise RuntimeError('checkout serve/__init__ ran')\n",
    "train/__init__.py": "raise RuntimeError('checkout train/__init__ ran')\n",
    # modules the build replaces: must be shadowed
    "kernels/dequant_matmul.py": "ORIGIN = 'checkout'\n",
    "kernels/fp8_matmul.py": "ORIGIN = 'checkout'\n",
    "kernels/moe_routing.py": "ORIGIN = 'checkout'\n",
    "kernels/paged_attention.py": "ORIGIN = 'checkout'\n",
    "serve/quantize.py": "ORIGIN = 'checkout'\n",
    "train/fp8.py": "ORIGIN = 'checkout'\n",
    # modules the build does not provide: must come from the checkout
    "kernels/attention_fwd.py": """
        import kernels  # noqa: F401
        ORIGIN = 'checkout'
        def flash_attention(q, k, v, causal=True, scale=None, return_lse=False):
            return q
    """,
    "kernels/attention_bwd.py": """
        import kernels  # noqa: F401
        ORIGIN = 'checkout'
        def flash_attention_backward(*a, **k):
            return None
    """,
    "kernels/moe_backward.py": """
        import kernels  # noqa: F401
        ORIGIN = 'checkout'
        def combine_backward(*a):
            return None
        def scatter_add_rows(*a):
            return None
    """,
    "kernels/autograd_ops.py": """
        from kernels.attention_bwd import flash_attention_backward
        from kernels.attention_fwd import flash_attention
        from kernels.dequant_matmul import int8_dgrad, int8_matmul
        from kernels.moe_backward import combine_backward, scatter_add_rows
        from kernels.moe_routing import combine_rows, gather_rows, sort_by_expert
        ORIGIN = 'checkout'
        def flash_attention_train(q, k, v, causal=True, scale=None):
            return flash_attention(q, k, v, causal, scale)
        def moe_dispatch_combine_train(*a):
            return None
        class QuantLinearSTE:
            def quantizer(self):
                from serve.quantize import quantize_int8
                return quantize_int8
    """,
    "serve/kv_cache.py": "ORIGIN = 'checkout'\nclass PagedKVCache:\n    pass\n",
    "serve/engine.py": """
        from serve.kv_cache import PagedKVCache
        from train.model import Transformer, naive_attention
        ORIGIN = 'checkout'
        def decode_kernel():
            from kernels.paged_attention import paged_attention_decode
            return paged_attention_decode
    """,
    "train/config.py": "ORIGIN = 'checkout'\nclass ModelConfig:\n    pass\n",
    "train/model.py": """
        from train.config import ModelConfig
        ORIGIN = 'checkout'
        class Transformer:
            pass
        def naive_attention(*a):
            return None
        def train_kernels():
            from kernels.autograd_ops import flash_attention_train, moe_dispatch_combine_train
            from kernels.moe_routing import moe_dispatch_combine
            return flash_attention_train, moe_dispatch_combine_train, moe_dispatch_combine
    """,
}

PROBE = """
import importlib, json, sys
out = {}
for name in sys.argv[1:]:
    m = importlib.import_module(name)
    out[name] = m.__file__
import kernels, kernels.autograd_ops as ao, kernels.dequant_matmul as dq, kernels.moe_routing as mr
import serve.engine as eng, serve.quantize as sq, train.model as tm
out["ste_binds_build_gemm"] = ao.int8_matmul is dq.int8_matmul and ao.int8_dgrad is dq.int8_dgrad
out["autograd_binds_build_routing"] = ao.gather_rows is mr.gather_rows and ao.combine_rows is mr.combine_rows
out["ste_quantizer_is_build"] = ao.QuantLinearSTE().quantizer() is sq.quantize_int8
out["engine_decode_is_build"] = eng.decode_kernel().__module__
fa, mdt, mdc = tm.train_kernels()
out["model_kernels"] = [fa.__module__, mdt.__module__, mdc.__module__]
out["interpreter"] = kernels.INTERPRETER
print(json.dumps(out))
"""

BUILD_MODULES = ["kernels.dequant_matmul", "kernels.fp8_matmul", "kernels.moe_routing",
                 "kernels.paged_attention", "kernels.moe_grouped", "kernels.int8_ste",
                 "serve.quantize", "train.fp8"]
CHECKOUT_MODULES = ["kernels.attention_fwd", "kernels.attention_bwd", "kernels.moe_backward",
                    "kernels.autograd_ops", "serve.kv_cache", "serve.engine", "train.model",
                    "train.config"]


def _write_checkout(root):
    for rel, text in STUBS.items():
        f = root / rel
        f.parent.mkdir(parents=True, exist_ok=True)
        f.write_text(textwrap.dedent(text).lstrip())


def _probe(pythonpath, modules):
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(str(p) for p in pythonpath))
    r = subprocess.run([sys.executable, "-c", PROBE, *modules], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_reference_modules_resolve_through_the_overlay(tmp_path):
    checkout = tmp_path / "checkout"
    _write_checkout(checkout)
    out = _probe([PKG, checkout], BUILD_MODULES + CHECKOUT_MODULES)
    for name in BUILD_MODULES:
        assert out[name].startswith(str(PKG)), (name, out[name])
    for name in CHECKOUT_MODULES:
        assert out[name].startswith(str(checkout)), (name, out[name])
    assert out["ste_binds_build_gemm"] and out["autograd_binds_build_routing"]
    assert out["ste_quantizer_is_build"]
    assert out["engine_decode_is_build"] == "kernels.paged_attention"
    assert out["model_kernels"] == ["kernels.autograd_ops", "kernels.autograd_ops", "kernels.moe_routing"]
    assert out["interpreter"] is False


def test_build_alone_has_no_autograd_ops_module(tmp_path):
    """Without a checkout the build does not pretend to provide the reference's
    attention / MoE autograd module; its INT8 STE lives in kernels.int8_ste."""
    env = dict(os.environ, PYTHONPATH=str(PKG))
    code = ("import importlib.util as u, json; print(json.dumps([u.find_spec(n) is not None for n in "
            "('kernels.autograd_ops', 'kernels.int8_ste', 'serve.engine', 'train.model')]))")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300, cwd=tmp_path)
    assert r.returncode == 0, r.stderr[-3000:]
    assert json.loads(r.stdout.strip().splitlines()[-1]) == [False, True, False, False]
