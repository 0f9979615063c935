"""Host-side behaviour of the drop-in modules (no GPU): kernel entry points refuse
host tensors instead of computing elsewhere, the load-time quantizers and the
use_kernel=False paths match the oracle, and the module surface matches the
reference's."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from conftest import golden
from oracle import ref

from kernels.dequant_matmul import int4_matmul, int8_dgrad, int8_matmul
from kernels.fp8_matmul import E4M3_MAX, decode_e4m3, dequantize_e4m3, fp8_matmul, quantize_e4m3
from kernels.moe_grouped import int4_grouped_gate_up, int4_grouped_matmul
from kernels.moe_routing import combine_rows, moe_dispatch_combine
from serve.quantize import (QuantLinear, dequantize_int4, dequantize_int8, model_weight_bytes,
                            quantize_int4, quantize_int8, quantize_model)


def test_kernel_entry_points_refuse_host_tensors():
    a = torch.randn(2, 64)
    w8, s8 = quantize_int8(torch.randn(16, 64))
    w4, s4 = quantize_int4(torch.randn(16, 64), 32)
    with pytest.raises(TypeError, match="HIP device"):
        int8_matmul(a, w8, s8)
    with pytest.raises(TypeError, match="HIP device"):
        int4_matmul(a, w4, s4, 32)
    with pytest.raises(TypeError, match="HIP device"):
        int8_dgrad(torch.randn(2, 16), w8, s8)
    with pytest.raises(TypeError, match="HIP device"):
        decode_e4m3(torch.arange(256, dtype=torch.uint8))
    bits = quantize_e4m3(a, 0.01)
    with pytest.raises(TypeError, match="HIP device"):
        fp8_matmul(bits, bits, 0.01, 0.01)
    with pytest.raises(TypeError, match="HIP device"):
        int4_grouped_matmul(a.bfloat16(), w4[None], s4[None], torch.tensor([2]), 32)
    with pytest.raises(TypeError, match="HIP device"):
        int4_grouped_gate_up(a.bfloat16(), w4[None], s4[None], w4[None], s4[None], torch.tensor([2]), 32)
    with pytest.raises(TypeError, match="HIP device"):
        combine_rows(torch.randn(4, 8), torch.rand(2, 2), torch.arange(4).reshape(2, 2))
    from kernels.paged_attention import paged_attention_decode
    with pytest.raises(TypeError, match="HIP device"):
        paged_attention_decode(torch.randn(1, 2, 16), torch.randn(4, 2, 8, 16), torch.randn(4, 2, 8, 16),
                               torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))
    # the routed MoE forward has no host path either: its combine is the HIP kernel
    experts = [nn.Linear(64, 64, bias=False) for _ in range(2)]
    with pytest.raises(TypeError, match="HIP device"):
        moe_dispatch_combine(a, torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.long), experts)


def test_int4_matmul_keeps_reference_assert():
    with pytest.raises(AssertionError):
        int4_matmul(torch.randn(2, 64), torch.zeros(4, 16, dtype=torch.uint8),
                    torch.ones(4, 2), 32)


def test_host_quantizers_match_oracle():
    d = golden("quant_int8")
    q, s = quantize_int8(torch.from_numpy(d["w"]))
    assert np.array_equal(q.numpy(), d["w_q"]) and np.array_equal(s.numpy(), d["scale"])
    d = golden("quant_int4")
    for gs in (16, 32, 64, 128):
        p, s = quantize_int4(torch.from_numpy(d[f"w_g{gs}"]), gs)
        assert np.array_equal(p.numpy(), d[f"packed_g{gs}"])
        assert np.array_equal(s.numpy(), d[f"scale_g{gs}"])
    e = golden("e4m3_encode")
    assert np.array_equal(quantize_e4m3(torch.from_numpy(e["x_rows"]),
                                        torch.from_numpy(e["s_rows"])).numpy(), e["q_rows"])


def test_host_dequantizers_match_oracle():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(24, 96, generator=g)
    q, s = quantize_int8(w)
    assert np.array_equal(dequantize_int8(q, s).numpy(), ref.dequantize_int8(q.numpy(), s.numpy()))
    p, s = quantize_int4(w, 32)
    assert np.array_equal(dequantize_int4(p, s, 32).numpy(),
                          ref.dequantize_int4(p.numpy(), s.numpy(), 32))
    bits = torch.arange(256, dtype=torch.uint8)
    assert np.array_equal(dequantize_e4m3(bits, 0.5).numpy(),
                          ref.dequantize_e4m3(bits.numpy(), 0.5), equal_nan=True)


def test_quantlinear_reference_path_on_host():
    """test_quantize.py:52-58 shape: QuantLinear(use_kernel=False) equals x @ dequant(W)^T."""
    lin = nn.Linear(48, 32, bias=False)
    x = torch.randn(2, 7, 48)
    for bits in (8, 4):
        ql = QuantLinear(lin, bits=bits, group_size=16, use_kernel=False)
        y = ql(x)
        assert y.shape == (2, 7, 32)
        wq, sc = ql.w_q.numpy(), ql.scale.numpy()
        want = ref.int8_matmul(x.reshape(-1, 48).numpy(), wq, sc) if bits == 8 else \
            ref.int4_matmul(x.reshape(-1, 48).numpy(), wq, sc, 16)
        assert np.allclose(y.reshape(-1, 32).detach().numpy(), want, rtol=1e-5, atol=1e-5)
        assert ql.weight_bytes() == wq.nbytes + sc.nbytes
    with pytest.raises(AssertionError):
        QuantLinear(nn.Linear(4, 4, bias=True))
    with pytest.raises(AssertionError):
        QuantLinear(nn.Linear(4, 4, bias=False), bits=3)


class _Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.wq, self.wk, self.wv, self.wo = (nn.Linear(d, d, bias=False) for _ in range(4))


class _MLP(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.w_gate, self.w_up = nn.Linear(d, h, bias=False), nn.Linear(d, h, bias=False)
        self.w_down = nn.Linear(h, d, bias=False)


class _MoE(nn.Module):
    def __init__(self, d, h, e):
        super().__init__()
        self.router = nn.Linear(d, e, bias=False)
        self.experts = nn.ModuleList(_MLP(d, h) for _ in range(e))


class _Block(nn.Module):
    def __init__(self, d, h, moe):
        super().__init__()
        self.attn = _Attn(d)
        self.is_moe = moe
        self.mlp = _MoE(d, h, 2) if moe else _MLP(d, h)


class _Model(nn.Module):
    def __init__(self, d=64, h=128):
        super().__init__()
        self.embed = nn.Embedding(32, d)
        self.blocks = nn.ModuleList([_Block(d, h, False), _Block(d, h, True)])


def test_quantize_model_swaps_every_block_linear():
    """serve/quantize.py:98-115: attention and (expert) MLP linears become QuantLinear,
    the router and embeddings stay fp; memory shrinks (test_quantize.py:88-97)."""
    m = _Model()
    q8 = quantize_model(m, bits=8, use_kernel=False)
    q4 = quantize_model(m, bits=4, use_kernel=False)
    n_q = sum(isinstance(x, QuantLinear) for x in q8.modules())
    assert n_q == 4 + 3 + 4 + 3 * 2
    assert isinstance(q8.blocks[1].mlp.router, nn.Linear)
    assert isinstance(m.blocks[0].attn.wq, nn.Linear)          # original untouched
    fp = model_weight_bytes(m)
    assert model_weight_bytes(q8) < fp * 0.5 and model_weight_bytes(q4) < model_weight_bytes(q8)


def test_moe_experts_on_host_are_not_stacked():
    """The grouped INT4 expert path needs device buffers; host-quantized experts (the
    reference CLI quantizes before moving to the GPU) are stacked later, on the device."""
    from serve.quantize import stacked_int4_experts
    q4 = quantize_model(_Model(), bits=4, use_kernel=True)
    experts = q4.blocks[1].mlp.experts
    assert stacked_int4_experts(experts) is None
    assert experts[0].__dict__.get("_int4_stack") is None


def test_fp8_linear_emulation_on_host():
    """train/fp8.py: FP8Linear(use_kernel=False) forward equals the decoded-operand matmul."""
    from train.fp8 import DynamicScaler, FP8Linear
    torch.manual_seed(1)
    lin = nn.Linear(16, 12, bias=False)
    f = FP8Linear(lin)
    x = torch.randn(5, 16)
    y = f(x)
    sx = DynamicScaler().scale_for(x)
    sw = DynamicScaler().scale_for(lin.weight)
    xb = ref.quantize_e4m3(x.numpy(), sx)
    wb = ref.quantize_e4m3(lin.weight.detach().numpy(), sw)
    want = ref.dequantize_e4m3(xb, sx) @ ref.dequantize_e4m3(wb, sw).T
    assert np.allclose(y.detach().numpy(), want, rtol=1e-5, atol=1e-6)
    assert E4M3_MAX == 448.0


def test_scale1_underflows_small_values():
    """test_fp8.py:51-59 of the reference, on the host codec: gradient-sized values flush
    to zero at scale 1.0 and survive at the amax scale (what dynamic scaling is for)."""
    torch.manual_seed(0)
    g = torch.randn(1000) * 1e-4
    dead = dequantize_e4m3(quantize_e4m3(g, 1.0), 1.0)
    s = float(g.abs().amax()) / E4M3_MAX
    alive = dequantize_e4m3(quantize_e4m3(g, s), s)
    assert (dead == 0).float().mean() > 0.5
    assert (alive == 0).float().mean() < 0.01


def test_delayed_scaler_tracks_amax():
    """test_fp8.py:62-71 of the reference: the first call uses the just-in-time amax, later
    calls the amax history, which forgets after `history` calls."""
    from train.fp8 import DynamicScaler
    s = DynamicScaler(history=4)
    t = torch.ones(10)
    assert abs(s.scale_for(t * 448) - 1.0) < 1e-6
    assert abs(s.scale_for(t) - 1.0) < 1e-6
    for _ in range(4):
        s.scale_for(t)
    assert s.scale_for(t) < 0.01


# ------------------------------------------------------------------ quantized checkpoints


@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_checkpoint_roundtrip_host(tmp_path, bits):
    """save_quantized / load_quantized: the loaded model holds bit-identical QuantLinear
    buffers and fp parameters, without running the quantizer again."""
    from serve.quantize import load_quantized, read_quantized_metadata, save_quantized
    torch.manual_seed(1)
    m = _Model()
    q = quantize_model(m, bits=bits, group_size=32, use_kernel=False)
    path = tmp_path / "q.safetensors"
    save_quantized(q, path, extra_metadata={"vocab": "abc"})
    meta = read_quantized_metadata(path)
    assert meta["vocab"] == "abc" and sum(k.startswith("q:") for k in meta) == 4 + 3 + 4 + 3 * 2
    assert meta["q:blocks.0.attn.wq"] == f"{bits},32,64"
    torch.manual_seed(2)                     # a different random init: everything must load
    loaded = load_quantized(_Model(), path, use_kernel=False)
    sq, sl = q.state_dict(), loaded.state_dict()
    assert sq.keys() == sl.keys()
    for k in sq:
        assert sq[k].dtype == sl[k].dtype and torch.equal(sq[k], sl[k]), k
    for a, b in zip(q.modules(), loaded.modules()):
        assert type(a) is type(b)
        if isinstance(a, QuantLinear):
            assert (a.bits, a.group_size, a.in_features, a.out_features) == \
                (b.bits, b.group_size, b.in_features, b.out_features)
    assert model_weight_bytes(loaded) == model_weight_bytes(q)
    x = torch.randn(3, 64)
    assert torch.equal(loaded.blocks[0].attn.wq(x), q.blocks[0].attn.wq(x))
    # the file holds the quantized weights, not fp copies
    fp_bytes = sum(v.numel() * v.element_size() for v in m.state_dict().values())
    assert path.stat().st_size < fp_bytes * (0.5 if bits == 8 else 0.3)


def test_quantized_checkpoint_rejects(tmp_path):
    from safetensors.torch import save_file
    from serve.quantize import load_quantized, save_quantized
    with pytest.raises(ValueError, match="no QuantLinear"):
        save_quantized(_Model(), tmp_path / "fp.safetensors")
    q = quantize_model(_Model(), bits=4, use_kernel=False)
    path = tmp_path / "q.safetensors"
    save_quantized(q, path)
    with pytest.raises(ValueError, match="stores"):
        load_quantized(_Model(d=64, h=192), path, use_kernel=False)     # hidden size differs
    with pytest.raises(ValueError, match="reserved"):
        save_quantized(q, path, extra_metadata={"format": "x"})
    other = tmp_path / "other.safetensors"
    save_file({"a": torch.zeros(2)}, str(other), metadata={"format": "mls-quantized", "version": "0"})
    with pytest.raises(ValueError, match="version"):
        load_quantized(_Model(), other)
    save_file({"a": torch.zeros(2)}, str(other), metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a quantized checkpoint"):
        load_quantized(_Model(), other)
