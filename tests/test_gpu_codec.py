"""gfx950 e4m3 codec and weight quantizers vs the CPU oracle: bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import ref

from kernels.fp8_matmul import decode_e4m3, dequantize_e4m3, quantize_e4m3
from serve.quantize import quantize_int4, quantize_int8

pytestmark = pytest.mark.gpu


def _bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def test_decode_kat(dev):
    bits = torch.arange(256, dtype=torch.uint8, device=dev)
    out = decode_e4m3(bits).cpu().numpy()
    assert np.array_equal(_bits(out), _bits(ref.e4m3_decode(np.arange(256, dtype=np.uint8))))


@pytest.mark.parametrize("n,offset", [(1 << 20, 0), (1000003, 0), (4099, 3)])
def test_decode_random(dev, n, offset):
    g = torch.Generator().manual_seed(n)
    host = torch.randint(0, 256, (n + offset,), dtype=torch.uint8, generator=g)
    bits = host.to(dev)[offset:]                   # offset 3: unaligned storage
    out = decode_e4m3(bits).cpu().numpy()
    assert np.array_equal(_bits(out), _bits(ref.e4m3_decode(host[offset:].numpy())))


@pytest.mark.parametrize("part", ["boundary", "random"])
def test_encode_golden(dev, part):
    e = golden("e4m3_encode")
    x = torch.from_numpy(e[f"x_{part}"]).to(dev)
    assert np.array_equal(quantize_e4m3(x, 1.0).cpu().numpy(), e[f"q_{part}"])


def test_encode_scaled_and_rows(dev):
    e = golden("e4m3_encode")
    xs = torch.from_numpy(e["x_scaled"]).to(dev)
    assert np.array_equal(quantize_e4m3(xs, float(e["scale"])).cpu().numpy(), e["q_scaled"])
    xr = torch.from_numpy(e["x_rows"]).to(dev)
    sr = torch.from_numpy(e["s_rows"]).to(dev)
    assert np.array_equal(quantize_e4m3(xr, sr).cpu().numpy(), e["q_rows"])
    s0 = torch.tensor(float(e["scale"]), dtype=torch.float32, device=dev)      # 0-d tensor
    assert np.array_equal(quantize_e4m3(xs, s0).cpu().numpy(),
                          ref.quantize_e4m3(e["x_scaled"], np.float32(e["scale"])))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_encode_16bit_inputs(dev, dtype):
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(300, 257, generator=g) * 40).to(dtype)
    s = 0.37
    want = ref.quantize_e4m3(x.float().numpy(), s)
    assert np.array_equal(quantize_e4m3(x.to(dev), s).cpu().numpy(), want)


def test_encode_general_broadcast(dev):
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4, 6, 32, generator=g) * 10
    s = torch.rand(32, generator=g) + 0.05                 # per column: general path
    want = ref.quantize_e4m3(x.numpy(), s.numpy())
    assert np.array_equal(quantize_e4m3(x.to(dev), s.to(dev)).cpu().numpy(), want)


def test_dequantize(dev):
    bits = torch.arange(256, dtype=torch.uint8).repeat(3, 1)
    s_rows = torch.tensor([[0.5], [3.0], [1e-3]])
    want = ref.dequantize_e4m3(bits.numpy(), s_rows.numpy())
    got = dequantize_e4m3(bits.to(dev), s_rows.to(dev)).cpu().numpy()
    assert np.array_equal(got, want, equal_nan=True)
    got = dequantize_e4m3(bits.to(dev), 0.125).cpu().numpy()
    assert np.array_equal(got, ref.dequantize_e4m3(bits.numpy(), 0.125), equal_nan=True)


def test_quantize_int8_golden_and_large(dev):
    d = golden("quant_int8")
    q, s = quantize_int8(torch.from_numpy(d["w"]).to(dev))
    assert np.array_equal(q.cpu().numpy(), d["w_q"])
    assert np.array_equal(_bits(s.cpu().numpy()), _bits(d["scale"]))
    g = torch.Generator().manual_seed(8)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    q, s = quantize_int8(w.to(dev))
    rq, rs = ref.quantize_int8(w.numpy())
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(_bits(s.cpu().numpy()), _bits(rs))


@pytest.mark.parametrize("gs", [16, 32, 64, 128])
def test_quantize_int4_golden(dev, gs):
    d = golden("quant_int4")
    p, s = quantize_int4(torch.from_numpy(d[f"w_g{gs}"]).to(dev), gs)
    assert np.array_equal(p.cpu().numpy(), d[f"packed_g{gs}"])
    assert np.array_equal(_bits(s.cpu().numpy()), _bits(d[f"scale_g{gs}"]))


def test_quantize_int4_large(dev):
    g = torch.Generator().manual_seed(9)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    p, s = quantize_int4(w.to(dev), 128)
    rp, rs = ref.quantize_int4(w.numpy(), 128)
    assert np.array_equal(p.cpu().numpy(), rp) and np.array_equal(_bits(s.cpu().numpy()), _bits(rs))


@pytest.mark.parametrize("N,K,gs,stride", [
    (64, 768, 256, 0),      # vector path, last 512-k span partial
    (33, 1024, 512, 0),     # one group per span
    (17, 96, 8, 0),         # one lane per group
    (40, 960, 96, 0),       # group not a power of two: generic path
    (12, 60, 6, 0),         # tiny odd-ish group: generic path
    (50, 512, 32, 3),       # rows not 16-byte aligned: generic path
])
def test_quantize_int4_paths(dev, N, K, gs, stride):
    """Both INT4 quantizer paths (one wavefront per 512-k span with shuffle-reduced
    group maxima; one thread per group) against the oracle, bit-exact, including
    all-zero groups and exact .5 ties."""
    g = torch.Generator().manual_seed(N * K + gs)
    full = torch.randn(N, K + stride, generator=g) * 0.05
    full[3, :gs] = 0.0                                       # an all-zero group
    full[5, :gs] = torch.arange(gs, dtype=torch.float32) * 0.5 - gs / 4   # ties at .5
    w = full[:, :K]
    p, s = quantize_int4(w.to(dev) if stride == 0 else full.to(dev)[:, :K], gs)
    rp, rs = ref.quantize_int4(w.contiguous().numpy(), gs)
    assert np.array_equal(p.cpu().numpy(), rp)
    assert np.array_equal(_bits(s.cpu().numpy()), _bits(rs))


@pytest.mark.parametrize("N,K,stride", [(70, 4100, 0), (9, 4098, 0), (31, 1000, 2)])
def test_quantize_int8_paths(dev, N, K, stride):
    g = torch.Generator().manual_seed(N + K)
    full = torch.randn(N, K + stride, generator=g) * 0.05
    full[2] = 0.0
    w = full[:, :K]
    q, s = quantize_int8(w.to(dev) if stride == 0 else full.to(dev)[:, :K])
    rq, rs = ref.quantize_int8(w.contiguous().numpy())
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(_bits(s.cpu().numpy()), _bits(rs))
