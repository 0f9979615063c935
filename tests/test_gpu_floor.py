"""bench.py's timing-only kernel copies (libmls_floor.so, not the product): the clocked
copies of the M = 1 GEMV run the library's kernel body and must give the library's
output bit for bit, and every wavefront of a clocked launch must leave an ordered pair
of clocks. bench.py splits the headline step into execution and launch from them."""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import PKG

pytestmark = pytest.mark.gpu


def _floor():
    lib = ctypes.CDLL(str(PKG / "libmls_floor.so"))
    lib.mlsf_gemv1_clocked.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mlsf_empty_clocked.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mlsf_stream_clocked.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _ordered(clk):
    c = clk.cpu()
    return bool((c[:, 0] > 0).all()) and bool((c[:, 1] >= c[:, 0]).all())


@pytest.mark.parametrize("wait", [0, 1])
@pytest.mark.parametrize("bits,N", [(4, 4096), (8, 4096), (4, 1000), (8, 1001)])
def test_clocked_gemv_matches_library(dev, bits, N, wait):
    from kernels.dequant_matmul import int4_matmul, int8_matmul
    from serve.quantize import quantize_int4, quantize_int8
    K = 4096
    g = torch.Generator(device=dev).manual_seed(bits + N)
    x = torch.randn(1, K, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    if bits == 4:
        q, s = quantize_int4(w, 128)
        s = s.to(torch.float16)
        want = int4_matmul(x, q, s, 128)
        ld_sn, group, waves = s.stride(0), 128, 4 * ((N + 15) // 16)
    else:
        q, s = quantize_int8(w)
        s = s.to(torch.float16)
        want = int8_matmul(x, q, s)
        ld_sn, group, waves = 1, 0, 4 * ((N + 3) // 4)
    y = torch.full((1, N), float("nan"), dtype=torch.bfloat16, device=dev)
    clk = torch.zeros(waves, 2, dtype=torch.int64, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = _floor().mlsf_gemv1_clocked(bits, x.data_ptr(), q.data_ptr(), q.stride(0), s.data_ptr(), ld_sn, group,
                                     y.data_ptr(), N, K, wait, clk.data_ptr(), st)
    assert rc == waves
    assert torch.equal(y, want)
    assert _ordered(clk)


def test_clocked_floor_kernels_write_every_wave(dev):
    lib = _floor()
    st = torch.cuda.current_stream(dev).cuda_stream
    blocks = 256
    clk = torch.zeros(blocks * 4, 2, dtype=torch.int64, device=dev)
    assert lib.mlsf_empty_clocked(blocks, clk.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert _ordered(clk)
    buf = torch.randint(0, 2**31 - 1, (8_667_136 // 4,), device=dev, dtype=torch.int32)
    sink = torch.zeros(blocks * 8, dtype=torch.int32, device=dev)
    for store in (0, 1):
        for wait in (0, 1):
            clk.zero_()
            assert lib.mlsf_stream_clocked(buf.data_ptr(), 8_667_136, blocks, sink.data_ptr(), store, wait,
                                           clk.data_ptr(), st) == 0
            torch.cuda.synchronize()
            assert _ordered(clk)


def test_clocked_gemv_rejects_other_shapes():
    """Shapes the clocked copy was not instantiated for fail on the host, before a launch."""
    lib = _floor()
    assert lib.mlsf_gemv1_clocked(4, 1, 1, 2048, 1, 32, 64, 1, 4096, 4096, 0, 1, None) == -1   # group 64
    assert lib.mlsf_gemv1_clocked(4, 1, 1, 1024, 1, 16, 128, 1, 4096, 2048, 0, 1, None) == -1  # K 2048
    assert lib.mlsf_gemv1_clocked(2, 1, 1, 4096, 1, 1, 0, 1, 4096, 4096, 0, 1, None) == -1     # bits
