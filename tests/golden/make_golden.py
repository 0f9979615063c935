"""Writes the golden fixtures under tests/golden/ (run once; outputs are committed).

    python tests/golden/make_golden.py

Expected values come from PyTorch's CPU ops applied in the order the reference
applies them (serve/quantize.py:18-36, kernels/fp8_matmul.py:103-110,
train/model.py:158-162, kernels/moe_routing.py:116-130, and the tests'
dequantize-then-fp32-matmul oracles, test_quantize.py:37, 48 and
test_fp8.py:47). torch is the library the reference computes with, so these
vectors pin the numpy oracle to the reference's semantics without importing the
reference. Inputs are seeded; every array is stored, so replaying a fixture
needs neither torch's RNG nor this script.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
E4M3_MAX = 448.0


def t_quantize_int8(w):
    scale = (w.abs().amax(dim=1) / 127.0).clamp(min=1e-8)
    w_q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return w_q, scale


def t_quantize_int4(w, gs):
    N, K = w.shape
    g = w.reshape(N, K // gs, gs)
    scale = (g.abs().amax(dim=2) / 7.0).clamp(min=1e-8)
    q = (torch.round(g / scale[:, :, None]).clamp(-8, 7) + 8).reshape(N, K).to(torch.uint8)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous(), scale


def t_dequant_int4(packed, scale, gs):
    N, K = packed.shape[0], packed.shape[1] * 2
    q = torch.empty(N, K, dtype=torch.uint8)
    q[:, 0::2] = packed & 0x0F
    q[:, 1::2] = packed >> 4
    return ((q.float() - 8.0).reshape(N, K // gs, gs) * scale[:, :, None]).reshape(N, K)


def t_quantize_e4m3(x, scale):
    return (x.float() / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def e4m3_boundary_inputs() -> np.ndarray:
    """Every finite e4m3 magnitude, the midpoints between neighbours, each +-1 and
    +-2 fp32 ulp, both signs, plus specials and values beyond the clamp."""
    vals = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    vals = vals.astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2.0
    base = np.concatenate([vals, mids, [464.0, 480.0, 448.0 * 1.0001, 1e4, 3e38]]).astype(np.float32)
    bits = base.view(np.uint32).astype(np.int64)
    around = np.concatenate([bits + d for d in (-2, -1, 0, 1, 2)])
    around = around[(around >= 0) & (around < 0x7F800000)].astype(np.uint32).view(np.float32)
    specials = np.array([0.0, np.inf, np.nan, 1e-45, 2.0 ** -10, 2.0 ** -9 * 0.5], dtype=np.float32)
    pos = np.concatenate([around, specials])
    return np.concatenate([pos, -pos]).astype(np.float32)


def main() -> None:
    g = torch.Generator().manual_seed(0)

    # e4m3 decode KAT (test_fp8.py:16-26): torch's view of all 256 bytes
    bits = torch.arange(256, dtype=torch.uint8)
    np.savez_compressed(HERE / "e4m3_decode_kat.npz", bits=bits.numpy(),
                        value=bits.view(torch.float8_e4m3fn).float().numpy())

    # e4m3 encode: boundaries + random spread of magnitudes; scale 1 and a real scale
    xb = torch.from_numpy(e4m3_boundary_inputs())
    xr = torch.randn(200_000, generator=g) * torch.exp2(torch.randint(-24, 12, (200_000,), generator=g).float())
    xs = torch.randn(4096, generator=g) * 3
    s_real = float(xs.abs().amax()) / E4M3_MAX
    rows = torch.randn(64, 96, generator=g)
    rows[5] *= 1e-3
    rows[7] = 0.0
    s_rows = rows.abs().amax(dim=1, keepdim=True) / E4M3_MAX
    s_rows[7] = 1.0
    np.savez_compressed(
        HERE / "e4m3_encode.npz",
        x_boundary=xb.numpy(), q_boundary=t_quantize_e4m3(xb, 1.0).numpy(),
        x_random=xr.numpy(), q_random=t_quantize_e4m3(xr, 1.0).numpy(),
        x_scaled=xs.numpy(), scale=np.float64(s_real), q_scaled=t_quantize_e4m3(xs, s_real).numpy(),
        x_rows=rows.numpy(), s_rows=s_rows.numpy(), q_rows=t_quantize_e4m3(rows, s_rows).numpy(),
        dq_scaled=(t_quantize_e4m3(xs, s_real).view(torch.float8_e4m3fn).float() * s_real).numpy())

    # INT8 quantizer: random rows, an all-zero row, a row with exact .5 ties
    w8 = torch.randn(64, 512, generator=g) * 0.02
    w8[3] = 0.0
    w8[9] = torch.arange(512, dtype=torch.float32) - 255.5       # amax 255.5 -> k/2 ties
    w8[10, :4] = torch.tensor([127.0, 0.5, -0.5, 1.5])
    w8[10, 4:] = 0.0
    q8, s8 = t_quantize_int8(w8)
    np.savez_compressed(HERE / "quant_int8.npz", w=w8.numpy(), w_q=q8.numpy(), scale=s8.numpy())

    # INT4 quantizer at several group sizes, with a zero group and tie values
    out = {}
    for gs in (16, 32, 64, 128):
        w4 = torch.randn(32, 256, generator=g) * 0.02
        w4[2, :gs] = 0.0
        w4[4, :gs] = (torch.arange(gs, dtype=torch.float32) % 15 - 7) / 2.0
        p4, s4 = t_quantize_int4(w4, gs)
        out[f"w_g{gs}"], out[f"packed_g{gs}"], out[f"scale_g{gs}"] = w4.numpy(), p4.numpy(), s4.numpy()
    np.savez_compressed(HERE / "quant_int4.npz", **out)

    # config A: INT8, x fp32 [8, 512], W ~ N(0, 0.02) [2048, 512], seed 0
    ga = torch.Generator().manual_seed(0)
    xa = torch.randn(8, 512, generator=ga)
    wa = torch.randn(2048, 512, generator=ga) * 0.02
    qa, sa = t_quantize_int8(wa)
    ya = xa @ (qa.float() * sa[:, None]).t()
    np.savez_compressed(HERE / "gemm_int8_config_a.npz", x=xa.numpy(), w_q=qa.numpy(),
                        scale=sa.numpy(), y=ya.numpy())

    # INT4 GEMM at a reference test shape (test_quantize.py:40-49) plus a g128 case
    cases = {}
    for name, (M, N, K, gs) in {"t1": (4, 32, 64, 16), "t2": (9, 33, 32, 16), "t3": (1, 16, 64, 32),
                                "g128": (3, 40, 512, 128)}.items():
        a = torch.randn(M, K, generator=g)
        w = torch.randn(N, K, generator=g)
        p, s = t_quantize_int4(w, gs)
        cases[f"{name}_a"], cases[f"{name}_packed"], cases[f"{name}_scale"] = a.numpy(), p.numpy(), s.numpy()
        cases[f"{name}_gs"] = np.int64(gs)
        cases[f"{name}_y"] = (a @ t_dequant_int4(p, s, gs).t()).numpy()
    np.savez_compressed(HERE / "gemm_int4_small.npz", **cases)

    # FP8 GEMM at the reference test shapes (test_fp8.py:39-48)
    cases = {}
    for name, (M, N, K) in {"t1": (8, 16, 32), "t2": (17, 33, 48), "t3": (1, 16, 16)}.items():
        a = torch.randn(M, K, generator=g)
        b = torch.randn(N, K, generator=g)
        sa_ = float(a.abs().amax()) / E4M3_MAX
        sb_ = float(b.abs().amax()) / E4M3_MAX
        ab, bb = t_quantize_e4m3(a, sa_), t_quantize_e4m3(b, sb_)
        y = (ab.view(torch.float8_e4m3fn).float() * sa_) @ (bb.view(torch.float8_e4m3fn).float() * sb_).t()
        cases.update({f"{name}_a": ab.numpy(), f"{name}_b": bb.numpy(), f"{name}_sa": np.float64(sa_),
                      f"{name}_sb": np.float64(sb_), f"{name}_y": y.numpy()})
    np.savez_compressed(HERE / "fp8_small.npz", **cases)

    # routing (train/model.py:158-162, kernels/moe_routing.py:116-130)
    logits = torch.randn(64, 8, generator=g)
    probs = torch.softmax(logits.float(), dim=-1)
    wts, ex = torch.topk(probs, 2, dim=-1)
    wts = wts / wts.sum(dim=-1, keepdim=True)
    flat = ex.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=8)
    inv = torch.empty_like(order)
    inv[order] = torch.arange(flat.numel())
    np.savez_compressed(HERE / "route_small.npz", logits=logits.numpy(), weights=wts.numpy(),
                        experts=ex.numpy(), token_of_slot=(order // 2).numpy(),
                        counts=counts.numpy(), pos=inv.reshape(64, 2).numpy())
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
