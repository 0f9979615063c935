"""Grouped INT4 expert GEMM (one launch over all experts) vs the per-expert oracle loop."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref

from kernels.moe_grouped import int4_grouped_matmul, segment_offsets
from kernels.moe_routing import gather_rows, route_topk, sort_by_expert
from serve.quantize import quantize_int4

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _experts(dev, E, N, K, gs, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    packed, scales = [], []
    for _ in range(E):
        p, s = quantize_int4(torch.randn(N, K, generator=g, device=dev) * 0.02, gs)
        packed.append(p)
        scales.append(s.to(torch.float16))
    return torch.stack(packed), torch.stack(scales)


@pytest.mark.parametrize("counts", [[5, 0, 130, 1], [0, 0, 0, 64], [300, 1, 1, 1]])
def test_grouped_small(dev, counts):
    E, N, K, gs = 4, 384, 256, 128
    P, S = _experts(dev, E, N, K, gs, sum(counts))
    M = sum(counts)
    g = torch.Generator().manual_seed(M)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    cnt = torch.tensor(counts, device=dev)
    out = int4_grouped_matmul(a.to(dev), P, S, cnt, gs)
    off = np.concatenate([[0], np.cumsum(counts)])
    want = ref.grouped_int4_matmul(a.float().numpy(), P.cpu().numpy(), S.float().cpu().numpy(), off, gs)
    ok, worst = ref.close_bf16(out.float().cpu().numpy(), want)
    assert ok, f"worst {worst:.3g}"
    out2 = int4_grouped_matmul(a.to(dev), P, S, segment_offsets(cnt), gs)  # offsets form
    assert torch.equal(out, out2)


@pytest.mark.parametrize("gs,dtype", [(32, torch.bfloat16), (64, torch.float16), (256, torch.bfloat16),
                                      (128, torch.float16)])
def test_grouped_group_sizes(dev, gs, dtype):
    """Group boundaries inside a 64-k stage (32), at every stage (64), every fourth stage
    (256); fp16 activations; ragged N; a segment split over several row chunks."""
    counts = [7, 170, 0, 33, 96]
    E, N, K = len(counts), 200, 512
    P, S = _experts(dev, E, N, K, gs, gs)
    M = sum(counts)
    g = torch.Generator().manual_seed(gs)
    a = torch.randn(M, K, generator=g).to(dtype)
    out = int4_grouped_matmul(a.to(dev), P, S, torch.tensor(counts, device=dev), gs)
    assert out.dtype == dtype
    off = np.concatenate([[0], np.cumsum(counts)])
    want = ref.grouped_int4_matmul(a.float().numpy(), P.cpu().numpy(), S.float().cpu().numpy(), off, gs)
    ok, worst = ref.close_bf16(out.float().cpu().numpy(), want)
    assert ok, f"worst {worst:.3g}"


@pytest.mark.parametrize("K,gs", [(8192, 128), (14336, 128), (4096, 64)])
def test_grouped_many_groups(dev, K, gs):
    """More than 32 groups per row: the 128-group scale table (64 and 112 groups; the
    expert MLP's unsplit down projection at H = 14336)."""
    counts = [40, 0, 130, 7]
    E, N = len(counts), 256
    P, S = _experts(dev, E, N, K, gs, K + gs)
    M = sum(counts)
    g = torch.Generator().manual_seed(K)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    out = int4_grouped_matmul(a.to(dev), P, S, torch.tensor(counts, device=dev), gs)
    off = np.concatenate([[0], np.cumsum(counts)])
    want = ref.grouped_int4_matmul(a.float().numpy(), P.cpu().numpy(), S.float().cpu().numpy(), off, gs)
    ok, worst = ref.close_bf16(out.float().cpu().numpy(), want)
    assert ok, f"K={K} gs={gs}: worst {worst:.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_fused_gather(dev, dtype):
    """a_rows: the dispatch gather inside the activation load gives the same bits as the
    grouped GEMM on gather_rows' output (same rows, same arithmetic); repeated and unsorted
    token indices; an index outside the token matrix reads a zero row."""
    T, E, k, K, N, gs = 90, 5, 2, 384, 256, 64
    P, S = _experts(dev, E, N, K, gs, 21)
    x = torch.randn(T, K, device=dev).to(dtype)
    g = torch.Generator(device=dev).manual_seed(3)
    ex = torch.randint(0, E, (T, k), generator=g, device=dev)
    tok, counts, _ = sort_by_expert(ex, E)
    want = int4_grouped_matmul(gather_rows(x, tok), P, S, counts, gs)
    got = int4_grouped_matmul(x, P, S, counts, gs, a_rows=tok)
    assert torch.equal(got, want)
    bad = tok.clone()
    bad[3] = T + 5
    bad[7] = -1
    got = int4_grouped_matmul(x, P, S, counts, gs, a_rows=bad)
    assert torch.equal(got[3], torch.zeros_like(got[3])) and torch.equal(got[7], torch.zeros_like(got[7]))
    keep = torch.ones(T * k, dtype=torch.bool, device=dev)
    keep[3] = keep[7] = False
    assert torch.equal(got[keep], want[keep])


def test_config_e(dev):
    """512 tokens, hidden 4096, 8 experts with W_up [14336, 4096]
    INT4 g128, top-2 softmax routing from logits ~ N(0, 1), expert-sorted segments."""
    T, D, E, H, gs = 512, 4096, 8, 14336, 128
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g, device=dev)
    w, ex = route_topk(logits, 2)
    tok, counts, pos = sort_by_expert(ex, E)
    a = gather_rows(x, tok)
    P, S = _experts(dev, E, H, D, gs, 1)
    out = int4_grouped_matmul(a, P, S, counts, gs)
    assert out.shape == (T * 2, H) and out.dtype == torch.bfloat16
    off = [0] + torch.cumsum(counts, 0).tolist()
    worst = -1.0
    for e in range(E):
        lo, hi = off[e], off[e + 1]
        if hi == lo:
            continue
        q = torch.empty(H, D, dtype=torch.uint8, device=dev)
        q[:, 0::2] = P[e] & 0x0F
        q[:, 1::2] = P[e] >> 4
        wd = ((q.float() - 8).reshape(H, D // gs, gs) * S[e].float()[:, :, None]).reshape(H, D)
        want = a[lo:hi].float() @ wd.t().contiguous()
        err = (out[lo:hi].float() - want).abs() - (1e-2 + 1e-2 * want.abs())
        worst = max(worst, float(err.max()))
    assert worst <= 0, f"config E worst excess {worst:.3g}"
    # one expert's rows against the CPU oracle
    e = int(torch.argmax(counts))
    lo, hi = off[e], off[e] + 8
    want = ref.int4_matmul(a[lo:hi].float().cpu().numpy(), P[e].cpu().numpy(), S[e].float().cpu().numpy(), gs)
    ok, w_ = ref.close_bf16(out[lo:hi].float().cpu().numpy(), want)
    assert ok, f"oracle rows worst {w_:.3g}"


def test_offsets_past_rows_are_clamped(dev):
    """Device offsets cannot be checked by the host without a sync; offsets that run past
    the activation rows (counts summing to more than M_total) are truncated at M_total in
    the kernels: the result equals the call with the truncated offsets, and nothing is
    read or written outside the operands."""
    from kernels.moe_grouped import int4_grouped_gate_up
    E, N, K, gs, M = 4, 256, 256, 128, 100
    P, S = _experts(dev, E, N, K, gs, 17)
    a = torch.randn(M, K, generator=torch.Generator().manual_seed(18)).to(torch.bfloat16).to(dev)
    bad = torch.tensor([0, 30, 70, 137, 160], dtype=torch.int32, device=dev)
    good = torch.tensor([0, 30, 70, 100, 100], dtype=torch.int32, device=dev)
    out = int4_grouped_matmul(a, P, S, bad, gs)
    assert torch.equal(out, int4_grouped_matmul(a, P, S, good, gs))
    P2, S2 = _experts(dev, E, N, K, gs, 19)
    h = int4_grouped_gate_up(a, P, S, P2, S2, bad, gs)
    assert torch.equal(h, int4_grouped_gate_up(a, P, S, P2, S2, good, gs))
