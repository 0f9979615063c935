"""Paged-attention decode on the GPU (kernels/paged_attention.py:33-118) against the
oracle: the reference's own tests (test_serving.py:62-106) plus dtypes, head sizes
that take the 16-byte-row kernel and the generic one, block sizes, context splits,
zero contexts and invalid block ids.

Tolerances: fp32 rtol = atol = 1e-4 (the reference test's), 16-bit pools/queries
rtol = atol = 1e-2 (ref.close_bf16) against the fp64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref

from kernels.paged_attention import paged_attention_decode

pytestmark = pytest.mark.gpu


def _cache(lens, H, D, bs, num_blocks, seed, dtype=torch.float32):
    """A paged pool with each sequence's tokens in random blocks; tables padded with 0."""
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(num_blocks, H, bs, D, generator=g)
    vp = torch.randn(num_blocks, H, bs, D, generator=g)
    free = torch.randperm(num_blocks, generator=g).tolist()
    tables = [[free.pop() for _ in range((L + bs - 1) // bs)] for L in lens]
    mb = max(1, max(len(t) for t in tables))
    tab = torch.tensor([t + [0] * (mb - len(t)) for t in tables], dtype=torch.int32)
    ctx = torch.tensor(lens, dtype=torch.int32)
    return kp.to(dtype), vp.to(dtype), tab, ctx


def _run(q, kp, vp, tab, ctx, dev, scale=None):
    out = paged_attention_decode(q.to(dev), kp.to(dev), vp.to(dev), tab.to(dev), ctx.to(dev), scale)
    want = ref.paged_attention_decode(q.float().numpy(), kp.float().numpy(), vp.float().numpy(),
                                      tab.numpy(), ctx.numpy(), scale)
    return out, want


def _check(out, want, what):
    o = out.float().cpu().numpy()
    if out.dtype == torch.float32:
        assert np.allclose(o, want, rtol=1e-4, atol=1e-4), f"{what}: max err {np.abs(o - want).max():.3g}"
    else:
        ok, worst = ref.close_bf16(o, want)
        assert ok, f"{what}: worst {worst:.3g}"


@pytest.mark.parametrize("lens", [[7], [16], [5, 23, 12], [1, 1, 40]])
def test_matches_contiguous(dev, lens):
    """test_serving.py:62-84 of the reference: H=4, D=32, block 8, fp32."""
    kp, vp, tab, ctx = _cache(lens, 4, 32, 8, 32, sum(lens))
    q = torch.randn(len(lens), 4, 32, generator=torch.Generator().manual_seed(1))
    out, want = _run(q, kp, vp, tab, ctx, dev)
    assert out.shape == q.shape and out.dtype == q.dtype
    _check(out, want, f"lens={lens}")


def test_respects_context_len(dev):
    """test_serving.py:87-106: poisoned slots past the context must not leak in."""
    kp, vp, tab, ctx = _cache([5], 2, 16, 8, 4, 3)
    kp[tab[0, 0], :, 5:] = 1e6
    vp[tab[0, 0], :, 5:] = 1e6
    q = torch.randn(1, 2, 16)
    out, want = _run(q, kp, vp, tab, ctx, dev)
    _check(out, want, "poisoned")
    assert out.abs().max().item() < 100


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64), (torch.bfloat16, 256),
                                     (torch.float32, 16), (torch.float32, 128), (torch.float32, 24),
                                     (torch.bfloat16, 80), (torch.float16, 8),
                                     # 16-byte chunks per row of 2 and 64: the narrowest and
                                     # widest lane groups of the score reduction
                                     (torch.float32, 8), (torch.bfloat16, 512)])
@pytest.mark.parametrize("bs", [1, 8, 16, 32])
def test_dtypes_head_dims_block_sizes(dev, dtype, D, bs):
    lens = [1, bs, bs + 1, 3 * bs + 5, 37]
    kp, vp, tab, ctx = _cache(lens, 3, D, bs, 64 * 3 + 10, D * bs)
    q = torch.randn(len(lens), 3, D, generator=torch.Generator().manual_seed(D)).to(dtype)
    out, want = _run(q, kp.to(dtype), vp.to(dtype), tab, ctx, dev)
    _check(out, want, f"{dtype} D={D} bs={bs}")


def test_fp32_query_on_16bit_cache(dev):
    """The engine's mix (serve/engine.py:137-144): model-dtype queries, cache-dtype pools."""
    kp, vp, tab, ctx = _cache([9, 33, 2], 4, 64, 16, 16, 5, torch.bfloat16)
    q = torch.randn(3, 4, 64)
    out, want = _run(q, kp, vp, tab, ctx, dev, scale=0.2)
    assert out.dtype == torch.float32
    ok, worst = ref.close_bf16(out.cpu().numpy(), want)
    assert ok, worst


@pytest.mark.parametrize("lens,H", [([5000], 2), ([3000, 17, 1200], 4)])
def test_split_context(dev, lens, H):
    """Few (sequence, head) pairs and long tables: the context is split over several
    wavefronts and merged through the workspace."""
    bs = 16
    nblk = sum((L + bs - 1) // bs for L in lens) + 4
    kp, vp, tab, ctx = _cache(lens, H, 64, bs, nblk, 11, torch.bfloat16)
    q = torch.randn(len(lens), H, 64).to(torch.bfloat16)
    out, want = _run(q, kp, vp, tab, ctx, dev)
    _check(out, want, f"split {lens}")


def test_zero_context_and_invalid_blocks(dev):
    """A zero context gives zeros (the reference's l_safe rule); a block id outside the
    pool inside the context is skipped: its tokens weigh 0."""
    H, D, bs = 2, 32, 8
    kp, vp, tab, ctx = _cache([0, 20, 20], H, D, bs, 16, 7)
    tab[2, 1] = 1000                       # tokens 8..15 of sequence 2: no such block
    q = torch.randn(3, H, D)
    out = paged_attention_decode(q.to(dev), kp.to(dev), vp.to(dev), tab.to(dev), ctx.to(dev)).cpu()
    assert out[0].abs().max().item() == 0.0
    want1 = ref.paged_attention_decode(q[1:2].numpy(), kp.numpy(), vp.numpy(), tab[1:2].numpy(), ctx[1:2].numpy())
    assert np.allclose(out[1].numpy(), want1[0], rtol=1e-4, atol=1e-4)
    keep = [j for j in range(20) if j // bs != 1]
    for h in range(H):
        k = np.stack([kp[tab[2, j // bs], h, j % bs].numpy() for j in keep])
        v = np.stack([vp[tab[2, j // bs], h, j % bs].numpy() for j in keep])
        assert np.allclose(out[2, h].numpy(), ref.attention(q[2, h].numpy(), k, v, D ** -0.5), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("layout", ["heads_major", "one_seq_odd_stride", "one_head_odd_stride"])
def test_query_layouts(dev, layout):
    """Dense but permuted or size-1-strided queries (the reference makes q contiguous
    and accepts any layout): the output is a fresh dense [n_seqs, H, D] tensor equal
    to the result for the contiguous query."""
    lens = [9, 30, 17] if layout != "one_seq_odd_stride" else [25]
    H = 1 if layout == "one_head_odd_stride" else 4
    kp, vp, tab, ctx = _cache(lens, H, 32, 8, 24, 11)
    g = torch.Generator().manual_seed(12)
    n = len(lens)
    if layout == "heads_major":          # strides (D, n*D, 1): x.transpose(0, 1)
        q = torch.randn(H, n, 32, generator=g).to(dev).transpose(0, 1)
    elif layout == "one_seq_odd_stride":  # [1, H, D] view whose seq stride is below H*D
        q = torch.randn(H, 32, generator=g).to(dev).unsqueeze(0).as_strided((1, H, 32), (1, 32, 1))
    else:                                # [n, 1, D] view whose head stride is below D
        q = torch.randn(n, 32, generator=g).to(dev).as_strided((n, 1, 32), (32, 1, 1))
    out = paged_attention_decode(q, kp.to(dev), vp.to(dev), tab.to(dev), ctx.to(dev))
    assert out.shape == (n, H, 32) and out.is_contiguous()
    dense = paged_attention_decode(q.contiguous(), kp.to(dev), vp.to(dev), tab.to(dev), ctx.to(dev))
    assert torch.equal(out, dense)
    _check(out, ref.paged_attention_decode(q.cpu().numpy(), kp.numpy(), vp.numpy(), tab.numpy(),
                                           ctx.numpy()), layout)


def test_large_batch_against_torch(dev):
    """A serving-sized batch (64 sequences, 8 heads, D=128, bf16, contexts up to 700)
    against torch's attention on gathered contiguous K/V in fp32."""
    g = torch.Generator().manual_seed(21)
    lens = torch.randint(1, 700, (64,), generator=g).tolist()
    H, D, bs = 8, 128, 16
    nblk = sum((L + bs - 1) // bs for L in lens) + 8
    kp, vp, tab, ctx = _cache(lens, H, D, bs, nblk, 22, torch.bfloat16)
    q = torch.randn(64, H, D, generator=g).to(torch.bfloat16)
    out = paged_attention_decode(q.to(dev), kp.to(dev), vp.to(dev), tab.to(dev), ctx.to(dev)).float().cpu()
    for s in range(0, 64, 7):
        L = lens[s]
        idx = [(tab[s, j // bs].item(), j % bs) for j in range(L)]
        k = torch.stack([kp[b, :, r] for b, r in idx], 1).float()       # [H, L, D]
        v = torch.stack([vp[b, :, r] for b, r in idx], 1).float()
        want = torch.softmax((k @ q[s].float()[:, :, None])[..., 0] * D ** -0.5, -1)[:, None, :] @ v
        ok, worst = ref.close_bf16(out[s].numpy(), want[:, 0].numpy())
        assert ok, f"seq {s} (L={L}): worst {worst:.3g}"


def test_bench_shape(dev):
    """The bench's workload at full size: 64 sequences x 32 heads x 2048 cached tokens,
    D = 128, bf16 pools in blocks of 16 handed out in a shuffled order. 16 sampled
    (sequence, head) pairs against torch's attention on the gathered K/V in fp32."""
    S, H, D, ctx, bs = 64, 32, 128, 2048, 16
    g = torch.Generator(device=dev).manual_seed(8)
    nb = S * ctx // bs
    kp = torch.randn(nb, H, bs, D, generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn(nb, H, bs, D, generator=g, device=dev).to(torch.bfloat16)
    tab = torch.randperm(nb, generator=g, device=dev).to(torch.int32).reshape(S, ctx // bs).contiguous()
    lens = torch.full((S,), ctx, dtype=torch.int32, device=dev)
    q = torch.randn(S, H, D, generator=g, device=dev).to(torch.bfloat16)
    out = paged_attention_decode(q, kp, vp, tab, lens)
    assert out.shape == (S, H, D) and out.dtype == torch.bfloat16
    pick = torch.randint(0, S * H, (16,), generator=torch.Generator().manual_seed(3)).tolist()
    for sh in pick:
        s, h = divmod(sh, H)
        blocks = tab[s].long()
        k = kp[blocks, h].reshape(ctx, D).float()         # [ctx, D] in token order
        v = vp[blocks, h].reshape(ctx, D).float()
        p = torch.softmax((k @ q[s, h].float()) * D ** -0.5, 0)
        want = (p[None, :] @ v)[0]
        ok, worst = ref.close_bf16(out[s, h].float().cpu().numpy(), want.cpu().numpy())
        assert ok, f"seq {s} head {h}: worst {worst:.3g}"
