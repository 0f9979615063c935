"""The allocation-free paged-attention decode (mls_paged_attention_decode_noalloc): the
same kernels as mls_paged_attention_decode with the context-split workspace in a
static device array instead of a caller buffer. Called through the C ABI and checked
bit for bit against the caller-workspace entry point on the same inputs, twice in a
row (the second call smaller, so it runs over what the first left in the array),
plus a call that needs no split and the host-side rejection of a split larger than
the array."""

from __future__ import annotations

import pytest
import torch

import kernels
from kernels._hip import dt_code

SCRATCH_FLOATS = 2 * 1024 * 1024  # MLS_PAGED_SCRATCH_FLOATS in include/mls.h


def _cache(n_seqs, H, D, bs, ctx, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    nb_per = -(-ctx // bs)
    nb = n_seqs * nb_per + 3
    kp = torch.randn(nb, H, bs, D, generator=g).to(dtype).to(dev)
    vp = torch.randn(nb, H, bs, D, generator=g).to(dtype).to(dev)
    tab = torch.randperm(nb, generator=g)[:n_seqs * nb_per].reshape(n_seqs, nb_per).to(torch.int32).to(dev)
    lens = torch.randint(ctx // 2, ctx + 1, (n_seqs,), generator=g).to(torch.int32)
    lens[0] = ctx
    q = torch.randn(n_seqs, H, D, generator=g).to(dtype).to(dev)
    return q, kp, vp, tab, lens.to(dev)


def _args(q, kp, vp, tab, lens, out):
    n, H, D = q.shape
    return (q.data_ptr(), dt_code(q.dtype, "q"), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(),
            dt_code(kp.dtype, "kv"), kp.stride(0), kp.stride(1), kp.stride(2), kp.shape[0], tab.data_ptr(),
            tab.stride(0), tab.shape[1], lens.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
            n, H, D, kp.shape[2], float(D) ** -0.5)


def _both(q, kp, vp, tab, lens):
    """(caller-workspace result, allocation-free result, workspace floats the split needs)."""
    L = kernels.lib()
    st = torch.cuda.current_stream(q.device).cuda_stream
    n, H, D = q.shape
    need = L.mls_paged_attention_workspace(n, H, D, tab.shape[1])
    ws = torch.empty(max(need, 1), dtype=torch.float32, device=q.device)
    ref = torch.empty_like(q)
    kernels.check(L.mls_paged_attention_decode(*_args(q, kp, vp, tab, lens, ref), ws.data_ptr(), need, st),
                  "mls_paged_attention_decode")
    out = torch.full_like(q, float("nan"))
    kernels.check(L.mls_paged_attention_decode_noalloc(*_args(q, kp, vp, tab, lens, out), st),
                  "mls_paged_attention_decode_noalloc")
    torch.cuda.synchronize()
    return ref, out, need


def test_noalloc_rejects_a_split_above_the_static_array():
    """Host-side check, before any HIP call (16-byte aligned dummy pointers, no GPU):
    32 sequences x 64 heads of D = 512 in bf16 split in two need 2,105,344 floats."""
    L = kernels.load_library()
    n, H, D, bs, mb = 32, 64, 512, 16, 16
    assert L.mls_paged_attention_workspace(n, H, D, mb) == n * H * 2 * (D + 2) > SCRATCH_FLOATS
    bf = kernels.MLS_BF16
    rc = L.mls_paged_attention_decode_noalloc(16, bf, H * D, D, 16, 16, bf, D * bs * H, D * bs, D, n * mb,
                                              16, mb, mb, 16, 16, H * D, D, n, H, D, bs, 0.05, None)
    msg = L.mls_last_error().decode()
    assert rc == kernels.MLS_ERR_ARG and "static scratch" in msg, msg


@pytest.mark.gpu
def test_noalloc_matches_caller_workspace_twice(dev):
    # first call: 8 sequences x 32 heads of 128 (bf16), contexts up to 3000 tokens in
    # blocks of 16 -> the context splits over 16 wavefronts per (sequence, head)
    q, kp, vp, tab, lens = _cache(8, 32, 128, 16, 3000, torch.bfloat16, 1, dev)
    ref, out, need = _both(q, kp, vp, tab, lens)
    assert 0 < need <= SCRATCH_FLOATS
    assert torch.equal(out, ref)
    # second call, smaller: 3 sequences x 4 heads of 64 (fp16), shorter contexts; the
    # array still holds the first call's partials
    q2, kp2, vp2, tab2, lens2 = _cache(3, 4, 64, 8, 700, torch.float16, 2, dev)
    ref2, out2, need2 = _both(q2, kp2, vp2, tab2, lens2)
    assert 0 < need2 < need
    assert torch.equal(out2, ref2)
    # a batch that needs no split (the scratch is not touched) and an fp32 one again
    q3, kp3, vp3, tab3, lens3 = _cache(64, 64, 128, 16, 64, torch.bfloat16, 3, dev)
    ref3, out3, need3 = _both(q3, kp3, vp3, tab3, lens3)
    assert need3 == 0 and torch.equal(out3, ref3)
    q4, kp4, vp4, tab4, lens4 = _cache(2, 2, 32, 8, 900, torch.float32, 4, dev)
    ref4, out4, need4 = _both(q4, kp4, vp4, tab4, lens4)
    assert need4 > 0 and torch.equal(out4, ref4)
    # and the result is the attention itself: sequence 0, head 0 of the first call
    blocks = tab[0].long()
    k = kp[blocks, 0].float().reshape(-1, 128)[:3000]
    v = vp[blocks, 0].float().reshape(-1, 128)[:3000]
    p = torch.softmax(k @ q[0, 0].float() * 128 ** -0.5, dim=0)
    want = p @ v
    assert torch.allclose(out[0, 0].float(), want, rtol=1e-2, atol=1e-2)
