"""Paged-attention decode over a block-scattered KV cache, on gfx950.

Same function, arguments and result as the reference (kernels/paged_attention.py:
93-118): q [n_seqs, H, D]; k_pool / v_pool [num_blocks, H, block_size, D] (one
(block, head) slab contiguous, K and V with the same strides); block_tables
[n_seqs, max_blocks] int32; context_lens [n_seqs] int32 (the new token already
written and counted); scale defaults to D^-0.5. Returns [n_seqs, H, D] in q's dtype.

The kernel (csrc/paged_attn.hip) walks each sequence's block table and keeps an
online softmax, one wavefront per (sequence, head, context split); with few
(sequence, head) pairs and long tables the context is split over several wavefronts
and merged by a second kernel through a workspace this wrapper allocates (its size
comes from mls_paged_attention_workspace). Tokens at or past a sequence's context
length weigh 0; a zero context gives a zero output.
"""

from __future__ import annotations

import torch

import kernels
from kernels._hip import dt_code, require_hip, stream


def paged_attention_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor,
                           scale: float | None = None) -> torch.Tensor:
    dev = require_hip("paged_attention_decode", q, k_pool, v_pool, block_tables, context_lens)
    n_seqs, H, D = q.shape
    num_blocks, Hk, block_size, Dk = k_pool.shape
    if (Hk, Dk) != (H, D) or v_pool.shape != k_pool.shape or v_pool.dtype != k_pool.dtype:
        raise ValueError(f"paged_attention_decode: q {tuple(q.shape)}, pools {tuple(k_pool.shape)} / "
                         f"{tuple(v_pool.shape)} do not match")
    scale = scale if scale is not None else D ** -0.5
    # a fresh dense output whatever q's layout (empty_like would copy q's strides)
    out = torch.empty(n_seqs, H, D, dtype=q.dtype, device=dev)
    if n_seqs == 0:
        return out
    # the library reads q rows with unit inner stride and non-overlapping heads and
    # sequences (q_sh >= D, q_ss >= H*D); any other layout is copied dense first
    # (clone, not contiguous(): a size-1 dimension may keep any stride under contiguous())
    if q.stride(2) != 1 or q.stride(1) < D or q.stride(0) < H * D:
        q = q.clone(memory_format=torch.contiguous_format)
    st = k_pool.stride()
    if (st[3] != 1 or st[2] < D or st[1] < st[2] * block_size or st[0] < st[1] * H
            or v_pool.stride() != st):
        k_pool = k_pool.clone(memory_format=torch.contiguous_format)
        v_pool = v_pool.clone(memory_format=torch.contiguous_format)
    bt = block_tables.to(torch.int32).contiguous()
    ctx = context_lens.to(torch.int32).contiguous()
    if bt.dim() != 2 or bt.shape[0] != n_seqs or ctx.shape != (n_seqs,):
        raise ValueError(f"paged_attention_decode: block_tables {tuple(bt.shape)} / context_lens "
                         f"{tuple(ctx.shape)} for {n_seqs} sequences")
    max_blocks = bt.shape[1]
    L = kernels.lib()
    ws_n = L.mls_paged_attention_workspace(n_seqs, H, D, max_blocks)
    ws = torch.empty(max(ws_n, 1), dtype=torch.float32, device=dev)
    kernels.check(L.mls_paged_attention_decode(
        q.data_ptr(), dt_code(q.dtype, "paged_attention_decode q"), q.stride(0), q.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), dt_code(k_pool.dtype, "paged_attention_decode pools"),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2), num_blocks,
        bt.data_ptr(), bt.stride(0) if n_seqs > 1 else max_blocks, max_blocks, ctx.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1), n_seqs, H, D, block_size, float(scale),
        ws.data_ptr(), ws_n, stream(dev)), "paged_attention_decode")
    return out
