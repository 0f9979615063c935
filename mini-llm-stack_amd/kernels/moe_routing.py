"""Top-k routing and expert-sorted dispatch: the harness around the grouped INT4
GEMM (kernels.moe_grouped). Same conventions as the reference:

- route_topk: softmax in fp32 over router logits, top-k, renormalised
  (train/model.py:158-162);
- sort_by_expert: stable sort of the T*k (token, slot) assignments by expert,
  per-expert counts and the inverse permutation (kernels/moe_routing.py:116-130);
- gather_rows: out[i] = x[idx[i]] (kernels/moe_routing.py:89-97).

These are index bookkeeping on the device (torch ops); the weighted combine of
expert outputs is outside the quantized-linear path.
"""

from __future__ import annotations

import torch


def route_topk(logits: torch.Tensor, k: int):
    """(weights [T, k] fp32, experts [T, k] int64)."""
    probs = torch.softmax(logits.float(), dim=-1)
    weights, experts = torch.topk(probs, k, dim=-1)
    weights = weights / weights.sum(dim=-1, keepdim=True)
    return weights, experts


def sort_by_expert(experts_idx: torch.Tensor, n_experts: int):
    """(token_of_slot [T*k], counts [E], pos [T, k]) for expert-contiguous dispatch."""
    T, k = experts_idx.shape
    flat = experts_idx.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=n_experts)
    pos = torch.empty_like(order)
    pos[order] = torch.arange(T * k, device=flat.device)
    return order // k, counts, pos.reshape(T, k)


def gather_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    return x.index_select(0, idx.to(torch.int64))
