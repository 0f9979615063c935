"""Top-k routing and expert-sorted dispatch: the harness around the grouped INT4
GEMM (kernels.moe_grouped). Same conventions as the reference:

- route_topk: softmax in fp32 over router logits, top-k, renormalised
  (train/model.py:158-162);
- sort_by_expert: stable sort of the T*k (token, slot) assignments by expert,
  per-expert counts and the inverse permutation (kernels/moe_routing.py:116-130);
- gather_rows: out[i] = x[idx[i]] (kernels/moe_routing.py:89-97).

- combine_rows: out[t] = sum_k w[t, k] * expert_out[pos[t, k]], one gfx950 block per
  output row, no atomics (kernels/moe_routing.py:52-76, 100-113);
- combine_partials: the same over the fp32 partial products of a K-split expert GEMM;
- moe_dispatch_combine: the routed MoE forward (kernels/moe_routing.py:133-153). When
  the experts are SwiGLU MLPs whose projections are INT4 QuantLinear with stacked
  buffers (serve.quantize.quantize_model stacks them), the per-expert loop becomes two
  grouped launches and the combine (kernels.moe_grouped.int4_expert_mlp_combine);
  otherwise each expert module runs on its segment as in the reference.

sort and gather are index bookkeeping on the device (torch ops).
"""

from __future__ import annotations

import torch

import kernels
from kernels._hip import dt_code, ld, require_hip, stream


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


def _combine_dt(dtype: torch.dtype, what: str) -> int:
    """dtype code of a combine operand: the three GEMM dtypes and fp64."""
    return kernels.MLS_F64 if dtype == torch.float64 else dt_code(dtype, what)


def combine_rows(expert_out: torch.Tensor, weights: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """out[t] = sum_k weights[t, k] * expert_out[pos[t, k]], output in expert_out's dtype,
    accumulated in fp32, or in fp64 when expert_out is fp64 (the reference's ACC64, which
    its fp64 gradcheck relies on; kernels/moe_routing.py:54-72, 100-113)."""
    dev = require_hip("combine_rows", expert_out, weights, pos)
    T, K = pos.shape
    D = expert_out.shape[1]
    x = expert_out if expert_out.stride(1) == 1 else expert_out.contiguous()
    w = weights.contiguous()
    p = pos.to(torch.int64).contiguous()
    out = torch.empty(T, D, dtype=x.dtype, device=dev)
    kernels.check(kernels.lib().mls_moe_combine(
        x.data_ptr(), _combine_dt(x.dtype, "combine_rows"), ld(x), x.shape[0], 1, 0, w.data_ptr(),
        _combine_dt(w.dtype, "combine_rows weights"), p.data_ptr(), T, K, out.data_ptr(),
        _combine_dt(out.dtype, "combine_rows"), ld(out), D, stream(dev)), "combine_rows")
    return out


def combine_partials(partials: torch.Tensor, weights: torch.Tensor, pos: torch.Tensor,
                     out_dtype: torch.dtype) -> torch.Tensor:
    """combine_rows over the fp32 partial products [splits, rows, D] of a K-split expert
    GEMM: out[t] = sum_k weights[t, k] * sum_p partials[p, pos[t, k]], in out_dtype."""
    dev = require_hip("combine_partials", partials, weights, pos)
    S, R, D = partials.shape
    T, K = pos.shape
    x = partials.contiguous()
    w = weights.contiguous()
    p = pos.to(torch.int64).contiguous()
    out = torch.empty(T, D, dtype=out_dtype, device=dev)
    kernels.check(kernels.lib().mls_moe_combine(
        x.data_ptr(), dt_code(x.dtype, "combine_partials"), D, R, S, R * D, w.data_ptr(),
        dt_code(w.dtype, "combine_partials weights"), p.data_ptr(), T, K, out.data_ptr(),
        dt_code(out_dtype, "combine_partials"), ld(out), D, stream(dev)), "combine_partials")
    return out


def moe_dispatch_combine(flat: torch.Tensor, weights: torch.Tensor, experts_idx: torch.Tensor,
                         expert_modules) -> torch.Tensor:
    """Routed MoE forward (kernels/moe_routing.py:133-153): sort the (token, slot)
    assignments by expert, gather the rows, run every expert on its contiguous segment,
    combine weighted by the router. flat [T, D], weights [T, k], experts_idx [T, k]."""
    from kernels.moe_grouped import int4_expert_mlp_combine, segment_offsets
    from serve.quantize import stacked_int4_experts

    n_experts = len(expert_modules)
    token_of_slot, counts, pos = sort_by_expert(experts_idx, n_experts)
    st = stacked_int4_experts(expert_modules)
    if st is not None and flat.dtype in (torch.bfloat16, torch.float16):
        # the gather runs inside the gate/up kernel's activation load (a_rows)
        return int4_expert_mlp_combine(flat, segment_offsets(counts), st["w_gate"][0], st["w_gate"][1],
                                       st["w_up"][0], st["w_up"][1], st["w_down"][0], st["w_down"][1],
                                       st["group_size"], weights, pos, a_rows=token_of_slot)
    dispatched = gather_rows(flat, token_of_slot)
    expert_out = torch.empty_like(dispatched)
    start = 0
    for e, cnt in enumerate(counts.tolist()):
        if cnt:
            expert_out[start:start + cnt] = expert_modules[e](dispatched[start:start + cnt])
        start += cnt
    return combine_rows(expert_out, weights, pos)
