"""INT4 weight-only GEMM over expert-sorted token segments, one launch for all experts.

The reference runs a quantized MoE layer as a Python loop over experts, one
int4_matmul per non-empty expert segment after a host sync on the counts
(kernels/moe_routing.py:145-151 through QuantLinear, serve/quantize.py:110-114).
Here the segment offsets stay on the device and a single gfx950 MFMA launch
covers every (expert, row tile, column tile); each workgroup finds its expert
from the offsets. Weights of all experts are stacked: packed [E, N, K/2] and
scales [E, N, K/group] in the INT4 layout of kernels.dequant_matmul.
"""

from __future__ import annotations

import torch

import kernels
from kernels._hip import dt_code, ld, require_hip, rows, stream


def segment_offsets(counts: torch.Tensor) -> torch.Tensor:
    """int32 [E+1] exclusive prefix sum of per-expert row counts (on the device)."""
    off = torch.zeros(counts.numel() + 1, dtype=torch.int32, device=counts.device)
    off[1:] = torch.cumsum(counts.reshape(-1).to(torch.int64), 0).to(torch.int32)
    return off


def _offsets(counts_or_offsets: torch.Tensor, E: int, fn: str) -> torch.Tensor:
    if counts_or_offsets.numel() == E:
        return segment_offsets(counts_or_offsets)
    if counts_or_offsets.numel() == E + 1:
        return counts_or_offsets.reshape(-1).to(torch.int32).contiguous()
    raise ValueError(f"{fn}: expected {E} counts or {E + 1} offsets, got {counts_or_offsets.numel()}")


def _row_index(a_rows: torch.Tensor | None, M: int, fn: str) -> torch.Tensor | None:
    if a_rows is None:
        return None
    if a_rows.numel() != M:
        raise ValueError(f"{fn}: a_rows has {a_rows.numel()} entries, expected one per sorted row ({M})")
    return a_rows.reshape(-1).to(torch.int32).contiguous()


def int4_grouped_matmul(a_sorted: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor,
                        counts_or_offsets: torch.Tensor, group_size: int,
                        a_rows: torch.Tensor | None = None) -> torch.Tensor:
    """out[r] = a_sorted[r] @ dequant(w_packed[e], scale[e], group_size).T for every row r
    of expert e's segment. counts_or_offsets: per-expert counts [E] or offsets [E+1]
    (int, on the device). a_sorted [M_total, K] bf16/fp16 -> out [M_total, N] same dtype.
    With a_rows (int [M_total], the token of each sorted slot: sort_by_expert's
    token_of_slot), a_sorted is the unsorted token matrix and sorted row r is its row
    a_rows[r]: the dispatch gather (gather_rows, kernels/moe_routing.py:144) happens inside
    the activation load."""
    dev = require_hip("int4_grouped_matmul", a_sorted, w_packed, scale, counts_or_offsets)
    if w_packed.dim() != 3 or w_packed.dtype != torch.uint8:
        raise ValueError(f"int4_grouped_matmul: w_packed must be uint8 [E, N, K/2], got "
                         f"{w_packed.dtype} {tuple(w_packed.shape)}")
    E, N, Kh = w_packed.shape
    M, K = a_sorted.shape
    idx = None
    if a_rows is not None:
        require_hip("int4_grouped_matmul", a_rows)
        idx = _row_index(a_rows, a_rows.numel(), "int4_grouped_matmul")
        M = idx.numel()
    assert K % group_size == 0 and K == Kh * 2
    G = K // group_size
    if tuple(scale.shape) != (E, N, G):
        raise ValueError(f"int4_grouped_matmul: scale shape {tuple(scale.shape)}, expected {(E, N, G)}")
    off = _offsets(counts_or_offsets, E, "int4_grouped_matmul")
    adt = dt_code(a_sorted.dtype, "int4_grouped_matmul")
    a = rows(a_sorted)
    w = w_packed if w_packed.is_contiguous() else w_packed.contiguous()
    if scale.dtype not in (torch.float32, torch.float16):
        scale = scale.to(torch.float32)
    s = scale if scale.is_contiguous() else scale.contiguous()
    sdt = dt_code(s.dtype, "int4_grouped_matmul scale")
    c = torch.empty(M, N, dtype=a.dtype, device=dev)
    if idx is None:
        kernels.check(kernels.lib().mls_int4_grouped_gemm(
            a.data_ptr(), adt, ld(a), off.data_ptr(), E, M,
            w.data_ptr(), N * Kh, Kh, s.data_ptr(), sdt, N * G, G, 1, group_size,
            c.data_ptr(), adt, ld(c), N, K, stream(dev)), "int4_grouped_matmul")
    else:
        kernels.check(kernels.lib().mls_int4_grouped_gemm_rows(
            a.data_ptr(), adt, ld(a), idx.data_ptr(), a.shape[0], off.data_ptr(), E, M,
            w.data_ptr(), N * Kh, Kh, s.data_ptr(), sdt, N * G, G, 1, group_size,
            c.data_ptr(), adt, ld(c), N, K, stream(dev)), "int4_grouped_matmul")
    return c


def int4_grouped_gate_up(a_sorted: torch.Tensor, wg_packed: torch.Tensor, sg: torch.Tensor,
                         wu_packed: torch.Tensor, su: torch.Tensor,
                         counts_or_offsets: torch.Tensor, group_size: int,
                         a_rows: torch.Tensor | None = None) -> torch.Tensor:
    """h[r] = silu(a_sorted[r] @ dequant(wg[e]).T) * (a_sorted[r] @ dequant(wu[e]).T) for
    every row r of expert e's segment: the first half of a SwiGLU expert MLP
    (train/model.py:127-135) with INT4 gate/up weights, one launch for all experts.
    wg/wu packed [E, H, K/2], sg/su [E, H, K/group] (same dtype) -> h [M_total, H].
    a_rows: as for int4_grouped_matmul (the dispatch gather fused into the load)."""
    dev = require_hip("int4_grouped_gate_up", a_sorted, wg_packed, sg, wu_packed, su, counts_or_offsets)
    for w in (wg_packed, wu_packed):
        if w.dim() != 3 or w.dtype != torch.uint8:
            raise ValueError(f"int4_grouped_gate_up: packed weights must be uint8 [E, H, K/2], got "
                             f"{w.dtype} {tuple(w.shape)}")
    if wg_packed.shape != wu_packed.shape or sg.shape != su.shape or sg.dtype != su.dtype:
        raise ValueError("int4_grouped_gate_up: gate and up weights/scales must have equal shapes and dtypes")
    E, H, Kh = wg_packed.shape
    M, K = a_sorted.shape
    idx = None
    if a_rows is not None:
        require_hip("int4_grouped_gate_up", a_rows)
        idx = _row_index(a_rows, a_rows.numel(), "int4_grouped_gate_up")
        M = idx.numel()
    assert K % group_size == 0 and K == Kh * 2
    G = K // group_size
    if tuple(sg.shape) != (E, H, G):
        raise ValueError(f"int4_grouped_gate_up: scale shape {tuple(sg.shape)}, expected {(E, H, G)}")
    off = _offsets(counts_or_offsets, E, "int4_grouped_gate_up")
    adt = dt_code(a_sorted.dtype, "int4_grouped_gate_up")
    a = rows(a_sorted)
    wg = wg_packed if wg_packed.is_contiguous() else wg_packed.contiguous()
    wu = wu_packed if wu_packed.is_contiguous() else wu_packed.contiguous()
    if sg.dtype not in (torch.float32, torch.float16):
        sg, su = sg.to(torch.float32), su.to(torch.float32)
    sg = sg if sg.is_contiguous() else sg.contiguous()
    su = su if su.is_contiguous() else su.contiguous()
    sdt = dt_code(sg.dtype, "int4_grouped_gate_up scale")
    h = torch.empty(M, H, dtype=a.dtype, device=dev)
    if idx is None:
        kernels.check(kernels.lib().mls_int4_grouped_gate_up(
            a.data_ptr(), adt, ld(a), off.data_ptr(), E, M, wg.data_ptr(), wu.data_ptr(), H * Kh, Kh,
            sg.data_ptr(), su.data_ptr(), sdt, H * G, G, 1, group_size,
            h.data_ptr(), adt, ld(h), H, K, stream(dev)), "int4_grouped_gate_up")
    else:
        kernels.check(kernels.lib().mls_int4_grouped_gate_up_rows(
            a.data_ptr(), adt, ld(a), idx.data_ptr(), a.shape[0], off.data_ptr(), E, M, wg.data_ptr(),
            wu.data_ptr(), H * Kh, Kh, sg.data_ptr(), su.data_ptr(), sdt, H * G, G, 1, group_size,
            h.data_ptr(), adt, ld(h), H, K, stream(dev)), "int4_grouped_gate_up")
    return h


def int4_expert_mlp(a_sorted: torch.Tensor, counts_or_offsets: torch.Tensor,
                    wg: torch.Tensor, sg: torch.Tensor, wu: torch.Tensor, su: torch.Tensor,
                    wd: torch.Tensor, sd: torch.Tensor, group_size: int) -> torch.Tensor:
    """SwiGLU expert MLP w_down(silu(w_gate(x)) * w_up(x)) (train/model.py:127-135) with
    INT4 weights for every expert's row segment: two launches (gate/up fused with the
    activation, then down). wd packed [E, D, H/2], sd [E, D, H/group] -> [M_total, D]."""
    E = wg.shape[0]
    off = _offsets(counts_or_offsets, E, "int4_expert_mlp")
    h = int4_grouped_gate_up(a_sorted, wg, sg, wu, su, off, group_size)
    return int4_grouped_matmul(h, wd, sd, off, group_size)


def grouped_splits(M_total: int, E: int, N: int, K: int, group_size: int) -> int:
    """K splits the partial-product down projection uses for this shape (1: none)."""
    return int(kernels.lib().mls_int4_grouped_splits(M_total, E, N, K, group_size))


def int4_grouped_matmul_partial(a_sorted: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor,
                                counts_or_offsets: torch.Tensor, group_size: int, splits: int) -> torch.Tensor:
    """int4_grouped_matmul as `splits` fp32 partial products over equal K ranges:
    [splits, M_total, N], whose sum over the first axis is the product (the reduction is
    left to the consumer, e.g. kernels.moe_routing.combine_partials)."""
    dev = require_hip("int4_grouped_matmul_partial", a_sorted, w_packed, scale, counts_or_offsets)
    E, N, Kh = w_packed.shape
    M, K = a_sorted.shape
    assert K % group_size == 0 and K == Kh * 2
    G = K // group_size
    off = _offsets(counts_or_offsets, E, "int4_grouped_matmul_partial")
    adt = dt_code(a_sorted.dtype, "int4_grouped_matmul_partial")
    a = rows(a_sorted)
    w = w_packed if w_packed.is_contiguous() else w_packed.contiguous()
    if scale.dtype not in (torch.float32, torch.float16):
        scale = scale.to(torch.float32)
    sc = scale if scale.is_contiguous() else scale.contiguous()
    part = torch.empty(splits, M, N, dtype=torch.float32, device=dev)
    kernels.check(kernels.lib().mls_int4_grouped_gemm_partial(
        a.data_ptr(), adt, ld(a), off.data_ptr(), E, M, w.data_ptr(), N * Kh, Kh, sc.data_ptr(),
        dt_code(sc.dtype, "int4_grouped_matmul_partial scale"), N * G, G, 1, group_size, splits,
        part.data_ptr(), N, M * N, N, K, stream(dev)), "int4_grouped_matmul_partial")
    return part


def int4_expert_mlp_combine(a_sorted: torch.Tensor, counts_or_offsets: torch.Tensor,
                            wg: torch.Tensor, sg: torch.Tensor, wu: torch.Tensor, su: torch.Tensor,
                            wd: torch.Tensor, sd: torch.Tensor, group_size: int,
                            weights: torch.Tensor, pos: torch.Tensor,
                            a_rows: torch.Tensor | None = None) -> torch.Tensor:
    """The routed MoE layer after routing: the INT4 SwiGLU expert MLP of every segment
    (int4_expert_mlp) and the router-weighted combine back to token order
    (kernels/moe_routing.py:144-153). With a_rows (sort_by_expert's token_of_slot),
    a_sorted is the unsorted token matrix [T, D] and the dispatch gather happens inside the
    gate/up kernel's activation load. When the down projection's output is narrow (few
    column tiles), it runs as fp32 partial products over K splits that the combine adds,
    so that it still fills the GPU. Returns [T, D] in a_sorted's dtype."""
    from kernels.moe_routing import combine_partials, combine_rows
    E = wg.shape[0]
    off = _offsets(counts_or_offsets, E, "int4_expert_mlp_combine")
    h = int4_grouped_gate_up(a_sorted, wg, sg, wu, su, off, group_size, a_rows=a_rows)
    D, H = wd.shape[1], wd.shape[2] * 2
    splits = grouped_splits(h.shape[0], E, D, H, group_size)
    if splits > 1:
        part = int4_grouped_matmul_partial(h, wd, sd, off, group_size, splits)
        return combine_partials(part, weights, pos, a_sorted.dtype)
    return combine_rows(int4_grouped_matmul(h, wd, sd, off, group_size), weights, pos)
