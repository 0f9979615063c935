"""Weight-only quantization: INT8 (per-row symmetric) and INT4 (group-wise).

Same functions, classes and buffer layouts as the reference's serve/quantize.py
(:18-129), so a serving engine built on nn.Linear slots runs unchanged:

INT8: scale[n] = max|w[n]| / 127 (floored at 1e-8); w_q = round-half-even(w / scale)
      clamped to [-127, 127].
INT4: per group of `group_size` along K, scale = max|w_group| / 7 (floored at
      1e-8); q = clamp(round(w / scale), -8, 7) + 8, two nibbles per byte with
      even k in the low nibble.

Quantization is load-time work. On HIP tensors it runs the gfx950 quantizer
kernels (bit-exact: IEEE division, ties to even); on host tensors (a model
quantized before it is moved to the GPU, as the reference's CLI does) it runs
the reference's host op sequence, which is the definition the kernels match.
QuantLinear(use_kernel=True) runs the fused HIP GEMMs of kernels.dequant_matmul;
use_kernel=False keeps the reference's dequantize-then-matmul path.

Unlike the reference, this module does not import the model package (the
reference imports train.model only for a type annotation, :15): quantize_model
finds the Linear slots by attribute name.
"""

from __future__ import annotations

import torch
import torch.nn as nn


def _hip_quantizer():
    import kernels
    from kernels._hip import ld, stream
    return kernels, ld, stream


def quantize_int8(w: torch.Tensor):
    """(w_q int8 [N, K], scale fp32 [N]) -- serve/quantize.py:18-21."""
    if w.device.type != "cuda":
        scale = (w.abs().amax(dim=1) / 127.0).clamp(min=1e-8)
        w_q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
        return w_q, scale
    kernels, ld, stream = _hip_quantizer()
    w32 = w.detach().to(torch.float32)
    if w32.stride(1) != 1:
        w32 = w32.contiguous()
    N, K = w32.shape
    w_q = torch.empty(N, K, dtype=torch.int8, device=w.device)
    scale = torch.empty(N, dtype=torch.float32, device=w.device)
    kernels.check(kernels.lib().mls_quantize_int8(
        w32.data_ptr(), N, K, ld(w32), w_q.data_ptr(), ld(w_q), scale.data_ptr(),
        stream(w.device)), "quantize_int8")
    return w_q, scale


def dequantize_int8(w_q: torch.Tensor, scale: torch.Tensor):
    return w_q.float() * scale[:, None]


def quantize_int4(w: torch.Tensor, group_size: int = 32):
    """(packed uint8 [N, K/2], scale fp32 [N, K/group_size]) -- serve/quantize.py:28-36."""
    N, K = w.shape
    assert K % group_size == 0
    if w.device.type != "cuda" or group_size % 2 or K % 2:
        g = w.reshape(N, K // group_size, group_size)
        scale = (g.abs().amax(dim=2) / 7.0).clamp(min=1e-8)
        q = torch.round(g / scale[:, :, None]).clamp(-8, 7) + 8
        q = q.reshape(N, K).to(torch.uint8)
        packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
        return packed, scale
    kernels, ld, stream = _hip_quantizer()
    w32 = w.detach().to(torch.float32)
    if w32.stride(1) != 1:
        w32 = w32.contiguous()
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=w.device)
    scale = torch.empty(N, K // group_size, dtype=torch.float32, device=w.device)
    kernels.check(kernels.lib().mls_quantize_int4(
        w32.data_ptr(), N, K, ld(w32), group_size, packed.data_ptr(), ld(packed),
        scale.data_ptr(), stream(w.device)), "quantize_int4")
    return packed, scale


def dequantize_int4(packed: torch.Tensor, scale: torch.Tensor, group_size: int):
    N = packed.shape[0]
    K = packed.shape[1] * 2
    q = torch.empty(N, K, dtype=torch.uint8, device=packed.device)
    q[:, 0::2] = packed & 0x0F
    q[:, 1::2] = packed >> 4
    w = q.float() - 8.0
    w = w.reshape(N, K // group_size, group_size) * scale.float()[:, :, None]
    return w.reshape(N, K)


class QuantLinear(nn.Module):
    """Drop-in nn.Linear replacement holding quantized weights (serve/quantize.py:50-95).

    use_kernel=True runs the fused gfx950 dequant GEMM; False runs the
    reference path (explicit dequant then matmul), kept for correctness tests
    and host execution.
    """

    def __init__(self, linear: nn.Linear, bits: int = 8, group_size: int = 32,
                 use_kernel: bool = True):
        super().__init__()
        assert linear.bias is None
        assert bits in (4, 8)
        self.bits, self.group_size, self.use_kernel = bits, group_size, use_kernel
        self.out_features, self.in_features = linear.weight.shape
        w = linear.weight.detach().float()
        if bits == 8:
            w_q, scale = quantize_int8(w)
        else:
            w_q, scale = quantize_int4(w, group_size)
        self.register_buffer("w_q", w_q)
        self.register_buffer("scale", scale)

    @classmethod
    def from_quantized(cls, w_q: torch.Tensor, scale: torch.Tensor, bits: int, group_size: int,
                       in_features: int, use_kernel: bool = True) -> "QuantLinear":
        """A QuantLinear around buffers that are already quantized (a quantized
        checkpoint): no fp weight, no quantization pass."""
        assert bits in (4, 8)
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.bits, self.group_size, self.use_kernel = bits, group_size, use_kernel
        self.out_features, self.in_features = w_q.shape[0], in_features
        want = in_features if bits == 8 else in_features // 2
        if w_q.dim() != 2 or w_q.shape[1] != want:
            raise ValueError(f"QuantLinear.from_quantized: w_q {tuple(w_q.shape)} does not hold "
                             f"{in_features} int{bits} columns")
        self.register_buffer("w_q", w_q)
        self.register_buffer("scale", scale)
        return self

    def dequant(self) -> torch.Tensor:
        if self.bits == 8:
            return dequantize_int8(self.w_q, self.scale)
        return dequantize_int4(self.w_q, self.scale, self.group_size)

    def weight_bytes(self) -> int:
        return self.w_q.numel() * self.w_q.element_size() + \
            self.scale.numel() * self.scale.element_size()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.reshape(-1, self.in_features)
        if self.use_kernel:
            from kernels.dequant_matmul import int4_matmul, int8_matmul
            if self.bits == 8:
                y = int8_matmul(flat, self.w_q, self.scale)
            else:
                y = int4_matmul(flat, self.w_q, self.scale, self.group_size)
        else:
            y = flat @ self.dequant().to(flat.dtype).t()
        return y.reshape(*shape[:-1], self.out_features)


_ATTN_SLOTS = ("wq", "wk", "wv", "wo")
_MLP_SLOTS = ("w_gate", "w_up", "w_down")


def quantize_model(model: nn.Module, bits: int = 8, group_size: int = 32,
                   use_kernel: bool = True) -> nn.Module:
    """Replace all block linears with QuantLinear (router/embed/head stay fp)
    (serve/quantize.py:98-115). Walks model.blocks; each block's .attn holds
    wq/wk/wv/wo and its .mlp holds w_gate/w_up/w_down, or, when blk.is_moe,
    .mlp.experts is a list of such MLPs."""
    import copy
    model = copy.deepcopy(model)
    for blk in model.blocks:
        a = blk.attn
        for name in _ATTN_SLOTS:
            setattr(a, name, QuantLinear(getattr(a, name), bits, group_size, use_kernel))
        mods = blk.mlp.experts if getattr(blk, "is_moe", False) else [blk.mlp]
        for m in mods:
            for name in _MLP_SLOTS:
                setattr(m, name, QuantLinear(getattr(m, name), bits, group_size, use_kernel))
        if getattr(blk, "is_moe", False):
            stacked_int4_experts(mods)
    return model


def _expert_slots_ok(experts) -> bool:
    """True when every expert is a SwiGLU MLP (w_down(silu(w_gate(x)) * w_up(x)),
    train/model.py:127-135) whose three projections are INT4 QuantLinear running the
    HIP kernels, with one shape, group size, scale dtype and device across experts, and
    shapes the grouped MFMA kernels take (K % 64 == 0, group % 32 == 0)."""
    if len(experts) == 0:
        return False
    ref = None
    for m in experts:
        lins = [getattr(m, n, None) for n in _MLP_SLOTS]
        if not all(isinstance(q, QuantLinear) and q.bits == 4 and q.use_kernel for q in lins):
            return False
        sig = tuple((tuple(q.w_q.shape), tuple(q.scale.shape), q.scale.dtype, q.group_size, q.w_q.device)
                    for q in lins)
        if ref is None:
            ref = sig
        elif sig != ref:
            return False
    g, u, d = ref
    D, H, group, dev = g[0][1] * 2, g[0][0], g[3], g[4]
    return (dev.type == "cuda" and u == g and d[0] == (D, H // 2) and group % 32 == 0
            and D % 64 == 0 and H % 64 == 0 and g[2] in (torch.float32, torch.float16))


def stacked_int4_experts(experts):
    """Stacked INT4 buffers of a list of SwiGLU experts, for the grouped kernels of
    kernels.moe_grouped: {"w_gate": (packed [E, H, D/2], scale [E, H, D/group]),
    "w_up": (...), "w_down": (packed [E, D, H/2], scale [E, D, H/group]),
    "group_size": g}, or None when the experts do not qualify (_expert_slots_ok).

    The stack is built once: each slot's buffers are copied into one [E, ...] tensor
    and every expert's QuantLinear buffers are re-pointed at views of it, so the
    per-expert modules and the stacked tensors share memory. Later calls only check
    that the buffers are still those views (they are not after .to() or a
    load_state_dict that replaced them) and rebuild when they are not."""
    if not _expert_slots_ok(experts):
        return None
    first = experts[0]
    st = first.__dict__.get("_int4_stack")
    if st is not None and len(st["experts"]) == len(experts) and all(
            a is b for a, b in zip(st["experts"], experts)):
        ok = True
        for name in _MLP_SLOTS:
            wq, sc = st[name]
            for e, m in enumerate(experts):
                q = getattr(m, name)
                if q.w_q.data_ptr() != wq[e].data_ptr() or q.scale.data_ptr() != sc[e].data_ptr():
                    ok = False
                    break
            if not ok:
                break
        if ok:
            return st
    st = {"experts": list(experts), "group_size": first.w_gate.group_size}
    with torch.no_grad():
        for name in _MLP_SLOTS:
            lins = [getattr(m, name) for m in experts]
            wq = torch.stack([q.w_q for q in lins]).contiguous()
            sc = torch.stack([q.scale for q in lins]).contiguous()
            for e, q in enumerate(lins):
                q.w_q = wq[e]
                q.scale = sc[e]
            st[name] = (wq, sc)
    first.__dict__["_int4_stack"] = st
    return st


def model_weight_bytes(model: nn.Module) -> int:
    """Bytes of QuantLinear buffers plus every distinct parameter (serve/quantize.py:118-129)."""
    total = 0
    seen = set()
    for m in model.modules():
        if isinstance(m, QuantLinear):
            total += m.weight_bytes()
    for p in model.parameters():
        if id(p) in seen:
            continue
        seen.add(id(p))
        total += p.numel() * p.element_size()
    return total


# ------------------------------------------------------------------ quantized checkpoints
#
# The reference saves the fp state dict and quantizes again at every load
# (serve/api.py:47, 79-81). A quantized checkpoint stores the QuantLinear buffers
# themselves (w_q, scale: serve/quantize.py:68-73) next to the model's fp parameters,
# in a safetensors file (plain tensors + a string header; loading executes nothing),
# so a load is a copy to the device and quantization runs once, on the GPU.
#
# Header ("__metadata__"): format = "mls-quantized", version = "1", and per quantized
# module "q:<module name>" = "<bits>,<group_size>,<in_features>". Tensors: the model's
# state dict (the QuantLinear buffers under their state-dict names, every other
# parameter and buffer as stored), each saved as its own contiguous copy.

QCKPT_FORMAT, QCKPT_VERSION = "mls-quantized", "1"


def save_quantized(model: nn.Module, path, extra_metadata: dict | None = None) -> None:
    """Write a model whose linears are QuantLinear (quantize_model's output) to a
    quantized safetensors checkpoint at `path`."""
    from safetensors.torch import save_file
    meta = {"format": QCKPT_FORMAT, "version": QCKPT_VERSION}
    for name, m in model.named_modules():
        if isinstance(m, QuantLinear):
            meta[f"q:{name}"] = f"{m.bits},{m.group_size},{m.in_features}"
    if len(meta) == 2:
        raise ValueError("save_quantized: the model holds no QuantLinear (run quantize_model first)")
    for k, v in (extra_metadata or {}).items():
        if k in meta or k.startswith("q:"):
            raise ValueError(f"save_quantized: metadata key {k!r} is reserved")
        meta[k] = str(v)
    tensors = {k: v.detach().contiguous().clone() for k, v in model.state_dict().items()}
    save_file(tensors, str(path), metadata=meta)


def read_quantized_metadata(path) -> dict:
    """The string header of a quantized checkpoint (format, version, modules, extras)."""
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        meta = dict(f.metadata() or {})
    if meta.get("format") != QCKPT_FORMAT:
        raise ValueError(f"{path}: not a quantized checkpoint (format {meta.get('format')!r})")
    if meta.get("version") != QCKPT_VERSION:
        raise ValueError(f"{path}: quantized checkpoint version {meta.get('version')!r}, "
                         f"this build reads {QCKPT_VERSION!r}")
    return meta


def _set_submodule(model: nn.Module, name: str, mod: nn.Module) -> None:
    parent, _, leaf = name.rpartition(".")
    setattr(model.get_submodule(parent) if parent else model, leaf, mod)


def load_quantized(model: nn.Module, path, device=None, use_kernel: bool = True) -> nn.Module:
    """Load a quantized checkpoint into `model` (the fp architecture, e.g. a freshly
    built Transformer; it is modified in place and returned): every module the header
    lists becomes a QuantLinear holding the stored buffers, then the remaining
    parameters load as a state dict (strict: missing or unexpected keys raise). With
    `device`, tensors are read straight onto it. MoE experts are stacked for the
    grouped kernels as quantize_model does."""
    from safetensors.torch import load_file
    meta = read_quantized_metadata(path)
    dev = torch.device(device) if device is not None else None
    tensors = load_file(str(path), device=str(dev) if dev is not None else "cpu")
    for key, spec in meta.items():
        if not key.startswith("q:"):
            continue
        name = key[2:]
        bits, group, in_features = (int(x) for x in spec.split(","))
        old = model.get_submodule(name)
        if not isinstance(old, (nn.Linear, QuantLinear)):
            raise ValueError(f"load_quantized: {name} is a {type(old).__name__}, not a linear layer")
        w_q, scale = tensors.pop(f"{name}.w_q"), tensors.pop(f"{name}.scale")
        out_features = old.out_features
        if w_q.shape[0] != out_features or in_features != old.in_features:
            raise ValueError(f"load_quantized: {name} stores {w_q.shape[0]}x{in_features}, "
                             f"the model has {out_features}x{old.in_features}")
        _set_submodule(model, name, QuantLinear.from_quantized(w_q, scale, bits, group, in_features, use_kernel))
    if dev is not None:
        model.to(dev)
    missing, unexpected = model.load_state_dict(tensors, strict=False)
    quant_keys = {k for k in model.state_dict() if k.endswith((".w_q", ".scale"))
                  and isinstance(model.get_submodule(k.rsplit(".", 1)[0]), QuantLinear)}
    missing = [k for k in missing if k not in quant_keys]
    if missing or unexpected:
        raise ValueError(f"load_quantized: missing {missing[:5]}, unexpected {unexpected[:5]}")
    for blk in getattr(model, "blocks", []):
        if getattr(blk, "is_moe", False):
            stacked_int4_experts(blk.mlp.experts)
    return model
