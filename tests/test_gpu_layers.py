"""The drop-in layers on the GPU: QuantLinear, quantize_model, the INT8 STE and
FP8Linear use the gfx950 kernels and agree with their reference paths."""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from oracle import ref

from kernels.int8_ste import Int8MatmulSTE, QuantLinearSTE
from serve.quantize import QuantLinear, dequantize_int8, quantize_int8, quantize_model

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _close(out, want, what):
    o, w = out.detach().float().cpu().numpy(), want.detach().float().cpu().numpy()
    ok, worst = ref.close_fp32(o, w) if out.dtype == torch.float32 else ref.close_bf16(o, w)
    assert ok, f"{what}: worst {worst:.3g}"


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 5, 8, 64, 300])   # draft, verify (gamma+1), batch, prompt
def test_quantlinear_kernel_vs_reference_path(dev, bits, dtype, M):
    torch.manual_seed(M + bits)
    lin = nn.Linear(512, 384, bias=False)
    qk = QuantLinear(lin, bits=bits, group_size=128, use_kernel=True).to(dev)
    qr = QuantLinear(lin, bits=bits, group_size=128, use_kernel=False).to(dev)
    x = torch.randn(M, 512, device=dev)
    # the reference path rounds dequantized weights to x.dtype; compare against fp32 math
    want = x.to(dtype).float() @ qr.dequant().t()
    _close(qk(x.to(dtype)), want, f"QuantLinear bits={bits} {dtype} M={M}")


def test_quantize_model_on_device_matches_host_quantization(dev):
    from test_host import _Model  # toy model with the reference's slot names
    m = _Model()
    host = quantize_model(m, bits=4, group_size=32, use_kernel=False)
    dq = quantize_model(m.to(dev), bits=4, group_size=32, use_kernel=True)
    for a, b in zip(host.modules(), dq.modules()):
        if isinstance(a, QuantLinear):
            assert torch.equal(a.w_q, b.w_q.cpu()) and torch.equal(a.scale, b.scale.cpu())
    x = torch.randn(3, 64, device=dev)
    blk = dq.blocks[0]
    _close(blk.attn.wq(x), x @ host.blocks[0].attn.wq.dequant().to(dev).t(), "quantized model slot")


def test_int8_ste_matches_reference(dev):
    """test_backward.py:151-170 on the device."""
    torch.manual_seed(1)
    x = torch.randn(9, 32, device=dev, requires_grad=True)
    w = torch.randn(24, 32, device=dev)
    w_q, s = quantize_int8(w)
    master = w.clone().requires_grad_(True)
    y = Int8MatmulSTE.apply(x, w_q, s, master)
    dy = torch.randn_like(y)
    y.backward(dy)
    x2 = x.detach().clone().requires_grad_(True)
    ref_y = x2 @ dequantize_int8(w_q, s).t()
    ref_y.backward(dy)
    _close(y.detach(), ref_y.detach(), "STE forward")
    _close(x.grad, x2.grad, "STE input grad")
    _close(master.grad, dy.t() @ x.detach(), "STE master grad")


def test_quant_ste_linear_grads(dev):
    """QuantLinearSTE (reference kernels/autograd_ops.py:120-134) on a 3-d input: the
    forward quantizes the fp32 master on the device and runs int8_matmul, the input
    gradient is int8_dgrad of the re-quantized weight and the master receives dy^T x."""
    torch.manual_seed(3)
    lin = QuantLinearSTE(48, 40).to(dev)
    x = torch.randn(2, 7, 48, device=dev, requires_grad=True)
    y = lin(x)
    assert y.shape == (2, 7, 40)
    w_q, s = quantize_int8(lin.weight.detach().cpu())  # host quantizer: bit-identical bytes
    wd = dequantize_int8(w_q, s).to(dev)
    _close(y.detach(), x.detach() @ wd.t(), "QuantLinearSTE forward")
    dy = torch.randn_like(y)
    y.backward(dy)
    _close(x.grad, dy @ wd, "QuantLinearSTE input grad")
    _close(lin.weight.grad, dy.reshape(-1, 40).t() @ x.detach().reshape(-1, 48), "QuantLinearSTE master grad")


def test_quant_ste_linear_learns(dev):
    """test_backward.py:173-190 on the device: a toy regression through the INT8 kernel
    forward and the int8_dgrad backward must collapse the loss."""
    torch.manual_seed(2)
    w_true = torch.randn(16, 32, device=dev)
    lin = QuantLinearSTE(32, 16).to(dev)
    opt = torch.optim.Adam(lin.parameters(), lr=3e-2)
    first = last = None
    for step in range(150):
        x = torch.randn(64, 32, device=dev)
        loss = ((lin(x) - x @ w_true.t()) ** 2).mean()
        opt.zero_grad()
        loss.backward()
        opt.step()
        if step == 0:
            first = loss.item()
        last = loss.item()
    assert last < first * 0.1, f"loss {first:.3f} -> {last:.3f}"


def test_fp8_linear_kernel_vs_emulation(dev):
    from train.fp8 import FP8Linear
    torch.manual_seed(2)
    lin = nn.Linear(256, 192, bias=False)
    fk = FP8Linear(lin, use_kernel=True).to(dev)
    fe = FP8Linear(lin, use_kernel=False).to(dev)
    x = torch.randn(70, 256, device=dev)
    _close(fk(x), fe(x), "FP8Linear forward")


def test_greedy_decode_tokens_identical(dev):
    """The engine / speculative call pattern (M = 1 draft steps, M = gamma + 1 verify,
    M = batch, M = prompt length) through a stack of QuantLinear layers: greedy tokens
    from the kernel path equal those of the use_kernel=False path."""
    torch.manual_seed(3)
    d, vocab = 256, 96
    emb = torch.randn(vocab, d, device=dev) * 0.5
    layers = [nn.Linear(d, d, bias=False) for _ in range(3)]
    head = torch.randn(vocab, d, device=dev) * 0.1
    for bits in (8, 4):
        stacks = {uk: [QuantLinear(l, bits=bits, group_size=64, use_kernel=uk).to(dev) for l in layers]
                  for uk in (True, False)}

        def run(uk, toks):
            h = emb[toks]
            for q in stacks[uk]:
                h = torch.tanh(q(h))
            return (h @ head.t()).argmax(-1)

        for M in (1, 5, 4, 40):
            toks = torch.randint(0, vocab, (M,), device=dev)
            for _ in range(6):
                a, b = run(True, toks), run(False, toks)
                assert torch.equal(a, b), f"bits={bits} M={M}"
                toks = a


def test_quantized_checkpoint_on_device(dev, tmp_path):
    """Quantize on the GPU, save, load straight onto the GPU: identical buffers and
    identical kernel outputs; a host-quantized checkpoint loads to the same bytes (the
    GPU quantizers are bit-exact); MoE experts come back stacked for the grouped path."""
    from serve.quantize import load_quantized, save_quantized, stacked_int4_experts
    from test_host import _Model
    torch.manual_seed(5)
    m = _Model()
    qd = quantize_model(m.to(dev), bits=4, group_size=32, use_kernel=True)
    path = tmp_path / "q4.safetensors"
    save_quantized(qd, path)
    loaded = load_quantized(_Model(), path, device=dev)
    for k, v in qd.state_dict().items():
        w = loaded.state_dict()[k]
        assert w.device.type == "cuda" and torch.equal(v, w), k
    x = torch.randn(5, 64, device=dev).to(torch.bfloat16)
    assert torch.equal(loaded.blocks[0].attn.wo(x), qd.blocks[0].attn.wo(x))
    assert stacked_int4_experts(loaded.blocks[1].mlp.experts) is not None
    # a checkpoint written from a host-quantized model holds the same bytes
    hpath = tmp_path / "q4_host.safetensors"
    save_quantized(quantize_model(m.cpu(), bits=4, group_size=32, use_kernel=False), hpath)
    hl = load_quantized(_Model(), hpath, device=dev)
    for k, v in loaded.state_dict().items():
        assert torch.equal(v, hl.state_dict()[k]), k


class _SwiGLU(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.w_gate, self.w_up = nn.Linear(d, h, bias=False), nn.Linear(d, h, bias=False)
        self.w_down = nn.Linear(h, d, bias=False)

    def forward(self, x):
        return self.w_down(torch.nn.functional.silu(self.w_gate(x)) * self.w_up(x))


class _Mix(nn.Module):
    """A per-token stand-in for attention with the reference's four slots:
    wo(wv(x) * sigmoid(wq(x) + wk(x)))."""

    def __init__(self, d):
        super().__init__()
        self.wq, self.wk, self.wv, self.wo = (nn.Linear(d, d, bias=False) for _ in range(4))

    def forward(self, x):
        return self.wo(self.wv(x) * torch.sigmoid(self.wq(x) + self.wk(x)))


class _Blk(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.attn, self.mlp = _Mix(d), _SwiGLU(d, h)

    def forward(self, x):
        x = x + self.attn(x)
        return x + self.mlp(x)


class _Net(nn.Module):
    """Input projection and head in full precision, two residual blocks with the
    reference's block layout and slot names (what quantize_model swaps)."""

    def __init__(self, d_in=64, d=128, h=256, classes=10):
        super().__init__()
        self.inp = nn.Linear(d_in, d, bias=False)
        self.blocks = nn.ModuleList(_Blk(d, h) for _ in range(2))
        self.head = nn.Linear(d, classes, bias=False)

    def forward(self, x):
        z = self.inp(x)
        for b in self.blocks:
            z = b(z)
        return self.head(z)


def test_quantized_model_accuracy(dev):
    """test_quantize.py:62-85 of the reference on the kernel path: train briefly in fp32,
    then the INT8 (INT4 g32) quantized model, run through the HIP kernels, loses at most
    3% (30%) of cross-entropy."""
    import torch.nn.functional as F
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(4096, 64, generator=g, device=dev)
    y = (x @ torch.randn(64, 10, generator=g, device=dev)).argmax(1)
    torch.manual_seed(5)
    m = _Net().to(dev)
    opt = torch.optim.Adam(m.parameters(), lr=1e-3)
    gb = torch.Generator(device=dev).manual_seed(1)
    for _ in range(60):
        idx = torch.randint(0, 4096, (64,), generator=gb, device=dev)
        loss = F.cross_entropy(m(x[idx]), y[idx])
        opt.zero_grad()
        loss.backward()
        opt.step()
    xe = x[:512].to(torch.bfloat16)
    with torch.no_grad():
        fp = float(F.cross_entropy(m.to(torch.bfloat16)(xe).float(), y[:512]))
        q8 = quantize_model(m, bits=8, use_kernel=True)
        q4 = quantize_model(m, bits=4, group_size=32, use_kernel=True)
        l8 = float(F.cross_entropy(q8(xe).float(), y[:512]))
        l4 = float(F.cross_entropy(q4(xe).float(), y[:512]))
    assert sum(isinstance(mm, QuantLinear) for mm in q8.modules()) == 14
    assert l8 < fp * 1.03, f"int8 {l8:.4f} vs fp {fp:.4f}"
    assert l4 < fp * 1.30, f"int4 {l4:.4f} vs fp {fp:.4f}"
