"""Benchmark of the gfx950 quantized-linear hot path; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps 512] [--warmup 64] [--only NAME] [--no-extra] [--no-cpu]

Headline: INT4 g128 decode GEMV, M = 1, K = N = 4096,
bf16 activations, fp16 group scales, bf16 output. A step is one launch over one
batch; consecutive steps read distinct copies of the packed weights (>= 1 GiB of
copies in total), so the 256 MB Infinity Cache cannot serve them and the data
really streams from HBM. The W warmup steps and the K timed steps are captured
back to back as one HIP graph, with a one-thread kernel that reads the GPU's
constant-rate realtime counter just before and just after the K timed steps; the
graph is replayed once and the elapsed time is the counter difference, so the
graph's own launch cost (~11.6 us per replay) stays outside it. The timed steps
start at the copy after the last warmup one, so no timed step re-reads what
warmup just read. value = algorithmic bytes x K / elapsed.

Parity gate (the reference refuses to benchmark when an on-device check fails,
kaggle/kaggle_bench.py:46-54): before a workload is timed, one of its outputs is
checked against torch fp32 arithmetic on the decoded operands on the GPU (sampled
rows for the large configs) under BASELINE's rule for that output: bf16 / fp16
|d| <= 1e-2 + 1e-2 |ref|; fp32 |d| <= 2^-9 max(|ref|, rms(ref)); quantizers bit
for bit. A row that fails carries no throughput. The headline failing ends the
run with no value. The native fp8 datapath is known to exceed config D's bf16
rule (its accumulation truncates); its rows are timed and marked
within_config_tolerance = false.

The other BASELINE configs (INT4 M = 4 / 16, the INT8 GEMV target, INT8 prefill,
FP8 e4m3 GEMM, INT4 MoE grouped GEMM), INT4 and INT8 at M = 2 (a speculative
decoding verify step with one draft token), the whole INT4 SwiGLU expert MLP of a
routed MoE layer, FP8Linear's backward at config D's shape, paged-attention
decode, the load-time INT4 quantizer and the reference's own published
bench_quantize shapes (N = K = 2048, fp16, M in {1, 16, 128}) are reported under
"extra" with the same protocol, followed by a 256 MiB streaming copy and, as
calibration only, the vendor library's GEMMs on config D's shape.

cpu_baseline times the reference's PyTorch CPU path (oracle/torch_cpu.py: the
QuantLinear(use_kernel=False) dequantize-then-matmul, and the FP8 linear's
emulation) on the host for a bounded sample: the headline layer, config C and
config D.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "mini-llm-stack_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "INT4/INT8/FP8 GEMM: HBM TB/s at M=1, TFLOP/s at M=2048 (% of roofline)"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
ROTATE_BYTES = 1 << 30
TRAFFIC_FILE = "profiles/traffic.json"

# bench_quantize.py's published T4 latencies (bench/results/quantize.json:30-118 of the
# reference), for the rows at its own shapes
REF_T4_MS = {("int8", 1): 1.2003, ("int4", 1): 0.879, ("int8", 16): 1.2098, ("int4", 16): 0.869,
             ("int8", 128): 4.0002, ("int4", 128): 1.9409}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- timing


WARM_MS = 50.0  # eager launches of each workload's steps ahead of its timed replay, ms
EAGER_TOO_MS = 0.05  # steps at least this long are also timed as eager launches
LAST_EAGER_MS = None  # that time for the last workload timed, ms per step
STAMP_GAPS = 5  # stamp-to-stamp gaps measured per timing, median subtracted
STAMP_GAP_US: list = []  # the stamp launch cost measured by each graph-timed workload
EAGER = False  # --eager: plain launches instead of graph replay (for counter collection)


_FLOOR_LIB = None


def _floor_lib():
    """libmls_floor.so: bench.py's calibration kernels (csrc/floor.hip), not the product."""
    global _FLOOR_LIB
    if _FLOOR_LIB is None:
        import ctypes
        lib = ctypes.CDLL(str(ROOT / "mini-llm-stack_amd" / "libmls_floor.so"))
        lib.mlsf_stamp.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.mlsf_wallclock_khz.argtypes = [ctypes.POINTER(ctypes.c_int)]
        _FLOOR_LIB = lib
    return _FLOOR_LIB


def time_steps(fns, warmup: int, steps: int) -> float:
    """ms per step: `warmup` then `steps` launches, fns[i % len(fns)] for step i
    (the timed steps continue the rotation where warmup stopped).

    The warmup and timed steps are captured as one HIP graph with a timestamp kernel
    (the GPU's constant-rate realtime counter, libmls_floor.so's mlsf_stamp) before and
    after the timed steps, and replayed once; the interval between the stamps holds the
    timed steps plus one stamp launch. That launch's share (~1.45 us, 0.07 us per step
    at K = 20) is measured in the same graph as the median gap between STAMP_GAPS + 1
    stamps launched back to back just before the first timed step, and subtracted.
    Timing the replay with events instead would add the graph's own launch cost,
    ~11.6 us per replay on the GPU (the headline GEMV: 3.68 + 11.6 / K us per step).
    Events around the whole replay check the stamps.

    The graph is replayed once untimed, the steps are launched eagerly for WARM_MS of
    wall time (many replays queued back to back made later replays of short-step
    graphs slower: the empty kernel 1.5 -> 4.9 us per launch), then every copy is read
    once more (1 GiB or more for the GEMVs, so the
    256 MB MALL no longer holds what the timed steps read), then timed: this library's
    kernels speed up over the first tens of milliseconds of sustained work, whether
    launched eagerly or replayed (INT8 prefill launched eagerly on one box: 0.199-0.203
    ms per step after 4 warmup steps, 0.177 ms after 64, 0.167-0.171 ms after 256), so
    a short run would time the ramp rather than the kernels."""
    import ctypes
    import torch
    n = len(fns)
    for f in fns:  # first calls: library load, LDS attributes, output pools
        f()
    torch.cuda.synchronize()
    if EAGER:
        for i in range(warmup):
            fns[i % n]()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for i in range(steps):
            fns[(warmup + i) % n]()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    lib = _floor_lib()
    khz = ctypes.c_int(0)
    if lib.mlsf_wallclock_khz(ctypes.byref(khz)) != 0 or khz.value <= 0:
        raise RuntimeError("bench: cannot read the GPU's realtime counter rate")
    stamps = torch.zeros(STAMP_GAPS + 2, dtype=torch.int64, device="cuda")

    def stamp(j, st):
        if lib.mlsf_stamp(ctypes.c_void_p(stamps.data_ptr() + 8 * j), ctypes.c_void_p(st)) != 0:
            raise RuntimeError("bench: timestamp launch failed")

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(warmup):
            fns[i % n]()
        for j in range(STAMP_GAPS + 1):
            stamp(j, st)
        for i in range(steps):
            fns[(warmup + i) % n]()
        stamp(STAMP_GAPS + 1, st)
    g.replay()  # rehearsal (see above)
    torch.cuda.synchronize()
    deadline, i = time.perf_counter() + WARM_MS * 1e-3, 0
    while time.perf_counter() < deadline:  # sustained work: eager launches, 16 at a time
        fns[i % n]()
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    for f in fns:  # every copy once more, so the timed steps' copies have left the MALL
        f()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    t = [int(v) for v in stamps.cpu()]
    gaps = sorted(t[j + 1] - t[j] for j in range(STAMP_GAPS))
    gap = gaps[STAMP_GAPS // 2]
    raw = (t[-1] - t[-2]) / khz.value
    ms = raw - gap / khz.value
    whole = start.elapsed_time(end)
    if not (gaps[0] > 0 and 0 < ms and raw <= whole * 1.001 + 0.01):
        raise RuntimeError(f"bench: timestamps {raw:.4f} ms (stamp gap {gap / khz.value:.4f} ms) "
                           f"inconsistent with the replay's {whole:.4f} ms")
    STAMP_GAP_US.append(gap / khz.value * 1e3)
    global LAST_EAGER_MS
    LAST_EAGER_MS = None
    if ms / steps >= EAGER_TOO_MS:  # long steps: also the same steps launched one by one
        for i in range(warmup):
            fns[i % n]()
        torch.cuda.synchronize()
        start.record()
        for i in range(steps):
            fns[(warmup + i) % n]()
        end.record()
        torch.cuda.synchronize()
        LAST_EAGER_MS = start.elapsed_time(end) / steps
    return ms / steps


def clocked_steps(fns, warmup: int, steps: int, waves: int) -> dict:
    """Execution spans of `steps` launches of a clocked kernel copy (libmls_floor.so), with
    time_steps' protocol (one graph of warmup + timed steps, one untimed replay, WARM_MS of
    eager launches, every copy once more, then the timed replay). fns[i](clocks_ptr)
    launches step i's kernel, whose every wavefront stores its {t0, t1} realtime clocks
    (first instruction; all memory operations complete) at clocks_ptr; timed step i
    writes its own slice, all other launches a scratch slice. Per timed launch: start =
    min t0, end = max t1, exec = end - start; across launches: period = start_(i+1) -
    start_i (the launch-to-launch time, what time_steps measures), gap = start_(i+1) -
    end_i (from the last wavefront's end to the next launch's first wavefront)."""
    import ctypes
    import torch
    lib = _floor_lib()
    khz = ctypes.c_int(0)
    if lib.mlsf_wallclock_khz(ctypes.byref(khz)) != 0 or khz.value <= 0:
        raise RuntimeError("bench: cannot read the GPU's realtime counter rate")
    n = len(fns)
    clocks = torch.zeros(steps + 1, waves, 2, dtype=torch.int64, device="cuda")
    base, slot = clocks.data_ptr(), waves * 16
    scratch = base + steps * slot
    for f in fns:
        f(scratch)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(warmup):
            fns[i % n](scratch)
        for i in range(steps):
            fns[(warmup + i) % n](base + i * slot)
    g.replay()
    torch.cuda.synchronize()
    deadline, i = time.perf_counter() + WARM_MS * 1e-3, 0
    while time.perf_counter() < deadline:
        fns[i % n](scratch)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    for f in fns:
        f(scratch)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    c = clocks[:steps].double().cpu()
    if bool((c[:, :, 0] == 0).any()) or bool((c[:, :, 1] < c[:, :, 0]).any()):
        raise RuntimeError("bench: a clocked launch left wavefront clocks unwritten or out of order")
    us = 1e3 / khz.value
    t0, t1 = c[:, :, 0], c[:, :, 1]
    start, end = t0.min(1).values, t1.max(1).values
    exec_ = (end - start) * us
    period = (start[1:] - start[:-1]) * us
    gap = (start[1:] - end[:-1]) * us
    med = lambda v: float(v.median())
    return {"exec_us": round(float(exec_.mean()), 3), "exec_us_median": round(med(exec_), 3),
            "period_us": round(float(period.mean()), 3), "gap_us": round(float(gap.mean()), 3),
            "gap_us_median": round(med(gap), 3),
            "ramp_us": round(float(((t0.max(1).values - start) * us).mean()), 3),
            "wave_us": round(float(((t1 - t0) * us).mean()), 3), "waves": waves, "launches": steps,
            "tick_us": round(us, 4)}


def graph_events_ms(fns, warmup: int, steps: int) -> float:
    """ms per step of `steps` launches captured in one graph and timed with events around
    a single replay (after one untimed replay): a cross-check of time_steps that needs no
    stamp kernel; the replay's own launch cost (~11.6 us) is spread over all steps."""
    import torch
    n = len(fns)
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(warmup + steps):
            fns[i % n]()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (warmup + steps)


def wall_median_ms(fn, warmup: int = 3, iters: int = 30) -> float:
    """The reference's own timing protocol (bench/_util.py:36-51): median host wall time
    of one call followed by a device synchronize."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


# ----------------------------------------------------------------------------- parity gate


def _deq8(q, s):
    return q.float() * s.float()[:, None]


def _deq4(p, s, gs):
    import torch
    N = p.shape[0]
    w = torch.stack(((p & 15).float() - 8.0, (p >> 4).float() - 8.0), dim=-1).reshape(N, -1)
    return (w.reshape(N, -1, gs) * s.float()[:, :, None]).reshape(N, -1)


def _fp8(bits, s, fmt="e4m3"):
    import torch
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    return bits.view(dt).float() * s


def gate(out, want, rule: str) -> dict:
    """BASELINE's tolerance for one output: the largest |d| / bound (<= 1 passes)."""
    import torch
    o, w = out.float(), want.float()
    if rule == "exact":
        bad = int((out != want).sum())
        return {"rule": "bit-exact", "ok": bad == 0, "mismatches": bad}
    if rule == "bf16":
        bound = 1e-2 + 1e-2 * w.abs()
        desc = "|d| <= 1e-2 + 1e-2|ref|"
    else:
        rms = float(w.double().pow(2).mean().sqrt())
        bound = (2.0 ** -9) * torch.clamp(w.abs(), min=rms)
        desc = "|d| <= 2^-9 max(|ref|, rms(ref))"
    ratio = ((o - w).abs() / bound.clamp(min=1e-30)).nan_to_num(nan=float("inf"))
    worst = float(ratio.max()) if ratio.numel() else 0.0
    return {"rule": desc, "ok": worst <= 1.0, "worst_ratio": round(worst, 4), "checked": int(o.numel())}


def _rows(M: int, n: int = 64):
    """Sampled row indices: the first, the last and evenly spread ones."""
    if M <= n:
        return list(range(M))
    step = (M - 1) / (n - 1)
    return sorted({int(round(i * step)) for i in range(n)})


# ----------------------------------------------------------------------------- workloads


def int4_gemv(dev, M: int, steps: int, warmup: int, N: int = 4096, K: int = 4096, gs: int = 128,
              act=None, scale_dtype=None, wstd: float = 0.02, seed: int = 0):
    import torch
    from kernels.dequant_matmul import int4_matmul
    from serve.quantize import quantize_int4
    act = act or torch.bfloat16
    scale_dtype = scale_dtype or torch.float16
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(act)
    p, s = quantize_int4(torch.randn(N, K, generator=g, device=dev) * wstd, gs)
    s = s.to(scale_dtype)
    par = gate(int4_matmul(x, p, s, gs), x.float() @ _deq4(p, s, gs).t(), "bf16" if act != torch.float32 else "fp32")
    wbytes = p.numel() + s.numel() * s.element_size()
    copies = max(2, -(-ROTATE_BYTES // wbytes))
    ps = [p] + [p.clone() for _ in range(copies - 1)]
    ss = [s] + [s.clone() for _ in range(copies - 1)]
    fns = [lambda i=i: int4_matmul(x, ps[i], ss[i], gs) for i in range(copies)]
    ms = None
    if par["ok"]:
        ms = time_steps(fns, warmup, steps)
    nbytes = wbytes + M * K * x.element_size() + M * N * x.element_size()
    return dict(ms=ms, bytes=nbytes, flops=2 * M * N * K, copies=copies, parity=par, call=fns[0])


def int8_gemv(dev, M: int, steps: int, warmup: int, N: int = 4096, K: int = 4096, act=None,
              scale_dtype=None, wstd: float = 0.02, seed: int = 1):
    import torch
    from kernels.dequant_matmul import int8_matmul
    from serve.quantize import quantize_int8
    act = act or torch.bfloat16
    scale_dtype = scale_dtype or torch.float16
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(act)
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * wstd)
    s = s.to(scale_dtype)
    par = gate(int8_matmul(x, q, s), x.float() @ _deq8(q, s).t(), "bf16" if act != torch.float32 else "fp32")
    wbytes = q.numel() + s.numel() * s.element_size()
    copies = max(2, -(-ROTATE_BYTES // wbytes))
    qs = [q] + [q.clone() for _ in range(copies - 1)]
    fns = [lambda i=i: int8_matmul(x, qs[i], s) for i in range(copies)]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    nbytes = wbytes + M * K * x.element_size() + M * N * x.element_size()
    return dict(ms=ms, bytes=nbytes, flops=2 * M * N * K, copies=copies, parity=par, call=fns[0])


def int8_prefill(dev, steps: int, warmup: int, M=2048, N=11008, K=4096, act=None):
    import torch
    from kernels.dequant_matmul import int8_matmul
    from serve.quantize import quantize_int8
    act = act or torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(2)
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
    s = s.to(torch.float16)
    copies = 6
    xs = [torch.randn(M, K, generator=g, device=dev).to(act) for _ in range(copies)]
    qs = [q] + [q.clone() for _ in range(copies - 1)]
    r = _rows(M)
    par = gate(int8_matmul(xs[0], q, s)[r], xs[0][r].float() @ _deq8(q, s).t(),
               "bf16" if act != torch.float32 else "fp32")
    fns = [lambda i=i: int8_matmul(xs[i], qs[i], s) for i in range(copies)]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    esz = xs[0].element_size()
    nbytes = N * K + N * 2 + M * K * esz + M * N * esz
    return dict(ms=ms, bytes=nbytes, flops=2 * M * N * K, copies=copies, parity=par)


def int4_prefill(dev, steps: int, warmup: int, M=2048, N=11008, K=4096, gs=128):
    """int4_matmul at config C's prefill shape (INT4 g128 weights, fp16 scales, bf16 x):
    the reference's INT4 QuantLinear on a 2048-token prompt (dequant_matmul.py:69-100)."""
    import torch
    from kernels.dequant_matmul import int4_matmul
    from serve.quantize import quantize_int4
    g = torch.Generator(device=dev).manual_seed(4)
    p, s = quantize_int4(torch.randn(N, K, generator=g, device=dev) * 0.02, gs)
    s = s.to(torch.float16)
    copies = 8
    xs = [torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    ps = [p] + [p.clone() for _ in range(copies - 1)]
    r = _rows(M)
    par = gate(int4_matmul(xs[0], p, s, gs)[r], xs[0][r].float() @ _deq4(p, s, gs).t(), "bf16")
    fns = [lambda i=i: int4_matmul(xs[i], ps[i], s, gs) for i in range(copies)]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    nbytes = N * K // 2 + N * (K // gs) * 2 + M * K * 2 + M * N * 2
    return dict(ms=ms, bytes=nbytes, flops=2 * M * N * K, copies=copies, parity=par)


def fp32_rows(dev, steps: int, warmup: int):
    """fp32 activations at the reference engine's call shapes (its serving path runs fp32
    end to end, serve/engine.py:166): M = 1 / 5 (decode of one / five sequences), 64 (a
    prefill chunk), 2048 (a long prompt), K = N = 4096, INT4 g128 and INT8 with fp16
    scales; and config C's INT8 prefill (2048 x 11008 x 4096) in fp32. M = 1 runs the
    VALU GEMV, larger M the bf16 hi + lo split on the matrix cores."""
    import torch
    out = []
    small = max(8, steps // 8)
    for bits in (4, 8):
        for M in (1, 5, 64, 2048):
            fn = int4_gemv if bits == 4 else int8_gemv
            r = fn(dev, M, steps if M <= 64 else small, warmup if M <= 64 else 4, act=torch.float32,
                   seed=40 + M + bits)
            name = f"fp32_int{bits}{'_g128' if bits == 4 else ''}_m{M}_4096x4096"
            row = _mfma_row(name, r, BF16_PEAK_TFLOPS) if M >= 2048 else _hbm_row(name, r)
            if row.get("ms_per_step") is not None and M >= 2048:
                row["hbm_frac"] = round(r["bytes"] / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            row["path"] = ("VALU GEMV (fp32 FMAs)" if M == 1 else
                           "bf16 hi + lo split, skinny MFMA GEMV" if M <= 16 else "bf16 hi + lo split, bf16 MFMA")
            out.append(row)
    r = int8_prefill(dev, small, 4, act=torch.float32)
    row = _mfma_row("fp32_int8_prefill_2048x11008x4096", r, BF16_PEAK_TFLOPS,
                    {"path": "bf16 hi + lo split, bf16 MFMA (two MFMAs per bf16 one)"})
    out.append(row)
    return out


def floor_rows(dev, steps: int, warmup: int, nbytes=8_667_136, copies=125, blocks=256):
    """The single-launch floor of the M = 1 GEMV rows (calibration kernels of
    mini-llm-stack_amd/libmls_floor.so, not this build's product): an empty kernel with the
    GEMV's grid, and a pure streaming read of the headline's bytes per launch, timed with the
    GEMV's protocol (one HIP graph over `copies` rotated buffers). The GEMV cannot go below
    the stream row's time; the empty row is the part of every launch that moves no data."""
    import ctypes
    import torch
    lib = ctypes.CDLL(str(ROOT / "mini-llm-stack_amd" / "libmls_floor.so"))
    lib.mlsf_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
    lib.mlsf_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mlsf_stream_store.argtypes = lib.mlsf_stream.argtypes
    g = torch.Generator(device=dev).manual_seed(9)
    bufs = [torch.randint(0, 2**31 - 1, (nbytes // 4,), generator=g, device=dev, dtype=torch.int32)
            for _ in range(copies)]
    sink = torch.zeros(1024 * 8, dtype=torch.int32, device=dev)  # 8 bytes per wavefront of 1024 blocks

    def st():
        return torch.cuda.current_stream(dev).cuda_stream

    def call(rc):
        if rc != 0:
            raise RuntimeError(f"floor kernel launch failed ({rc})")

    ms_empty = time_steps([lambda: call(lib.mlsf_empty(blocks, st()))], warmup, steps)
    best = None
    for nb in (256, 512, 1024):  # blocks of 4 wavefronts (the INT4 GEMV: 256, INT8: 512)
        if nbytes // 16 > nb * 4 * 64 * 16:  # the stream kernel issues at most 16 loads per lane
            continue
        fns = [lambda b=b, nb=nb: call(lib.mlsf_stream(b.data_ptr(), nbytes, nb, sink.data_ptr(), st()))
               for b in bufs]
        ms = time_steps(fns, warmup, steps)
        if best is None or ms < best[0]:
            best = (ms, nb)
    ms, nb_best = best
    gbs = nbytes / (ms * 1e-3) / 1e9
    # the same read at the GEMV's grid, every wavefront then storing one 8-byte word as the
    # GEMV does: what a launch that also writes its result costs
    fns = [lambda b=b: call(lib.mlsf_stream_store(b.data_ptr(), nbytes, blocks, sink.data_ptr(), st()))
           for b in bufs]
    ms_st = time_steps(fns, warmup, steps)
    gbs_st = nbytes / (ms_st * 1e-3) / 1e9
    note = "calibration kernels (libmls_floor.so), not this build's product; timed like the M=1 GEMV"
    return [{"name": f"floor_empty_kernel_{blocks}_blocks", "ms_per_step": round(ms_empty, 6), "note": note},
            {"name": f"floor_stream_read_{nbytes}B", "ms_per_step": round(ms, 6), "TB/s": round(gbs / 1e3, 4),
             "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbs / HBM_PEAK_GBS, 4)},
             "blocks": nb_best, "buffers_rotated": copies, "note": note},
            {"name": f"floor_stream_read_store_{nbytes}B", "ms_per_step": round(ms_st, 6),
             "TB/s": round(gbs_st / 1e3, 4),
             "roofline": {"bound": "hbm", "achieved": round(gbs_st, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbs_st / HBM_PEAK_GBS, 4)},
             "blocks": blocks, "buffers_rotated": copies, "stored_bytes": blocks * 4 * 8, "note": note}]


def clock_rows(dev, steps: int, warmup: int, long_steps: int = 2000):
    """Where an M = 1 step's time goes: the library's INT4 (headline) and INT8 GEMVs and
    the floor kernels at the same sizes and grids, as clocked copies (libmls_floor.so:
    gemv1.h's kernel body, or the calibration kernel, with realtime clocks read by every
    wavefront at its first instruction and after its last memory operation completed).
    Each row gives the copy's execution span per launch (first wavefront's start to last
    wavefront's end), the launch-to-launch period and the gap between launches, next to
    the library kernel's own step time from time_steps in the same run and, for the
    GEMVs, from events around one graph replay of `long_steps` launches. The clocked
    GEMV copies must reproduce the library's output bit for bit before they are timed."""
    import ctypes
    import torch
    from kernels.dequant_matmul import int4_matmul, int8_matmul
    from serve.quantize import quantize_int4, quantize_int8
    lib = _floor_lib()
    lib.mlsf_gemv1_clocked.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mlsf_empty_clocked.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mlsf_stream_clocked.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    N = K = 4096

    def st():
        return torch.cuda.current_stream(dev).cuda_stream

    def call(rc, want=0):
        if rc != want:
            raise RuntimeError(f"clocked kernel launch returned {rc}, expected {want}")

    out = []
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(1, K, generator=g, device=dev).to(torch.bfloat16)
    for bits in (4, 8):
        if bits == 4:
            w, s = quantize_int4(torch.randn(N, K, generator=g, device=dev) * 0.02, 128)
            lib_fn = lambda w, s: int4_matmul(x, w, s, 128)
            ld_sn, group, waves = s.stride(0), 128, N // 4
        else:
            w, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
            lib_fn = lambda w, s: int8_matmul(x, w, s)
            ld_sn, group, waves = 1, 0, N
        s = s.to(torch.float16)
        wbytes = w.numel() + s.numel() * 2
        nbytes = wbytes + 2 * K * 2
        copies = max(2, -(-ROTATE_BYTES // wbytes))
        ws = [w] + [w.clone() for _ in range(copies - 1)]
        ss = [s] + [s.clone() for _ in range(copies - 1)]
        y = torch.empty(1, N, dtype=torch.bfloat16, device=dev)
        clk = torch.zeros(waves, 2, dtype=torch.int64, device=dev)
        call(lib.mlsf_gemv1_clocked(bits, x.data_ptr(), w.data_ptr(), w.stride(0), s.data_ptr(), ld_sn, group,
                                    y.data_ptr(), N, K, 0, clk.data_ptr(), st()), waves)
        same = bool(torch.equal(y, lib_fn(w, s)))
        row = {"name": f"clocks_int{bits}_gemv_m1_4096x4096", "bytes_per_step": nbytes,
               "clocked_copy_bit_identical_to_library": same}
        if same:
            ms_lib = time_steps([lambda i=i: lib_fn(ws[i], ss[i]) for i in range(copies)], warmup, steps)
            ms_ev = graph_events_ms([lambda i=i: lib_fn(ws[i], ss[i]) for i in range(copies)], warmup, long_steps)
            def fns(wait):
                return [lambda p, i=i: call(lib.mlsf_gemv1_clocked(bits, x.data_ptr(), ws[i].data_ptr(),
                                                                   ws[i].stride(0), ss[i].data_ptr(), ld_sn, group,
                                                                   y.data_ptr(), N, K, wait, p, st()), waves)
                        for i in range(copies)]
            ck = clocked_steps(fns(0), warmup, steps, waves)
            ckw = clocked_steps(fns(1), warmup, steps, waves)
            row.update({"library_step_us": round(ms_lib * 1e3, 3),
                        f"library_step_us_events_{long_steps}_launches": round(ms_ev * 1e3, 3),
                        "clocked": ck, "clocked_memory_end": ckw,
                        "exec_TB/s": round(nbytes / (ck["exec_us"] * 1e-6) / 1e12, 4),
                        "exec_frac": round(nbytes / (ck["exec_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "step_frac": round(nbytes / (ms_lib * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        out.append(row)
        del ws, ss
        # the floor kernels at the same bytes and grid: an empty launch, a pure streaming read,
        # and the read with one 8-byte store per wavefront
        blocks = waves // 4
        gb = torch.Generator(device=dev).manual_seed(9)
        nb = (nbytes + 15) // 16 * 16
        bcopies = max(2, -(-ROTATE_BYTES // nb))
        bufs = [torch.randint(0, 2**31 - 1, (nb // 4,), generator=gb, device=dev, dtype=torch.int32)
                for _ in range(bcopies)]
        sink = torch.zeros(blocks * 8, dtype=torch.int32, device=dev)
        kinds = [("empty", None), ("stream_read", 0), ("stream_read_store", 1)]
        for kind, store in kinds:
            def sfns(wait):
                if store is None:
                    return [lambda p: call(lib.mlsf_empty_clocked(blocks, p, st()))]
                return [lambda p, b=b: call(lib.mlsf_stream_clocked(b.data_ptr(), nb, blocks, sink.data_ptr(), store,
                                                                    wait, p, st())) for b in bufs]
            ck = clocked_steps(sfns(0), warmup, steps, waves)
            r = {"name": f"clocks_floor_{kind}_{blocks}_blocks" + ("" if store is None else f"_{nb}B"),
                 "clocked": ck, "note": "calibration kernel (libmls_floor.so), clocked"}
            if store is not None:
                r["clocked_memory_end"] = clocked_steps(sfns(1), warmup, steps, waves)
                r["exec_TB/s"] = round(nb / (ck["exec_us"] * 1e-6) / 1e12, 4)
                r["period_TB/s"] = round(nb / (ck["period_us"] * 1e-6) / 1e12, 4)
            out.append(r)
        del bufs
    return out


def int8_dgrad_row(dev, steps: int, warmup: int, M=4096, N=11008, K=4096):
    """The INT8 STE backward's input gradient at a training shape (kernels/dequant_matmul.py:
    103-132): dx [M, K] = (dy [M, N] * s) @ W_q [N, K], bf16 dy. One step is the whole op:
    dy * s to bf16, the transposed weight copy, and the GEMM."""
    import torch
    from kernels.dequant_matmul import int8_dgrad
    from serve.quantize import quantize_int8
    g = torch.Generator(device=dev).manual_seed(5)
    q, s = quantize_int8(torch.randn(N, K, generator=g, device=dev) * 0.02)
    copies = 3
    dys = [torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    qs = [q] + [q.clone() for _ in range(copies - 1)]
    r = _rows(M)
    # the reference's arithmetic: dy * s rounded to bf16, then the dot (dequant_matmul.py:128)
    par = gate(int8_dgrad(dys[0], q, s)[r],
               (dys[0][r].float() * s.float()[None, :]).to(torch.bfloat16).float() @ q.float(), "bf16")
    fns = [lambda i=i: int8_dgrad(dys[i], qs[i], s) for i in range(copies)]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    nbytes = M * N * 2 + N * K + N * 4 + M * K * 2
    return dict(ms=ms, bytes=nbytes, flops=2 * M * N * K, copies=copies, parity=par)


def fp8_gemm(dev, steps: int, warmup: int, M=4096, N=8192, K=8192, native=False):
    import torch
    from kernels.fp8_matmul import E4M3_MAX, fp8_matmul, quantize_e4m3
    g = torch.Generator(device=dev).manual_seed(3)
    copies = 4
    ops = []
    for _ in range(copies):
        a = torch.randn(M, K, generator=g, device=dev)
        a = torch.where(torch.rand(M, K, generator=g, device=dev) < 0.01, a * 20, a)
        b = torch.randn(N, K, generator=g, device=dev)
        b = torch.where(torch.rand(N, K, generator=g, device=dev) < 0.01, b * 20, b)
        sa, sb = a.abs().amax(1) / E4M3_MAX, b.abs().amax(1) / E4M3_MAX
        ops.append((quantize_e4m3(a, sa[:, None]), quantize_e4m3(b, sb[:, None]), sa, sb))
        del a, b
    ab, bb, sa, sb = ops[0]
    r = _rows(M)
    out = fp8_matmul(ab, bb, sa, sb, out_dtype=torch.bfloat16, native=native)[r]
    par = gate(out, _fp8(ab[r], sa[r, None]) @ _fp8(bb, sb[:, None]).t(), "bf16")
    fns = [lambda o=o: fp8_matmul(o[0], o[1], o[2], o[3], out_dtype=torch.bfloat16, native=native)
           for o in ops]
    ms = time_steps(fns, warmup, steps) if (par["ok"] or native) else None
    nbytes = M * K + N * K + 4 * (M + N) + M * N * 2
    return dict(ms=ms, bytes=nbytes, flops=2 * M * N * K, copies=copies, parity=par)


def fp8_backward(dev, steps: int, warmup: int, M=4096, N=8192, K=8192, native=False):
    """FP8Linear's backward at config D's shape (train/fp8.py:80-95): dy [M,N] to e5m2,
    dx = dy W (dy times W^T [K,N]), dw = dy^T x (dy^T [N,M] times x^T [K,M]), as
    train/fp8.py runs it: dy encoded once in both layouts; x^T and W^T come from the
    forward's encode (which writes both layouts), like the saved operands; two
    2*M*N*K GEMMs. The scale of dy is taken as given (the
    reference reads it on the host before this work starts)."""
    import torch
    from kernels.fp8_matmul import E4M3_MAX, E5M2_MAX, fp8_matmul, quantize_e4m3_t, quantize_e5m2_t
    g = torch.Generator(device=dev).manual_seed(7)
    copies = 2
    sets = []
    for _ in range(copies):
        x = torch.randn(M, K, generator=g, device=dev)
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        dy = torch.randn(M, N, generator=g, device=dev) * 1e-3
        sx, sw = float(x.abs().amax()) / E4M3_MAX, float(w.abs().amax()) / E4M3_MAX
        sdy = float(dy.abs().amax()) / E5M2_MAX
        # the forward encodes x and W into both layouts and keeps the transposes
        sets.append((quantize_e4m3_t(x, sx)[1], quantize_e4m3_t(w, sw)[1], dy, sx, sw, sdy))

    def step(xbt, wbt, dy, sx, sw, sdy):
        dyb, dybt = quantize_e5m2_t(dy, sdy)
        dx = fp8_matmul(dyb, wbt, sdy, sw, torch.float32, native=native, a_format="e5m2")
        dw = fp8_matmul(dybt, xbt, sdy, sx, torch.float32, native=native, a_format="e5m2")
        return dx, dw

    xbt, wbt, dy, sx, sw, sdy = sets[0]
    dx, dw = step(*sets[0])
    dyh = _fp8(quantize_e5m2_t(dy, sdy)[0], sdy, "e5m2")
    rm, rn = _rows(M), _rows(N)
    p1 = gate(dx[rm], dyh[rm] @ _fp8(wbt, sw).t(), "fp32")
    p2 = gate(dw[rn], dyh[:, rn].t() @ _fp8(xbt, sx).t(), "fp32")
    par = {"dx": p1, "dw": p2, "ok": p1["ok"] and p2["ok"]}
    del dx, dw, dyh
    fns = [lambda st=st: step(*st) for st in sets]
    ms = time_steps(fns, warmup, steps) if (par["ok"] or native) else None
    nbytes = M * N * 4 + 2 * (M * N + N * K + M * K) + (M * K + N * K) * 4
    return dict(ms=ms, bytes=nbytes, flops=2 * 2 * M * N * K, copies=copies, parity=par)


def paged_attn(dev, steps: int, warmup: int, S=64, H=32, D=128, ctx=2048, bs=16):
    """Paged-attention decode (kernels/paged_attention.py): S sequences of `ctx` cached
    tokens each, H heads of D, bf16 pools in blocks of `bs` tokens handed out in a
    shuffled order (as a long-running pool fragments). HBM-bound on the K/V reads."""
    import torch
    from kernels.paged_attention import paged_attention_decode
    g = torch.Generator(device=dev).manual_seed(8)
    nb = S * ctx // bs
    kp = torch.randn(nb, H, bs, D, generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn(nb, H, bs, D, generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
    tables = perm.reshape(S, ctx // bs).contiguous()
    lens = torch.full((S,), ctx, dtype=torch.int32, device=dev)
    q = torch.randn(S, H, D, generator=g, device=dev).to(torch.bfloat16)
    out = paged_attention_decode(q, kp, vp, tables, lens)
    got, want = [], []
    for si in _rows(S, 8):
        blocks = tables[si].long()
        k = kp[blocks].float().permute(1, 0, 2, 3).reshape(H, ctx, D)
        v = vp[blocks].float().permute(1, 0, 2, 3).reshape(H, ctx, D)
        att = torch.softmax((k @ q[si].float()[:, :, None]).squeeze(-1) * D ** -0.5, dim=-1)
        want.append((att[:, None, :] @ v).squeeze(1))
        got.append(out[si])
    par = gate(torch.stack(got), torch.stack(want), "bf16")
    fns = [lambda: paged_attention_decode(q, kp, vp, tables, lens)]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    nbytes = 2 * S * ctx * H * D * 2 + 2 * S * H * D * 2 + S * (ctx // bs) * 4 + S * 4
    return dict(ms=ms, bytes=nbytes, flops=4 * S * H * ctx * D, copies=1, parity=par)


def _int4_experts(dev, g, E, n, k, gs):
    import torch
    from serve.quantize import quantize_int4
    P, S = [], []
    for _ in range(E):
        p, s = quantize_int4(torch.randn(n, k, generator=g, device=dev) * 0.02, gs)
        P.append(p)
        S.append(s.to(torch.float16))
    return torch.stack(P), torch.stack(S)


def _segment_rows(counts, per: int = 8):
    """Sampled rows of each expert's segment (its first and last `per // 2`) and the expert."""
    rows_, experts, start = [], [], 0
    for e, c in enumerate(counts):
        pick = sorted(set(list(range(start, start + min(c, per // 2))) +
                          list(range(max(start, start + c - per // 2), start + c))))
        rows_ += pick
        experts += [e] * len(pick)
        start += c
    return rows_, experts


def moe_int4(dev, steps: int, warmup: int, T=512, D=4096, E=8, H=14336, gs=128):
    """Config E: the grouped INT4 GEMM of every expert segment, the dispatch gather inside
    its activation load. The routing metadata (segment offsets, int32 row index) is made
    once, before the timed steps, as a MoE layer makes it once for its GEMMs."""
    import torch
    from kernels.moe_grouped import int4_grouped_matmul, segment_offsets
    from kernels.moe_routing import gather_rows, route_topk, sort_by_expert
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    _, ex = route_topk(torch.randn(T, E, generator=g, device=dev), 2)
    tok, counts, _ = sort_by_expert(ex, E)
    a = gather_rows(x, tok)
    sets = [_int4_experts(dev, g, E, H, D, gs) for _ in range(2)]
    cl = counts.tolist()
    # the dispatch gather runs inside the grouped kernel's activation load (a_rows = tok)
    off, tok32 = segment_offsets(counts), tok.to(torch.int32)
    y = int4_grouped_matmul(x, sets[0][0], sets[0][1], off, gs, a_rows=tok32)
    rs, es = _segment_rows(cl)
    want = torch.empty(len(rs), H, device=dev)
    for e in sorted(set(es)):
        sel = [i for i, ee in enumerate(es) if ee == e]
        want[sel] = a[[rs[i] for i in sel]].float() @ _deq4(sets[0][0][e], sets[0][1][e], gs).t()
    par = gate(y[rs], want, "bf16")
    fns = [lambda st=st: int4_grouped_matmul(x, st[0], st[1], off, gs, a_rows=tok32) for st in sets]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    rows_ = T * 2
    nbytes = E * H * D // 2 + E * H * (D // gs) * 2 + rows_ * D * 2 + rows_ * H * 2
    return dict(ms=ms, bytes=nbytes, flops=2 * rows_ * H * D, copies=len(sets), counts=cl, parity=par)


def moe_mlp_int4(dev, steps: int, warmup: int, T=512, D=4096, E=8, H=14336, gs=128):
    """The whole INT4 SwiGLU expert MLP of a routed MoE layer after routing: the fused
    gate/up launch with the dispatch gather in its activation load (silu(x Wg^T) * x Wu^T),
    the down launch, and the weighted combine back to token order
    (kernels/moe_routing.py:144-153 with INT4 experts). The gate
    checks the gate/up output against fp32 silu(gate) * up, and the layer output
    against an fp32 down projection and combine of that bf16 h (one GEMM against its
    fp32 oracle at a time, as the tests do)."""
    import torch
    from kernels.moe_grouped import int4_expert_mlp_combine, int4_grouped_gate_up, segment_offsets
    from kernels.moe_routing import gather_rows, route_topk, sort_by_expert
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    w, ex = route_topk(torch.randn(T, E, generator=g, device=dev), 2)
    w = w.to(torch.bfloat16)
    tok, counts, pos = sort_by_expert(ex, E)
    a = gather_rows(x, tok)
    off = segment_offsets(counts)
    sets = []
    for _ in range(2):
        mats = []
        for n, k in ((H, D), (H, D), (D, H)):
            mats += list(_int4_experts(dev, g, E, n, k, gs))
        sets.append(mats)
    wg, sg, wu, su, wd, sd = sets[0]
    cl = counts.tolist()
    # the dispatch gather runs inside the gate/up kernel's activation load (a_rows = tok)
    h = int4_grouped_gate_up(x, wg, sg, wu, su, off, gs, a_rows=tok)
    y = int4_expert_mlp_combine(x, off, *sets[0], gs, w, pos, a_rows=tok)
    rs, es = _segment_rows(cl)
    hw = torch.empty(len(rs), H, device=dev)
    for e in sorted(set(es)):
        sel = [i for i, ee in enumerate(es) if ee == e]
        xr = a[[rs[i] for i in sel]].float()
        hw[sel] = torch.nn.functional.silu(xr @ _deq4(wg[e], sg[e], gs).t()) * (xr @ _deq4(wu[e], su[e], gs).t())
    p1 = gate(h[rs], hw, "bf16")
    expert_of_row = torch.repeat_interleave(torch.arange(E, device=dev), counts)
    toks = _rows(T, 16)
    want = torch.zeros(len(toks), D, device=dev)
    deq_d = {}
    for i, t in enumerate(toks):
        for kk in range(pos.shape[1]):
            r = int(pos[t, kk])
            e = int(expert_of_row[r])
            if e not in deq_d:
                deq_d[e] = _deq4(wd[e], sd[e], gs)
            want[i] += w[t, kk].float() * (h[r:r + 1].float() @ deq_d[e].t())[0]
    del deq_d
    p2 = gate(y[toks], want, "bf16")
    par = {"gate_up": p1, "down_combine": p2, "ok": p1["ok"] and p2["ok"]}
    tok32 = tok.to(torch.int32)  # routing metadata made once per layer
    fns = [lambda m=m: int4_expert_mlp_combine(x, off, *m, gs, w, pos, a_rows=tok32) for m in sets]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    rows_ = T * 2
    nbytes = 3 * (E * H * D // 2 + E * H * (D // gs) * 2) + rows_ * D * 2 * 2 + rows_ * H * 2 * 2 + T * D * 2
    return dict(ms=ms, bytes=nbytes, flops=6 * rows_ * H * D, copies=len(sets), counts=cl, parity=par)


def _quantize_int4_torch(w, gs):
    """serve/quantize.py:28-36's torch op sequence, on whatever device w lives."""
    import torch
    N, K = w.shape
    gr = w.reshape(N, K // gs, gs)
    scale = (gr.abs().amax(dim=2) / 7.0).clamp(min=1e-8)
    q = (torch.round(gr / scale[:, :, None]).clamp(-8, 7) + 8).reshape(N, K).to(torch.uint8)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous(), scale


def quantize_int4_load(dev, steps: int, warmup: int, N=14336, K=4096, gs=128):
    """Load-time INT4 quantization of one fp32 weight matrix on the GPU
    (serve/quantize.py:28-36 semantics, bit-exact): reads N*K fp32, writes the packed
    nibbles and fp32 group scales. The gate compares sampled rows with the reference's
    torch op sequence run on the host (its CLI quantizes there); whether torch's own
    device kernels give the same bytes is recorded beside it."""
    import torch
    from serve.quantize import quantize_int4
    g = torch.Generator(device=dev).manual_seed(6)
    copies = 2
    ws = [torch.randn(N, K, generator=g, device=dev) * 0.02 for _ in range(copies)]
    p, s = quantize_int4(ws[0], gs)
    r = _rows(N, 256)
    hp, hs = _quantize_int4_torch(ws[0][r].cpu(), gs)
    par = gate(p[r].cpu(), hp, "exact")
    par["scales_exact"] = bool(torch.equal(s[r].cpu(), hs))
    par["ok"] = par["ok"] and par["scales_exact"]
    dp, ds = _quantize_int4_torch(ws[0], gs)
    # the reference's op sequence run by torch on the GPU (tensor / float multiplies by a
    # rounded reciprocal there) does not give the CPU bytes this kernel reproduces
    par["torch_device_ops_same_bytes"] = bool(torch.equal(dp, p) and torch.equal(ds, s))
    par["torch_device_ops_differing_bytes"] = int((dp != p).sum())
    par["torch_device_ops_differing_scales"] = int((ds != s).sum())
    del dp, ds
    fns = [lambda w=w: quantize_int4(w, gs) for w in ws]
    ms = time_steps(fns, warmup, steps) if par["ok"] else None
    nbytes = N * K * 4 + N * K // 2 + N * (K // gs) * 4
    return dict(ms=ms, bytes=nbytes, flops=0, copies=copies, parity=par)


def copy_calibration(dev, steps: int, warmup: int, nbytes: int = 256 << 20):
    """A plain streaming kernel of known traffic (torch's elementwise bitwise_not over
    int32: reads nbytes, writes nbytes). Its rocprofv3 FETCH_SIZE / WRITE_SIZE
    readings calibrate those counters to bytes, and its rate is the HBM bandwidth a
    simple streaming kernel reaches on this GPU."""
    import torch
    copies = 4
    srcs = [torch.full((nbytes // 4,), i + 1, dtype=torch.int32, device=dev) for i in range(copies)]
    dst = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    fns = [lambda s=s: torch.bitwise_not(s, out=dst) for s in srcs]
    ms = time_steps(fns, warmup, steps)
    return dict(ms=ms, bytes=2 * nbytes, flops=0, copies=copies)


def vendor_gemm(dev, steps: int, warmup: int, kind: str, M=4096, N=8192, K=8192):
    """Calibration only, never the product path: the vendor library (hipBLASLt, through
    torch) on config D's shape, timed with the same protocol, so the fp8 rows can be read
    against what the platform's own GEMM reaches on the same GPU. kind: "fp8_rowwise"
    (torch._scaled_mm with per-row scales, config D's form), "fp8_tensorwise", or
    "bf16" (torch.matmul). Returns None when the library path is unavailable."""
    import torch
    g = torch.Generator(device=dev).manual_seed(5)
    try:
        if kind == "bf16":
            a = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
            b = torch.randn(N, K, generator=g, device=dev).to(torch.bfloat16).t().contiguous().t()
            fns = [lambda: torch.matmul(a, b.t())]
        else:
            a = torch.randn(M, K, generator=g, device=dev).to(torch.float8_e4m3fn)
            b = torch.randn(N, K, generator=g, device=dev).to(torch.float8_e4m3fn)
            if kind == "fp8_rowwise":
                sa, sb = torch.rand(M, 1, device=dev) + 0.5, torch.rand(1, N, device=dev) + 0.5
            else:
                sa, sb = torch.tensor(0.7, device=dev), torch.tensor(1.3, device=dev)
            fns = [lambda: torch._scaled_mm(a, b.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)]
        fns[0]()
        torch.cuda.synchronize()
    except Exception as ex:  # not every torch build routes these to the GPU library
        log(f"vendor {kind}: unavailable ({type(ex).__name__}: {str(ex)[:120]})")
        return None
    # eager launches (a 0.2 ms GEMM hides the launch cost; no library call under capture)
    for _ in range(warmup):
        fns[0]()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        fns[0]()
    end.record()
    torch.cuda.synchronize()
    return dict(ms=start.elapsed_time(end) / steps, bytes=0, flops=2 * M * N * K, copies=1)


# ----------------------------------------------------------------------------- CPU baseline


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on, capped by
    OMP_NUM_THREADS when set (the GPU box gives one GPU's job a share of its cores and
    sets that variable to the share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n


def _time_cpu(fn, budget_s: float, min_iters: int = 3, max_iters: int = 1000, warm: bool = True):
    import numpy as np
    if warm:
        fn()  # first call: allocator, thread pool
    times = []
    t_end = time.perf_counter() + budget_s
    while (time.perf_counter() < t_end or len(times) < min_iters) and len(times) < max_iters:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(budget_s: float = 8.0):
    """The reference's PyTorch CPU path (oracle/torch_cpu.py, restating
    QuantLinear(use_kernel=False) = dequantize to fp32, round to x's dtype, x @ W^T,
    serve/quantize.py:75-78, 94; and the FP8 linear's emulation, train/fp8.py:77) timed
    on this host's cores with torch's CPU kernels: the headline layer (INT4 g128, M = 1,
    K = N = 4096, bf16 x, fp16 scales) for ~budget_s, then configs C and D (full size,
    up to 3 iterations each). Quantization is load-time and outside the timed region."""
    import torch
    from oracle import torch_cpu as tc
    threads = cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    N = K = 4096
    x = torch.randn(1, K, generator=g).to(torch.bfloat16)
    p, s = _quantize_int4_torch(torch.randn(N, K, generator=g) * 0.02, 128)
    s = s.to(torch.float16)
    t, n = _time_cpu(lambda: tc.quant_linear(x, p, s, 4, 128), budget_s)
    nbytes = N * K // 2 + N * (K // 128) * 2 + K * 2 + N * 2
    head = {"value": round(nbytes / t / 1e12, 6), "unit": "TB/s", "cores": threads, "kind": "port",
            "sample": f"{n} iterations of the headline layer (M=1, K=N=4096, INT4 g128, bf16 x, fp16 scales) "
                      f"through the reference's torch CPU path (dequantize_int4 in fp32, .to(bf16), x @ W^T); "
                      f"median {t * 1e3:.2f} ms per layer, torch CPU kernels on {threads} threads"}
    rows_ = []
    # config C: INT8 prefill, 2048 x 11008 x 4096, bf16 x, fp16 scales
    M, N, K = 2048, 11008, 4096
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sc = (torch.rand(N, generator=g) * 1e-3 + 1e-4).to(torch.float16)
    xc = torch.randn(M, K, generator=g).to(torch.bfloat16)
    t, n = _time_cpu(lambda: tc.quant_linear(xc, q, sc, 8), budget_s, min_iters=1, max_iters=3, warm=False)
    rows_.append({"config": "C: INT8 prefill 2048x11008x4096 bf16 (QuantLinear use_kernel=False)",
                  "value": round(2 * M * N * K / t / 1e12, 4), "unit": "TFLOP/s", "ms": round(t * 1e3, 2),
                  "iterations": n})
    del q, xc
    # config D: e4m3 4096 x 8192 x 8192, per-row scales, fp32 emulation
    M, N, K = 4096, 8192, 8192
    ab = torch.randint(0, 256, (M, K), generator=g, dtype=torch.uint8)
    bb = torch.randint(0, 256, (N, K), generator=g, dtype=torch.uint8)
    ab[(ab & 0x7F) == 0x7F] = 0  # no NaN patterns, as the encoder never makes them
    bb[(bb & 0x7F) == 0x7F] = 0
    sa, sb = torch.rand(M, 1, generator=g) * 1e-2, torch.rand(N, 1, generator=g) * 1e-2
    t, n = _time_cpu(lambda: tc.fp8_linear_emulated(ab, bb, sa, sb), budget_s, min_iters=1, max_iters=3, warm=False)
    rows_.append({"config": "D: e4m3 4096x8192x8192 per-row scales (FP8 linear emulation, fp32)",
                  "value": round(2 * M * N * K / t / 1e12, 4), "unit": "TFLOP/s", "ms": round(t * 1e3, 2),
                  "iterations": n})
    head["configs"] = rows_
    return head


# ----------------------------------------------------------------------------- main


def _failed_row(name, r):
    return {"name": name, "parity": r["parity"], "ms_per_step": None,
            "note": "output outside the config's tolerance: not timed"}


def _hbm_row(name, r, extra=None):
    if r.get("ms") is None:
        return _failed_row(name, r)
    gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
    row = {"name": name, "ms_per_step": round(r["ms"], 6), "TB/s": round(gbs / 1e3, 4),
           "TFLOP/s": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 3),
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)},
           "bytes_per_step": r["bytes"], "weight_copies": r["copies"]}
    _eager_field(row)
    if "parity" in r:
        row["parity"] = r["parity"]
    row.update(extra or {})
    return row


def _mfma_row(name, r, peak, extra=None):
    if r.get("ms") is None:
        return _failed_row(name, r)
    tf = r["flops"] / (r["ms"] * 1e-3) / 1e12
    if extra and "bf16_roofline_frac" in extra:
        extra = dict(extra, bf16_roofline_frac=round(tf / BF16_PEAK_TFLOPS, 4))
    gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
    row = {"name": name, "ms_per_step": round(r["ms"], 6), "TFLOP/s": round(tf, 2),
           "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": peak, "unit": "TFLOP/s",
                        "frac": round(tf / peak, 4)},
           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "flops_per_step": r["flops"],
           "copies": r["copies"]}
    _eager_field(row)
    if "parity" in r:
        row["parity"] = r["parity"]
    row.update(extra or {})
    return row


def _eager_field(row):
    """The same steps launched one by one right after the graph timing (events around
    them): the graph replay does not flatter the long steps; eager launches at the same
    point give the same time per step."""
    global LAST_EAGER_MS
    if LAST_EAGER_MS is not None:
        row["eager_ms_per_step"] = round(LAST_EAGER_MS, 6)
        LAST_EAGER_MS = None


def _native_row(name, r, extra):
    row = _mfma_row(name, r, FP8_PEAK_TFLOPS, extra)
    row["within_config_tolerance"] = bool(r["parity"]["ok"])
    if not r["parity"]["ok"]:
        row["note"] = ("the fp8 MFMA adds products in groups of 8 with ~13-bit alignment (truncating); "
                       "outputs exceed config D's tolerance, so this rate is not a parity-valid result")
    return row


def ref_shape_rows(dev, steps: int, warmup: int):
    """The reference's bench_quantize.py latency table shapes (bench/bench_quantize.py:
    44-68): N = K = 2048, fp16 activations, w ~ N(0, 1), fp32 scales, INT8 and INT4 g64,
    M in {1, 16, 128}; timed with this bench's protocol and with the reference's own
    (median host wall time with a synchronize per call), beside its published T4 numbers."""
    import torch
    out = []
    for M in (1, 16, 128):
        for bits in (8, 4):
            fn = int8_gemv if bits == 8 else int4_gemv
            kw = dict(N=2048, K=2048, act=torch.float16, scale_dtype=torch.float32, wstd=1.0, seed=10 + M)
            if bits == 4:
                kw["gs"] = 64
            r = fn(dev, M, steps, warmup, **kw)
            name = f"ref_shape_int{bits}{'_g64' if bits == 4 else ''}_m{M}_2048x2048_fp16"
            row = _hbm_row(name, r)
            if r.get("ms") is not None:
                wall = wall_median_ms(r["call"])
                row["ms_reference_protocol"] = round(wall, 4)
                row["reference_T4_ms"] = REF_T4_MS[(f"int{bits}", M)]
                row["speedup_vs_reference_T4_same_protocol"] = round(REF_T4_MS[(f"int{bits}", M)] / wall, 1)
            out.append(row)
    return out


def unquantized_rows(dev, steps: int, warmup: int):
    """The reference's own comparison points (bench/bench_quantize.py:44-68, published in
    bench/results/quantize.json): the unquantized GEMM a @ W^T (fp16, through torch: the
    vendor library) and the anti-pattern that dequantizes all of W and then multiplies
    (serve/quantize.py:24-25, 94), at its shapes (N = K = 2048, M in {1, 16, 128}, fp16), and
    the unquantized bf16 GEMM at the headline's shape (M = 1, K = N = 4096). Same protocol
    as the fused rows (graph replay over >= 1 GiB of rotated weight copies; torch's calls
    captured like this build's), plus the reference's own (median host wall time of a call
    and a synchronize, bench/_util.py:36-51). Calibration only: the vendor library and
    torch's elementwise kernels, not this build's."""
    import torch
    from serve.quantize import dequantize_int8, quantize_int8
    out = []
    shapes = [(M, 2048, 2048, torch.float16, f"m{M}_2048x2048_fp16") for M in (1, 16, 128)]
    shapes.append((1, 4096, 4096, torch.bfloat16, "m1_4096x4096_bf16"))
    for M, N, K, dt, tag in shapes:
        g = torch.Generator(device=dev).manual_seed(60 + M + N)
        a = torch.randn(M, K, generator=g, device=dev).to(dt)
        w = torch.randn(N, K, generator=g, device=dev)
        wfp = w.to(dt)
        copies = max(2, -(-ROTATE_BYTES // (N * K * 2)))
        ws = [wfp] + [wfp.clone() for _ in range(copies - 1)]
        impls = {"fp_matmul": (lambda i: a @ ws[i].t(), N * K * 2 + (M * K + M * N) * 2)}
        if dt == torch.float16:
            q8, s8 = quantize_int8(w)
            q8s = [q8] + [q8.clone() for _ in range(max(2, -(-ROTATE_BYTES // (N * K))) - 1)]
            impls["dequant_then_matmul_int8"] = (
                lambda i: a @ dequantize_int8(q8s[i % len(q8s)], s8).to(dt).t(), N * K + N * 4 + (M * K + M * N) * 2)
        for impl, (fn, nbytes) in impls.items():
            n = copies if impl == "fp_matmul" else len(q8s)
            fns = [lambda i=i: fn(i) for i in range(n)]
            try:
                ms = time_steps(fns, warmup, steps)
                how = "graph"
            except Exception as ex:  # a library call that cannot be captured: eager launches
                log(f"{impl} {tag}: graph capture failed ({type(ex).__name__}); timing eager launches")
                torch.cuda.synchronize()
                for i in range(warmup):
                    fns[i % n]()
                st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                st.record()
                for i in range(steps):
                    fns[(warmup + i) % n]()
                en.record()
                torch.cuda.synchronize()
                ms = st.elapsed_time(en) / steps
                how = "eager"
            row = {"name": f"unquantized_{impl}_{tag}", "ms_per_step": round(ms, 6),
                   "TB/s": round(nbytes / (ms * 1e-3) / 1e12, 4),
                   "roofline": {"bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                                "unit": "GB/s", "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
                   "bytes_per_step": nbytes, "launch": how,
                   "ms_reference_protocol": round(wall_median_ms(fns[0]), 4),
                   "calibration": "torch / the vendor library, not this build's kernels"}
            out.append(row)
        del ws
    return out


def load_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic.json), if any."""
    f = ROOT / TRAFFIC_FILE
    if f.exists():
        try:
            return json.loads(f.read_text()).get(name, {}).get("bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--only", default=None,
                    help="run one workload: int4_gemv, int4_m4, int4_m16, int8_gemv, int8_prefill, int4_prefill, "
                         "fp8_gemm, fp8_native, fp8_bwd, fp8_bwd_native, moe_int4, moe_mlp_int4, paged_attn, "
                         "quantize_int4, ref_shapes, unquantized (the reference's fp16 / dequantize-then-matmul "
                         "comparison rows), fp32 (fp32 activations), clocks (M=1 step split), "
                         "copy (counter calibration), vendor_fp8_rowwise / vendor_fp8_tensorwise / "
                         "vendor_bf16 / vendor_bf16_prefill (hipBLASLt calibration), cpu (the CPU baseline alone)")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="launch steps one by one instead of replaying a HIP graph (profiling)")
    ap.add_argument("--warm-ms", type=float, default=50.0,
                    help="eager launches of each workload's steps ahead of its timed replay, ms")
    args = ap.parse_args(argv)
    global EAGER, WARM_MS
    EAGER = args.eager
    WARM_MS = max(0.0, args.warm_ms)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs on a single MI355X and has no "
              "multi-GPU path; use --gpus 1", file=sys.stderr)
        return 2

    import torch
    torch.backends.cuda.matmul.allow_tf32 = False  # the parity gate's references are true fp32
    dev = torch.device("cuda:0")
    small = max(8, args.steps // 8)
    runners = {
        "int4_gemv": lambda: _hbm_row("int4_gemv_m1", int4_gemv(dev, 1, args.steps, args.warmup)),
        "int4_m2": lambda: _hbm_row("int4_gemv_m2", int4_gemv(dev, 2, args.steps, args.warmup)),
        "int4_m4": lambda: _hbm_row("int4_gemv_m4", int4_gemv(dev, 4, args.steps, args.warmup)),
        "int4_m16": lambda: _hbm_row("int4_gemv_m16", int4_gemv(dev, 16, args.steps, args.warmup)),
        "int8_gemv": lambda: _hbm_row("int8_gemv_m1", int8_gemv(dev, 1, args.steps, args.warmup)),
        "int8_m2": lambda: _hbm_row("int8_gemv_m2", int8_gemv(dev, 2, args.steps, args.warmup)),
        "int8_prefill": lambda: _mfma_row("int8_prefill_2048x11008x4096",
                                          int8_prefill(dev, small, 4), BF16_PEAK_TFLOPS),
        "int4_prefill": lambda: _mfma_row("int4_prefill_2048x11008x4096_g128", int4_prefill(dev, small, 4),
                                          BF16_PEAK_TFLOPS),
        "int8_dgrad": lambda: _mfma_row("int8_dgrad_4096x11008x4096_bf16", int8_dgrad_row(dev, small, 4),
                                        BF16_PEAK_TFLOPS,
                                        {"launches": "dy*s to bf16, W_q^T copy, INT8 MFMA GEMM (unit scales)"}),
        "fp8_gemm": lambda: _mfma_row("fp8_e4m3_4096x8192x8192_exact", fp8_gemm(dev, small, 4),
                                      FP8_PEAK_TFLOPS, {"datapath": "e4m3 widened to bf16, bf16 MFMA",
                                                        "bf16_roofline_frac": None}),
        "fp8_native": lambda: _native_row("fp8_e4m3_4096x8192x8192_native",
                                          fp8_gemm(dev, small, 4, native=True),
                                          {"datapath": "fp8 MFMA (8-product groups, 13-bit alignment)"}),
        "fp8_bwd": lambda: _mfma_row("fp8_linear_backward_4096x8192x8192_exact", fp8_backward(dev, small, 4),
                                     FP8_PEAK_TFLOPS, {"datapath": "e5m2/e4m3 widened to bf16, bf16 MFMA",
                                                       "gemms": "dx = dy W, dw = dy^T x, + e5m2 encode of dy in both layouts (x^T, W^T saved by the forward)",
                                                       "bf16_roofline_frac": None}),
        "fp8_bwd_native": lambda: _native_row("fp8_linear_backward_4096x8192x8192_native",
                                              fp8_backward(dev, small, 4, native=True),
                                              {"datapath": "fp8 MFMA, bf8 x fp8 operands"}),
        "moe_int4": lambda: (lambda r: _mfma_row("moe_int4_grouped_1024x14336x4096", r,
                                                 BF16_PEAK_TFLOPS,
                                                 {"hbm_roofline_frac": round(
                                                     r["bytes"] / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                                                  if r.get("ms") else None,
                                                  "segments": r["counts"]}))(
            moe_int4(dev, small, 4)),
        "moe_mlp_int4": lambda: (lambda r: _mfma_row("moe_int4_swiglu_mlp_T512_k2_E8_4096x14336", r,
                                                     BF16_PEAK_TFLOPS,
                                                     {"hbm_roofline_frac": round(
                                                         r["bytes"] / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                                                      if r.get("ms") else None,
                                                      "launches": "gate/up + down + combine",
                                                      "segments": r["counts"]}))(
            moe_mlp_int4(dev, small, 4)),
        "paged_attn": lambda: _hbm_row("paged_attention_decode_64seq_32h_d128_ctx2048_bf16",
                                       paged_attn(dev, small, 4)),
        "quantize_int4": lambda: _hbm_row("quantize_int4_14336x4096_g128", quantize_int4_load(dev, small, 4)),
        "ref_shapes": lambda: ref_shape_rows(dev, max(64, args.steps // 4), 16),
        "copy": lambda: _hbm_row("copy_256MiB", copy_calibration(dev, small, 4)),
        "floor": lambda: (floor_rows(dev, args.steps, args.warmup)
                          + floor_rows(dev, args.steps, args.warmup, nbytes=16_801_792, copies=64,
                                       blocks=512)[1:]),
        "cpu": lambda: cpu_baseline(),
        "clocks": lambda: clock_rows(dev, args.steps, args.warmup),
        "fp32": lambda: fp32_rows(dev, args.steps, args.warmup),
        "unquantized": lambda: unquantized_rows(dev, max(64, args.steps // 4), 16),
    }
    for kind, peak in (("fp8_rowwise", FP8_PEAK_TFLOPS), ("fp8_tensorwise", FP8_PEAK_TFLOPS),
                       ("bf16", BF16_PEAK_TFLOPS)):
        runners["vendor_" + kind] = (lambda kind=kind, peak=peak: (lambda r: None if r is None else _mfma_row(
            f"vendor_hipblaslt_{kind}_4096x8192x8192", r, peak,
            {"calibration": "vendor library through torch, not this build's kernels"}))(
            vendor_gemm(dev, small, 4, kind)))
    # the unquantized bf16 GEMM at config C's shape, the INT8 prefill row's comparison point
    runners["vendor_bf16_prefill"] = lambda: (lambda r: None if r is None else _mfma_row(
        "vendor_hipblaslt_bf16_2048x11008x4096", r, BF16_PEAK_TFLOPS,
        {"calibration": "vendor library through torch, not this build's kernels"}))(
        vendor_gemm(dev, small, 4, "bf16", M=2048, N=11008, K=4096))
    if args.only:
        log(f"running {args.only}")
        row = runners[args.only]()
        log(json.dumps(row))
        print(json.dumps({"only": args.only, "result": row}))
        return 0

    log("int4 GEMV M=1 (headline)")
    head = runners["int4_gemv"]()
    log(json.dumps(head))
    if head.get("ms_per_step") is None:
        print(json.dumps({"metric": METRIC, "value": None, "unit": "TB/s", "n_gpus": 1, "steps": args.steps,
                          "warmup": args.warmup, "error": "headline output outside tolerance: not benchmarked",
                          "parity": head["parity"]}), flush=True)
        return 1
    extra = []
    if not args.no_extra:
        for k in ("int4_m2", "int4_m4", "int4_m16", "int8_gemv", "int8_m2", "int8_prefill", "int4_prefill", "fp32",
                  "int8_dgrad",
                  "fp8_gemm", "fp8_native",
                  "fp8_bwd", "fp8_bwd_native", "moe_int4", "moe_mlp_int4", "paged_attn", "quantize_int4",
                  "ref_shapes", "unquantized", "copy", "floor", "clocks", "vendor_fp8_rowwise", "vendor_fp8_tensorwise",
                  "vendor_bf16", "vendor_bf16_prefill"):
            log(f"{k} ...")
            row = runners[k]()
            log(json.dumps(row))
            if isinstance(row, list):
                extra += row
            elif row is not None:
                extra.append(row)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline (the reference's torch CPU path on host cores, ~30 s)")
        cpu = cpu_baseline()
        log(json.dumps(cpu))

    ms = head["ms_per_step"]
    roof = dict(head["roofline"])
    roof["traffic"] = load_traffic("int4_gemv_m1")
    roof["traffic_source"] = (f"{TRAFFIC_FILE}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE per dispatch of this "
                              "kernel, scaled by the same counters on a copy kernel of known size; a stored "
                              "measurement, not taken in this run")
    # the step split into the kernel's execution on the GPU and the launch around it, from
    # the clocked copy of the same kernel body in this run (extra row clocks_int4_gemv_m1_...)
    ck = next((r for r in extra if r.get("name") == "clocks_int4_gemv_m1_4096x4096" and "clocked" in r), None)
    if ck is not None:
        c = ck["clocked"]
        roof["step_split"] = {"kernel_exec_us": c["exec_us"], "launch_gap_us": c["gap_us"],
                              "clocked_period_us": c["period_us"], "exec_frac": ck["exec_frac"],
                              "library_step_us_events_2000": ck["library_step_us_events_2000_launches"],
                              "source": "clocked copy of the kernel body (libmls_floor.so), realtime clocks per "
                                        "wavefront: exec = first wavefront start to last wavefront end"}
    line = {
        "metric": METRIC,
        "value": head["TB/s"],
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "INT4 g128 weight-only decode GEMV (BASELINE.json configs[1])",
                   "M": 1, "N": 4096, "K": 4096, "group": 128, "activations": "bf16",
                   "scales": "fp16", "output": "bf16", "bytes_per_step": head["bytes_per_step"],
                   "weight_copies_rotated": head["weight_copies"], "launch": "HIP graph replay",
                   "timing": "realtime stamps in the graph around the K steps, less the median "
                             "stamp-to-stamp launch gap, after one untimed replay and warm_ms of "
                             "eager launches",
                   "warm_ms": WARM_MS,
                   "stamp_gap_us": round(statistics.median(STAMP_GAP_US), 3) if STAMP_GAP_US else None},
        "parity": head["parity"],
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
