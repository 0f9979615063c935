"""Checks on the gfx950 assembly of kernels whose correctness rests on instruction order
the compiler could change (CPU only: hipcc cross-compiles the device code here).

The exact fp8 GEMM (csrc/gemm_bytes.hip) reads its LDS operands with inline-asm ds_read_b128
and ties each use to a partial `s_waitcnt lgkmcnt(N)`: LDS reads complete in order, so N
outstanding reads means the earlier ones have landed. Scalar-memory loads share that counter
and complete out of order, so one issued inside the loop (a kernel argument reloaded under
register pressure, say) would make those waits release operands that have not arrived. The
test builds the file exactly as build.py does and fails if any loop that holds the
ds_read_b128 reads also holds a scalar-memory instruction."""

from __future__ import annotations

import importlib.util
import os
import re
import shutil
import subprocess

import pytest

from conftest import ROOT

CSRC = ROOT / "mini-llm-stack_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")

# scalar-memory reads (they return through lgkmcnt, out of order)
SMEM = re.compile(r"^\s+s_(load|buffer_load|scratch_load|memtime|memrealtime)\w*\b")


def _build_module():
    spec = importlib.util.spec_from_file_location("mls_build", CSRC / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _device_asm(src: str, out):
    b = _build_module()
    cmd = [b.hipcc(), *b.common_flags(), *b.EXTRA_FLAGS.get(src, []), "--cuda-device-only", "-S",
           str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, f"hipcc -S {src} failed:\n{r.stderr[-3000:]}"
    return out.read_text()


def _loops(body: list[str]):
    """(first, last) line of every loop: a branch back to a label above it."""
    labels = {}
    for i, line in enumerate(body):
        m = re.match(r"^(\.LBB\S+):", line)
        if m:
            labels[m.group(1)] = i
    out = []
    for i, line in enumerate(body):
        m = re.match(r"^\s+s_(?:cbranch_\w+|branch)\s+(\.LBB\S+)", line)
        if m and m.group(1) in labels and labels[m.group(1)] < i:
            out.append((labels[m.group(1)], i))
    return out


def test_exact_fp8_gemm_loops_issue_no_scalar_loads(tmp_path):
    asm = _device_asm("gemm_bytes.hip", tmp_path / "gemm_bytes.s")
    starts = [(m.group(1), m.end()) for m in re.finditer(r"^(_Z\S*gemm_bytes_kernel\S*):", asm, re.M)]
    assert starts, "no gemm_bytes_kernel in the assembly"
    checked = 0
    for name, st in starts:
        body = asm[st:asm.index(".Lfunc_end", st)].splitlines()
        for a, b in _loops(body):
            seg = body[a:b + 1]
            if not any("ds_read_b128" in x for x in seg):
                continue
            checked += 1
            bad = [x.strip() for x in seg if SMEM.match(x)]
            assert not bad, f"{name}: scalar-memory instructions inside the operand-read loop: {bad[:4]}"
    assert checked >= len(starts), f"found {checked} operand-read loops in {len(starts)} kernels"


def test_scan_flags_a_planted_scalar_load():
    """The scan itself: a loop with an s_load between its reads is caught."""
    body = [".LBB0_1:", "\tds_read_b128 v[0:3], v4", "\ts_load_dword s2, s[0:1], 0x0",
            "\ts_waitcnt lgkmcnt(1)", "\ts_cbranch_scc1 .LBB0_1"]
    loops = _loops(body)
    assert loops == [(0, 4)]
    assert [x for x in body[0:5] if SMEM.match(x)] == ["\ts_load_dword s2, s[0:1], 0x0"]
