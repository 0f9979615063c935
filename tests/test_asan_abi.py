"""The C ABI's host-side argument validation (csrc/wq_abi.hip, csrc/abi.hip) under
AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

tests/asan/abi_validation.cpp calls every entry point of those files with arguments
the validation must reject (nulls, negative and overflowing sizes, bad dtypes, short
strides, empty problems); the kernel launchers are replaced by stubs that abort, so a
call that slips past validation fails too. The sanitizers instrument host code only
(-Xarch_host; the device code of the .hip files is compiled as usual and never runs),
with no recovery: any report ends the program with a non-zero status. The executable
links the sanitizer runtimes statically, so nothing is preloaded."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import ROOT

CSRC = ROOT / "mini-llm-stack_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/llvm/bin/clang++"

pytestmark = pytest.mark.skipif(not (os.path.exists(HIPCC) and os.path.exists(CLANG)),
                                reason="needs hipcc and ROCm's clang++")

SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def _compile(src, out):
    cmd = [HIPCC, "-std=c++17", "-O1", "-g", "--offload-arch=gfx950",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           *SAN, f"-I{CSRC}", f"-I{ROOT / 'include'}", "-c", str(src), "-o", str(out)]
    if str(src).endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]  # the driver includes the HIP headers through wq.h
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, f"compile {src.name} failed:\n{r.stderr[-3000:]}"


def test_abi_validation_under_asan_ubsan(tmp_path):
    objs = []
    for src in (CSRC / "wq_abi.hip", CSRC / "abi.hip", ROOT / "tests" / "asan" / "abi_validation.cpp"):
        o = tmp_path / (src.stem + ".o")
        _compile(src, o)
        objs.append(str(o))
    exe = tmp_path / "abi_validation"
    link = [CLANG, "-fsanitize=address,undefined", "-fno-sanitize-recover=all", *objs,
            "-L/opt/rocm/lib", "-lamdhip64", f"-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)]
    r = subprocess.run(link, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, f"link failed:\n{r.stderr[-3000:]}"
    env = dict(os.environ)
    # leaks at exit belong to the HIP runtime's static state, not to the validation
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1:verify_asan_link_order=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "all cases passed" in out, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
