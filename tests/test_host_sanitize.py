"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

Runs on the CPU, no GPU.  The two translation units that hold the host
logic (fas_api.cpp: argument checks, workspace layout, key-split plan,
parameter packing; fas_fwd_dispatch.cpp: mode dispatch) are compiled again
with the host-side sanitizers (`-Xarch_host -fsanitize=...`; the device
pass of these files has no kernels) and linked with the kernel objects of
the regular build and tests/sanitize/host_driver.cpp into an executable.
The driver sweeps fas_workspace_bytes over every variant up to the largest
sizes the ABI accepts, sends every entry point each kind of invalid
request, and valid small problems over host buffers that fail only at the
launch.  The test passes when the driver's checks hold and neither
sanitizer reports anything.
"""
from __future__ import annotations

import os
import subprocess

import pytest

from flash_attn_with_score_amd.csrc import build as fas_build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tests", "sanitize", "host_driver.cpp")
HOST_SOURCES = ["fas_api.cpp", "fas_fwd_dispatch.cpp"]
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, f"{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}"


def test_host_code_under_asan_and_ubsan(tmp_path):
    hipcc = fas_build.hipcc()
    kernel_objs = [fas_build.OBJ_DIR / (src.name + ".o") for src in fas_build.sources()
                   if src.name not in HOST_SOURCES]
    if not all(o.exists() for o in kernel_objs):
        fas_build.build(verbose=False)
    flags = ["-x", "hip", f"--offload-arch={fas_build.ARCH}", "-O1", "-g", "-std=c++17",
             f"-I{os.path.join(ROOT, 'include')}", f"-I{fas_build.CSRC}", *SAN]
    objs = []
    for name in HOST_SOURCES + [DRIVER]:
        src = name if os.path.isabs(name) else str(fas_build.CSRC / name)
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        _run([hipcc, *flags, "-c", src, "-o", obj])
        objs.append(obj)
    exe = str(tmp_path / "host_driver")
    _run([hipcc, f"--offload-arch={fas_build.ARCH}", *SAN, *objs, *map(str, kernel_objs),
          "-o", exe])
    env = dict(os.environ)
    # The HIP runtime keeps its own allocations until exit: leak reports
    # would be about it, not about this code.
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["HIP_VISIBLE_DEVICES"] = ""
    proc = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    report = proc.stdout + proc.stderr
    assert "runtime error" not in report, report[-4000:]
    assert "AddressSanitizer" not in report, report[-4000:]
    assert proc.returncode == 0, report[-4000:]
    assert "0 failures" in proc.stdout, report[-4000:]
