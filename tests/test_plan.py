"""The scan planning arithmetic (vectoraccelerate_amd/csrc/va_plan.hpp), checked on the CPU.

tests/cpp/plan_host.cpp includes the header the kernels' host code uses to size every search
(sample sizes, candidate and rerank capacities, the device fallback's buffers, the scratch the
drivers carve, the IVF tile shapes) and checks it at extreme shapes against 128-bit recomputations
and brute force.  Under oracle/run_sanitized.sh (VA_SANITIZE=1) the program is built with
AddressSanitizer + UndefinedBehaviorSanitizer, so an overflowing shift or signed product aborts it.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "cpp" / "plan_host.cpp"


def test_plan_arithmetic(tmp_path):
    exe = tmp_path / "plan_host"
    flags = ["-O1"]
    if os.environ.get("VA_SANITIZE"):
        flags += ["-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    proc = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", *flags, str(SRC), "-o", str(exe)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    env = dict(os.environ)
    env.pop("LD_PRELOAD", None)  # the program links its own sanitizer runtimes
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    print(run.stdout)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "ok" in run.stdout
