"""Host sanitizer run of the library's launch planners.

Builds every csrc/*.hip source with AddressSanitizer and
UndefinedBehaviorSanitizer on the host compilation (-Xarch_host; the device
code as for the library), links them with sanitize_planners.cpp into
_build/sanitize/sanitize_planners, and runs it: qasr_plan_decode and
qasr_plan_prefill over random batches, argument edges, the environment knobs
and the refusals, with the plans' invariants checked.  Host code only; no
device is needed.  Usage: python tests/sanitize_planners.py
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

TESTS = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(TESTS), "qwen3-asr-wgpu_amd"))
from build import INCLUDE, OBJ, ROCM_LIB, _compile, sources  # noqa: E402

SANITIZE_HOST = ["-g", "-fno-omit-frame-pointer",
                 "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=undefined"]
SAN_OBJ = os.path.join(OBJ, "sanitize")
SAN_EXE = os.path.join(SAN_OBJ, "sanitize_planners")


def build_sanitized() -> str:
    """The planner sanitizer driver (sanitize_planners.cpp): every source with
    host AddressSanitizer + UndefinedBehaviorSanitizer, linked into one
    executable.  The driver calls host code only; no device is needed."""
    os.makedirs(SAN_OBJ, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, SANITIZE_HOST, SAN_OBJ), srcs))
    drv = os.path.join(SAN_OBJ, "sanitize_planners.o")
    gxx = shutil.which("g++") or "g++"
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    steps = [
        [gxx, "-std=c++17", "-O1", "-g", *san, f"-I{INCLUDE}", "-c",
         os.path.join(TESTS, "sanitize_planners.cpp"), "-o", drv],
        [gxx, *san, "-o", SAN_EXE, drv, *objs, f"-L{ROCM_LIB}", "-lamdhip64", "-lrocblas",
         f"-Wl,-rpath,{ROCM_LIB}"],
    ]
    for cmd in steps:
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"sanitizer build failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return SAN_EXE


if __name__ == "__main__":
    exe = build_sanitized()
    sys.exit(subprocess.run([exe]).returncode)
