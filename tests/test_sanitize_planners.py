"""The launch planners under the host sanitizers: sanitize_planners.py builds
every source's host code with AddressSanitizer + UndefinedBehaviorSanitizer
and runs the driver (qasr_plan_decode / qasr_plan_prefill over random
batches, argument edges, environment knobs and refusals, invariants
checked).  Host code only; about a minute and a half, most of it hipcc."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "tests", "sanitize_planners.py")


@pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")),
                    reason="hipcc not installed")
@pytest.mark.skipif(not os.path.exists(SCRIPT), reason="sanitizer driver not in this tree")
def test_planners_clean_under_asan_ubsan():
    env = dict(os.environ)
    for v in ("QASR_DECODE_WGS", "QASR_DECODE_GRANULE", "QASR_DECODE_MAX_GRANULES", "QASR_PREFILL_TPS"):
        env.pop(v, None)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0"
    r = subprocess.run([sys.executable, SCRIPT], capture_output=True, text=True, env=env, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "0 failures" in r.stdout, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
