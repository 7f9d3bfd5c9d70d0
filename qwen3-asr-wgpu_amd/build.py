"""Build libqasr_attn.so (gfx950) in-tree with hipcc.

Every .hip file under csrc/ is compiled for gfx950 only, then linked into one
shared library next to this file.  Flags:
  -Xclang -target-feature -Xclang -packed-fp32-ops  no v_pk_{add,mul,fma}_f32
  -fhip-fp32-correctly-rounded-divide-sqrt           IEEE '/' and sqrtf (stage (a)
                                                     is bit-exact against the
                                                     reference CPU path)
Per file: prefill_attn.hip adds -amdgpu-mfma-vgpr-form, which keeps the MFMA
accumulators in VGPRs; otherwise its one-wave-per-SIMD kernel puts O in AGPRs
and every rescale and loop-carried copy goes through v_accvgpr moves.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "libqasr_attn.so")
OBJ = os.path.join(HERE, "_build")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ROCM_LIB = "/opt/rocm/lib"
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


PER_FILE = {
    "prefill_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, extra=(), obj_dir: str = OBJ) -> str:
    obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *extra, *PER_FILE.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    # rocBLAS serves the text decoder's projection GEMMs (decoder.hip).
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           f"-L{ROCM_LIB}", "-lrocblas", f"-Wl,-rpath,{ROCM_LIB}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
