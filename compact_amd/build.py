"""Build libcompact_amd.so from compact_amd/csrc/*.hip for gfx950.

`python -m compact_amd.build` (or `__graft_entry__.build()`) compiles every
HIP source with hipcc and links them into compact_amd/_build/libcompact_amd.so.
Cross-compiles without a GPU.  Flags that decide numerics:
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE division (codec bit-exactness)
  -fno-gpu-flush-denormals-to-zero           keep fp32 denormals
  -ffp-contract=off                          (codec, gemm*, adapters) no FMA contraction
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-fp32 instructions
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libcompact_amd.so")
ARCH = os.environ.get("CPT_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
]
# no FMA contraction in the codec, GEMM (every gemm*.hip unit) and adapter kernels
NO_CONTRACT = ("codec", "gemm", "adapters")


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found")
    return p


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), "-c", src, "-o", obj] + COMMON
    if os.path.basename(src).startswith(NO_CONTRACT):
        cmd.append("-ffp-contract=off")
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
