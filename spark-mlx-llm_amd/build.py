"""Build libsparkq.so (HIP kernels + C-ABI) for gfx950 with hipcc.

The library is written into the package directory (sparkq/libsparkq.so) so
that it ships with the source tree. Usage: python spark-mlx-llm_amd/build.py
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "sparkq", "libsparkq.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["w4a16.hip", "w4q.hip", "w4mr.hip", "w8a8.hip", "w8a16.hip", "w8aff.hip", "sdpa.hip", "sdpa_affine.hip", "sdpa_gen.hip",
           "layer.hip",
           "abi.cpp"]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops stay off: the compiler would otherwise form
    # v_pk_{add,mul,fma}_f32 from scalar float code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE division: the per-token quantizers must round x/scale correctly
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    f"-I{os.path.join(ROOT, 'include')}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build sparkq")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
