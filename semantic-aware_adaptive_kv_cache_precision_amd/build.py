"""Builds libmicroinfer_hip.so for gfx950 with hipcc, in-tree.

    python build.py            # compile every source, link the library

Every source is compiled on each call (the driver's build check depends on
that); objects go to csrc/_build/, the library to microinfer/.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = CSRC / "_build"
LIBRARY = HERE / "microinfer" / "libmicroinfer_hip.so"
ARCH = os.environ.get("MI_OFFLOAD_ARCH", "gfx950")

SOURCES = ["quant.hip", "page_jobs.hip", "pages.hip", "pointwise.hip", "attention.hip",
           "decode.hip", "prefill.hip", "dense.hip", "step.hip", "linear.cpp",
           "page_allocator.cpp", "shadow_store.cpp", "scores_rope.cpp", "kv_cache.cpp",
           "decode_step.cpp", "capi.cpp"]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
# The dense projections call hipBLASLt.
LIBS = [f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lhipblaslt"]

# Bit-exact arithmetic needs IEEE fp32 with nothing fused behind our back:
# no contraction, no fast-math, denormals kept. Packed fp32 instructions are
# disabled for the device.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
         f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument", f"-I{HERE.parent / 'include'}", f"-I{CSRC}"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    return "hipcc"


def compile_one(source: str) -> Path:
    obj = OUT_DIR / (source.replace(".", "_") + ".o")
    cmd = [hipcc(), *FLAGS, "-x", "hip", "-c", str(CSRC / source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{' '.join(cmd)}\n{result.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objects = list(pool.map(compile_one, SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects), *LIBS]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
