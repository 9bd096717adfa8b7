"""Build libedgeforge_hip.so in-tree: every HIP source of edgeforge_amd/csrc, compiled for gfx950.

    python -m edgeforge_amd.build        (or edgeforge_amd.build.build())

hipcc compiles each translation unit to an object (in parallel) and links the shared library next
to this file, so it travels with the source tree.  Always recompiles (the build check must build).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libedgeforge_hip.so")
SHIM = os.path.join(HERE, "libedgeforge_kern.so")
OBJ = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed FP32 instructions are disabled for all device code (hipcc -O3 would otherwise form
# v_pk_{add,mul,fma}_f32 from ordinary float code).
DEVICE_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if warn.strip():
        sys.stderr.write(warn + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    # C++ host shim (ef::hip, EdgeForge's signatures) over the C-ABI only: plain g++, no HIP headers
    shim_src = os.path.join(HERE, "host", "ef_hip_kern.cpp")
    cmd = ["g++", "-O2", "-std=c++20", "-fPIC", "-shared", "-Wall", "-DEF_HIP_STANDALONE", "-o", SHIM + ".tmp",
           shim_src, f"-L{HERE}", "-ledgeforge_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host shim build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(SHIM + ".tmp", SHIM)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources and {SHIM}")
    return LIB


if __name__ == "__main__":
    build()
