"""The C++ shim (edgeforge_amd/host/ef_hip_kern.cpp) built inside the reference's tree, as
INTEGRATION's Level-1 drop-in does: compiled with the reference's include/ directory and without
EF_HIP_STANDALONE, so the reference's own ef::WeightView, ef::kern::MatvecJob and ef::SamplerConfig
(include/ef/qkernels.h:28-78, include/ef/sampler.h:13-35) are the types, then linked with a program
that forwards each ef::kern entry point to ef::hip and the reference's quant.cpp (qtype_row_bytes,
which the reference's inline WeightView::row_bytes calls).  CPU only: nothing runs on a GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
HOST = os.path.join(ROOT, "edgeforge_amd", "host")
LIBDIR = os.path.join(ROOT, "edgeforge_amd")

needs_reference = pytest.mark.skipif(not os.path.exists(os.path.join(REF, "include", "ef", "qkernels.h")),
                                     reason="the reference's headers are not present")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, f"{' '.join(cmd)}\n{r.stdout}\n{r.stderr}"
    return r


@needs_reference
def test_shim_compiles_and_links_against_the_reference_headers(tmp_path):
    if not os.path.exists(os.path.join(LIBDIR, "libedgeforge_hip.so")):
        pytest.skip("libedgeforge_hip.so not built")
    flags = ["g++", "-std=c++20", "-O1", "-Wall", "-Werror", f"-I{REF}/include", f"-I{HOST}"]
    shim_o = str(tmp_path / "ef_hip_kern.o")
    _run(flags + ["-c", os.path.join(HOST, "ef_hip_kern.cpp"), "-o", shim_o])
    # the header really took the reference's branch: no standalone WeightView::row_bytes emitted
    nm = _run(["nm", "-C", "--defined-only", shim_o]).stdout
    assert "ef::WeightView::row_bytes" not in nm
    drop_o = str(tmp_path / "dropin.o")
    _run(flags + ["-c", os.path.join(ROOT, "tests", "cpp", "dropin_reference_types.cpp"), "-o", drop_o])
    quant_o = str(tmp_path / "quant.o")
    _run(["g++", "-std=c++20", "-O1", f"-I{REF}/include", "-c", os.path.join(REF, "src", "quant.cpp"), "-o", quant_o])
    exe = str(tmp_path / "dropin")
    _run(["g++", "-o", exe, drop_o, shim_o, quant_o, f"-L{LIBDIR}", "-ledgeforge_hip", f"-Wl,-rpath,{LIBDIR}"])
    assert "linked: 18 bytes" in _run([exe]).stdout
