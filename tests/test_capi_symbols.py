"""CPU checks of the drop-in boundary: the C-ABI library loads and exports every entry point that
include/ef_hip.h declares (no GPU call is made)."""
import ctypes as C
import os

import pytest

from edgeforge_amd import _lib as L


def test_library_exports_every_declared_symbol():
    assert os.path.exists(L.LIB_PATH), "build first: python -m edgeforge_amd.build"
    lib = C.CDLL(L.LIB_PATH)
    declared = L.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert set(L.header_symbols()) == set(L.SIGNATURES), set(L.header_symbols()) ^ set(L.SIGNATURES)


def test_calls_before_init_fail_with_state_error():
    lib = L.lib()
    import ctypes
    p = ctypes.c_void_p()
    if getattr(L, "_inited", False):
        pytest.skip("library already initialised in this process")
    assert lib.ef_hip_malloc(ctypes.byref(p), 16) == L.ESTATE
    assert b"ef_hip_init" in lib.ef_hip_last_error()


def test_row_bytes_matches_reference_rule():
    lib = L.lib()
    out = C.c_size_t()
    assert lib.ef_hip_row_bytes(L.Q4_0, 2048, C.byref(out)) == 0 and out.value == 64 * 18
    assert lib.ef_hip_row_bytes(L.Q8_0, 2048, C.byref(out)) == 0 and out.value == 64 * 34
    assert lib.ef_hip_row_bytes(L.BF16, 2048, C.byref(out)) == 0 and out.value == 4096
    assert lib.ef_hip_row_bytes(L.Q4_0, 30, C.byref(out)) == L.EINVAL
    assert b"divisible by 32" in lib.ef_hip_last_error()


def test_cpp_shim_exports_the_reference_signatures():
    """libedgeforge_kern.so defines ef::hip::{matvec, matvec_jobs, row_f32, argmax, Sampler::sample}
    with the reference's parameter lists (checked on the mangled names)."""
    import subprocess
    shim = os.path.join(os.path.dirname(L.LIB_PATH), "libedgeforge_kern.so")
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", shim], capture_output=True, text=True).stdout
    for sig in ("ef::hip::matvec(float*, ef::WeightView const&, float const*, ef::ThreadPool*)",
                "ef::hip::matvec_jobs(ef::kern::MatvecJob const*, unsigned long, ef::ThreadPool*)",
                "ef::hip::row_f32(float*, ef::WeightView const&, unsigned long)",
                "ef::hip::argmax(float const*, unsigned long)",
                "ef::hip::Sampler::sample(float const*, unsigned long, std::vector<int, std::allocator<int> > const&)"):
        assert sig in out, sig
