"""membench on the GPU (include/ef/membench.h, src/membench.cpp; tests/test_membench.cpp).

CPU: the closed-form pass checksum against a brute-force sum (tests/test_membench.cpp:9-16).
GPU: every run's sum equals the closed form times the pass count, and the reference's option
checks (tests/test_membench.cpp:40-62)."""
import ctypes as C

import numpy as np
import pytest

from edgeforge_amd import _lib as EL

MUL, ADD = np.uint64(0x9E3779B97F4A7C15), np.uint64(0x0123456789ABCDEF)


@pytest.mark.parametrize("n", [0, 1, 2, 3, 7, 8, 1000, 4097])
def test_closed_form_checksum(n):
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        brute = int(np.sum(i * MUL + ADD, dtype=np.uint64)) if n else 0
    assert EL.lib().ef_hip_membench_expected_pass_sum(n) == brute


@pytest.mark.gpu
def test_gpu_membench_checksums_and_options(hip):
    print("[case] membench 64 MiB x 2 passes", flush=True)
    o = EL.ef_hip_membench_options(64 << 20, 2, 2, 1)
    r = EL.ef_hip_membench_result()
    EL.call("ef_hip_membench", C.byref(o), C.byref(r))
    words = r.buffer_bytes // 8
    assert r.checksum_ok == 1 and r.passes == 2 and r.buffer_bytes <= 64 << 20
    with np.errstate(over="ignore"):
        assert r.expected_checksum == int(np.uint64(EL.lib().ef_hip_membench_expected_pass_sum(words)) * np.uint64(2))
    assert r.checksum == r.expected_checksum
    assert r.best_gbps >= r.median_gbps >= r.worst_gbps > 0
    for bad, msg in [((1 << 15, 1, 1, 0), "at least 64 KiB"), ((64 << 20, 0, 1, 0), "--runs"),
                     ((64 << 20, 1, 0, 0), "--passes"), ((64 << 20, 1, 1, -1), "--warmup"),
                     ((1 << 50, 1, 1, 0), "MiB")]:
        with pytest.raises(EL.HipError, match=msg):
            EL.call("ef_hip_membench", C.byref(EL.ef_hip_membench_options(*bad)), C.byref(r))
