"""The no-allocation sampler entry point (ef_hip_sample_noalloc: the library's fixed device scratch
instead of a workspace) against ef_hip_sample with a caller's workspace, through the C-ABI: ids
bit-identical on two calls in a row, the second smaller, and sizes above the scratch rejected."""
import ctypes as C

import numpy as np
import pytest

from edgeforge_amd import _lib as EL
from tests import _data as D

pytestmark = pytest.mark.gpu


def _cfg(d):
    return EL.ef_hip_sampler_config(d.get("temperature", 0.0), d.get("top_k", 0), d.get("top_p", 1.0),
                                    d.get("repetition_penalty", 1.0), 0)


def _both(hip, logits, V, B, cfg, hist, steps_seed):
    """ids of ef_hip_sample (own workspace) and ef_hip_sample_noalloc on the same inputs and seeds."""
    seeds = [steps_seed + 7 * b for b in range(B)]
    rng_a, rng_b = hip.RngStates(seeds), hip.RngStates(seeds)
    dl = hip.DeviceArray.from_host(logits)
    dh = hip.DeviceArray.from_host(hist)
    dn = hip.DeviceArray.from_host(np.full(B, hist.shape[1], np.int32))
    ws = hip.DeviceArray((EL.lib().ef_hip_sample_workspace_bytes(V, B),), np.uint8)
    oa, ob = hip.DeviceArray((B,), np.int32), hip.DeviceArray((B,), np.int32)
    c = _cfg(cfg)
    EL.call("ef_hip_sample", dl.ptr, V, B, V, C.byref(c), dh.ptr, dn.ptr, hist.shape[1], rng_a.buf.ptr, oa.ptr,
            ws.ptr, None)
    EL.call("ef_hip_sample_noalloc", dl.ptr, V, B, V, C.byref(c), dh.ptr, dn.ptr, hist.shape[1], rng_b.buf.ptr,
            ob.ptr, None)
    return oa.numpy(), ob.numpy()


def test_sample_noalloc_matches_sample_with_workspace(hip):
    print("[case] sample_noalloc: B=16 V=32000 full sort, then B=3 V=1000 top-k", flush=True)
    g = D.rng(4242)
    # call 1: the largest workspace use (no top-k: the split full sort over the keys)
    V, B = 32000, 16
    cfg = dict(temperature=0.7, top_k=0, top_p=0.9, repetition_penalty=1.3)
    logits = (g.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    hist = g.integers(0, V, size=(B, 64)).astype(np.int32)
    a, b = _both(hip, logits, V, B, cfg, hist, 11)
    assert np.array_equal(a, b), (a, b)
    # call 2: smaller (fewer sequences, smaller vocabulary, top-k): the scratch keeps call 1's bytes
    V, B = 1000, 3
    cfg = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    logits = (g.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)).astype(np.float32)
    hist = g.integers(0, V, size=(B, 16)).astype(np.int32)
    a, b = _both(hip, logits, V, B, cfg, hist, 23)
    assert np.array_equal(a, b), (a, b)


def test_sample_noalloc_rejects_sizes_above_the_scratch(hip):
    V, B = 32000, 64
    dl = hip.DeviceArray((B, V))
    out = hip.DeviceArray((B,), np.int32)
    c = _cfg(dict(temperature=0.0))
    with pytest.raises(EL.HipError, match="scratch"):
        EL.call("ef_hip_sample_noalloc", dl.ptr, V, B, V, C.byref(c), None, None, 0, None, out.ptr, None)
