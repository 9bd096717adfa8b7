"""CPU pinning of the oracle's packed GEMV (oracle/efo_gemv.c): scalar and AVX2 orders, row
dispatch, multi-job GEMV and the thread pool.

Pinned by: the reference's KATs (tests/test_qinfer.cpp:100-122), the float64 dequantize-then-dot
bound |got - exact| <= 1e-5 sum|w x| (tests/test_qinfer.cpp:57-98), structural identities (matvec
== per-row dot bit for bit, any thread count gives the same bits), the reference build bit for
bit, and golden outputs of that build committed under tests/golden.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from tests import _data as D

L = O.lib()
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not present")
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "fixtures.json")))


def dot(qtype, row, x, avx2):
    f = {(O.Q4_0, 0): L.efo_dot_q4_0, (O.Q4_0, 1): L.efo_dot_q4_0_avx2,
         (O.Q8_0, 0): L.efo_dot_q8_0, (O.Q8_0, 1): L.efo_dot_q8_0_avx2}[(qtype, int(avx2))]
    return f(O.ptr(np.ascontiguousarray(row), O._u8p), O.ptr(x, O._f32p), x.size)


def test_dot_layout_and_edge_codes():  # tests/test_qinfer.cpp:100-122
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:] = 0x88
    blk[5] = 0x0F
    x = np.zeros(32, np.float32)
    x[3], x[19] = 2.0, 0.5
    for avx2 in (0, 1):
        assert dot(O.Q4_0, blk, x, avx2) == 7.0 * 2.0 + -8.0 * 0.5
    blk[0:2] = 0
    assert dot(O.Q4_0, blk, x, 0) == 0.0 and dot(O.Q4_0, blk, x, 1) == 0.0
    b8 = np.zeros(34, np.uint8)
    b8[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b8[2], b8[33] = 256 - 127, 127
    ones = np.ones(32, np.float32)
    assert dot(O.Q8_0, b8, ones, 0) == 0.0 and dot(O.Q8_0, b8, ones, 1) == 0.0
    b8[7] = 3
    assert dot(O.Q8_0, b8, ones, 0) == 3.0 and dot(O.Q8_0, b8, ones, 1) == 3.0


@pytest.mark.parametrize("n", [32, 64, 96, 2048, 5632])
@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0])
def test_packed_dots_within_exact_bound_and_matvec_is_row_dots(qtype, n):
    W = D.random_rows(qtype, 24, n, seed=n + qtype)
    x = D.activations_with_outliers(n, n)
    w64 = D.dequant_exact(qtype, W, n)
    for backend in (O.SCALAR, O.AVX2):
        y = O.matvec(qtype, W.reshape(-1), x, backend=backend)
        assert D.rel_dot_error(w64, x, y).max() < 1e-5
        rows = np.array([dot(qtype, W[r], x, backend) for r in range(24)], np.float32)
        assert np.array_equal(rows.view(np.uint32), y.view(np.uint32))


def test_threadpool_covers_every_index_once():  # tests/test_qinfer.cpp:201-225
    import ctypes as C
    hits = {}

    @C.CFUNCTYPE(None, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t)
    def body(ctx, chunk, b, e):
        for i in range(b, e):
            hits[i] = hits.get(i, 0) + 1

    L.efo_pool_parallel_for.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_size_t]
    for T in (1, 2, 3, 8):
        pool = O.Pool(T)
        for n in (0, 1, 5, 100, 1001):
            for mc in (1, 16):
                hits.clear()
                L.efo_pool_parallel_for(pool.h, n, C.cast(body, C.c_void_p), None, mc)
                assert sorted(hits) == list(range(n)) and set(hits.values()) <= {1}
        pool.close()
    assert [L.efo_pool_chunk_begin(1001, 3, c) for c in range(4)] == [0, 333, 667, 1001]


def test_parallel_gemv_bit_identical_for_any_thread_count():  # tests/test_qinfer.cpp:227-263
    cols = 256
    x = D.normal(64, cols, 0.3)
    jobs = []
    for qt, rows in ((O.Q4_0, 300), (O.Q8_0, 37)):
        jobs.append((qt, O.quantize(qt, D.normal(rows, (rows, cols), 0.3)), x))
    for backend in (O.SCALAR, O.AVX2):
        ref = O.matvec_jobs(jobs, backend=backend)
        for T in (2, 3, 5, 8):
            pool = O.Pool(T)
            got = O.matvec_jobs(jobs, backend=backend, pool=pool)
            pool.close()
            assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(ref, got))


def test_avx2_and_scalar_agree_to_rounding():
    W = O.quantize(O.Q4_0, D.normal(1, (64, 2048), 0.02))
    x = D.normal(2, 2048)
    a = O.matvec(O.Q4_0, W.reshape(-1), x, backend=O.AVX2)
    s = O.matvec(O.Q4_0, W.reshape(-1), x, backend=O.SCALAR)
    assert np.abs(a - s).max() <= 1e-5 * np.abs(s).max()


@needs_ref
@pytest.mark.parametrize("threads", [1, 3])
def test_gemv_bit_identical_to_reference_build(threads):
    for qt in (O.Q4_0, O.Q8_0):
        for n in (32, 96, 2048, 5632):
            W = D.random_rows(qt, 40, n, seed=7 * n + qt)
            x = D.activations_with_outliers(n + 1, n)
            for backend in (O.SCALAR, O.AVX2):
                mine = O.matvec(qt, W.reshape(-1), x, backend=backend)
                ref = O.ref_matvec_jobs([(qt, W, x)], backend=backend, threads=threads)[0]
                assert np.array_equal(mine.view(np.uint32), ref.view(np.uint32)), (qt, n, backend)
            for r in (0, 39):
                f = O.ref().ref_dot_q4_0 if qt == O.Q4_0 else O.ref().ref_dot_q8_0
                assert np.float32(f(O.ptr(W[r], O._u8p), O.ptr(x, O._f32p), n)) == np.float32(dot(qt, W[r], x, 0))


@pytest.mark.parametrize("case", ["q4_2048", "q8_2048", "q4_5632"])
def test_gemv_matches_golden_reference_outputs(case):
    fx = GOLDEN["gemv"][case]
    qt, n = {"q4_2048": (O.Q4_0, 2048), "q8_2048": (O.Q8_0, 2048), "q4_5632": (O.Q4_0, 5632)}[case]
    W = D.random_rows(qt, fx["rows"], n, seed=fx["seed"])
    x = D.activations_with_outliers(fx["seed"] + 1, n)
    for backend, key in ((O.SCALAR, "scalar_bits"), (O.AVX2, "avx2_bits")):
        got = O.matvec(qt, W.reshape(-1), x, backend=backend).view(np.uint32).tolist()
        assert got == fx[key], (case, key)
