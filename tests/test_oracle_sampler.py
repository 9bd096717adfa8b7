"""CPU pinning of the oracle's sampler and RNG (oracle/efo_sampler.c).

Pinned by: ISO C++'s mandated 10000th output of std::mt19937_64 (9981545732273789042); the
closed form of libstdc++'s generate_canonical<double,53> checked against the library itself (the
reference build calls std::uniform_real_distribution); the reference's KATs and seeded-frequency
test (tests/test_tokenizer.cpp:152-191); invariants (greedy = argmax after penalty, no draw when
T <= 0, top-k=1 / tiny top-p deterministic); the reference build's Sampler id for id; and golden id
sequences made by that build.
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

import oracle as O
from tests import _data as D

L = O.lib()
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not present")
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "fixtures.json")))


class Mt(C.Structure):
    _fields_ = [("mt", C.c_uint64 * 312), ("idx", C.c_int)]


def words(seed, n):
    g = Mt()
    L.efo_mt64_seed(C.byref(g), seed)
    return [L.efo_mt64_next(C.byref(g)) for _ in range(n)]


def test_mt19937_64_standard_value():
    assert words(5489, 10000)[-1] == 9981545732273789042  # [rand.predef]


def test_canonical_double_closed_form():
    g, h = Mt(), Mt()
    L.efo_mt64_seed(C.byref(g), 99)
    L.efo_mt64_seed(C.byref(h), 99)
    for _ in range(2000):
        u = L.efo_mt64_next(C.byref(h))
        r = float(np.float64(u) / 2.0 ** 64)
        r = np.nextafter(1.0, 0.0) if r >= 1.0 else r
        assert L.efo_canonical_double(C.byref(g)) == r


@needs_ref
def test_rng_matches_the_library():
    n = 5000
    ref_w = np.empty(n, np.uint64)
    O.ref().ref_mt64_words(42, n, O.ptr(ref_w, O._u64p))
    assert words(42, n) == ref_w.tolist()
    ref_u = np.empty(n, np.float64)
    O.ref().ref_uniform_doubles(42, n, O.ptr(ref_u, O._f64p))
    g = Mt()
    L.efo_mt64_seed(C.byref(g), 42)
    assert [L.efo_canonical_double(C.byref(g)) for _ in range(n)] == ref_u.tolist()


def test_sampler_reference_kats():  # tests/test_tokenizer.cpp:152-172
    l = np.array([1.0, 3.0, 2.0, -1.0], np.float32)
    assert O.Sampler().sample(l) == 1
    s1 = O.Sampler(temperature=5.0, top_k=1)
    assert all(s1.sample(l) == 1 for _ in range(50))
    sp = O.Sampler(temperature=1.0, top_p=1e-6)
    assert all(sp.sample(l) == 1 for _ in range(50))
    sr = O.Sampler(repetition_penalty=2.0)
    assert sr.sample(l, [1, 1]) == 2
    assert sr.sample(np.array([-1.0, -1.5], np.float32), [0]) == 1
    with pytest.raises(ValueError):
        O.Sampler().sample(np.zeros(0, np.float32))


def test_sampler_seeded_distribution():  # tests/test_tokenizer.cpp:174-191
    l = np.log(np.array([0.7, 0.2, 0.1], np.float32)).astype(np.float32)
    a, b = O.Sampler(temperature=1.0, seed=42), O.Sampler(temperature=1.0, seed=42)
    xs = [a.sample(l) for _ in range(20000)]
    assert xs == [b.sample(l) for _ in range(20000)]
    f = np.bincount(xs, minlength=3) / 20000
    assert np.all(np.abs(f - [0.7, 0.2, 0.1]) < 0.02)


def test_sampler_invariants():
    g = np.random.default_rng(1)
    for _ in range(20):
        lg = (g.standard_normal(1000) * 3).astype(np.float32)
        hist = g.integers(0, 1000, 30)
        s = O.Sampler(repetition_penalty=1.3)
        pen = lg.copy()
        for t in dict.fromkeys(hist.tolist()):
            pen[t] = pen[t] / np.float32(1.3) if pen[t] > 0 else pen[t] * np.float32(1.3)
        assert s.sample(lg, hist) == int(np.argmax(pen)) and s.last_r() == -1.0  # greedy: no draw
        t = O.Sampler(temperature=0.8, top_k=40, top_p=0.95, seed=3)
        tok = t.sample(lg)
        ids, probs = t.last_keep()
        order = sorted(range(1000), key=lambda i: (-float(lg[i] / np.float32(0.8)), i))
        assert ids.tolist() == order[:len(ids)] and tok in ids.tolist()
        assert abs(probs.sum() - 1.0) < 1e-12 and np.all(np.diff(probs) <= 0)


CONFIGS = [(0.8, 40, 0.95, 1.1), (1.0, 0, 1.0, 1.0), (0.7, 0, 0.9, 1.3), (1.5, 1000, 1.0, 1.0),
           (0.0, 0, 1.0, 1.2), (5.0, 1, 1.0, 1.0), (1.0, 0, 1e-6, 1.0), (2.0, 2000, 0.5, 1.0)]


def sampler_inputs(ci, step, V=32000):
    g = np.random.default_rng(1000 * ci + step)
    lg = (g.standard_normal(V) * (3.0 if step % 2 == 0 else 1.0)).astype(np.float32)
    if step == 3:
        lg[100:110] = lg[100]
    hist = g.integers(0, V, 64).astype(np.int32)
    hist[0], hist[1] = -1, hist[2]
    return lg, hist


@needs_ref
@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_sampler_ids_match_reference_build(ci):
    T, k, p, rep = CONFIGS[ci]
    a, b = O.Sampler(T, k, p, rep, seed=77), O.RefSampler(T, k, p, rep, seed=77)
    for step in range(10):
        lg, hist = sampler_inputs(ci, step)
        assert a.sample(lg, hist) == b.sample(lg, hist), step


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_sampler_ids_match_golden_reference_sequences(ci):
    T, k, p, rep = CONFIGS[ci]
    a = O.Sampler(T, k, p, rep, seed=77)
    got = [a.sample(*sampler_inputs(ci, step)) for step in range(10)]
    assert got == GOLDEN["sampler"][str(ci)]


def test_exp_array_is_the_host_libm():
    """The host side of the device exp sweep: the oracle's exp equals CPython's math.exp (the same
    libm) on sampled points, and the closed forms exp(0) = 1, exp(-inf-side underflow) = 0, exp of a
    tiny argument = 1 rounded, and the subnormal range are kept."""
    import math
    x = -D.rng(17).uniform(0.0, 746.0, 4096)
    x = np.concatenate([x, [0.0, -0.0, -1e-300, -745.2, -740.0, -709.0, -1.0]])
    y = O.exp_array(x)
    assert all(y[i] == math.exp(x[i]) for i in range(x.size))
    assert y[-7] == 1.0 and y[-6] == 1.0 and y[-5] == 1.0 and y[-4] == 0.0
    assert 0.0 < y[-3] < np.finfo(np.float64).tiny  # exp(-740) is subnormal
    assert abs(y[-1] - 0.36787944117144233) <= np.spacing(0.36787944117144233)
