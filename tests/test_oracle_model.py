"""CPU pinning of the oracle's FP32 glue kernels and decode step (oracle/efo_model.c).

Pinned by: the reference's KATs and float64 references (tests/test_kernels.cpp:55-253), the
reference build's kernels bit for bit, the reference's own engine (Model::load_efq + Transformer,
src/model.cpp) run on an .efq file holding the same packed bytes (logits bit for bit at every
position, identical greedy tokens), the engine-level identity "quantized engine == its
dequantized F32 copy to 1e-4" (tests/test_qinfer.cpp:313-344), and golden tokens of that engine.
"""
import ctypes as C
import json
import os
import tempfile

import numpy as np
import pytest

import oracle as O
from edgeforge_amd.model import Config
from oracle.efq import write_efq
from oracle.model import HostModel, OracleModel

L = O.lib()
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not present")
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "fixtures.json")))
F = O._f32p


def close(a, b, rel, abs_tol=0.0):
    return abs(float(a) - float(b)) <= abs_tol + rel * max(abs(float(a)), abs(float(b)))


def rms(x, w, eps):
    out = np.empty_like(x)
    L.efo_rmsnorm(O.ptr(out, F), O.ptr(x, F), O.ptr(w, F), x.size, eps)
    return out


def test_rmsnorm_known_values():  # tests/test_kernels.cpp:104-134
    x = np.array([1, 2, 3, 4], np.float32)
    ones = np.ones(4, np.float32)
    r = np.sqrt(7.5)
    assert all(close(v, (i + 1) / r, 1e-6) for i, v in enumerate(rms(x, ones, 0.0)))
    o = rms(x, np.array([2, 0.5, -1, 0], np.float32), 0.0)
    assert close(o[0], 2 / r, 1e-6) and close(o[2], -3 / r, 1e-6) and o[3] == 0.0
    assert rms(np.zeros(4, np.float32), ones, 1e-5)[0] == 0.0
    assert close(rms(np.full(2, 1e-3, np.float32), np.ones(2, np.float32), 1e-6)[0], 1e-3 / np.sqrt(2e-6), 1e-6)


def test_softmax_stable_masked_and_silu():  # tests/test_kernels.cpp:136-181
    def sm(v):
        v = np.array(v, np.float32)
        L.efo_softmax_inplace(O.ptr(v, F), v.size)
        return v
    assert close(sm([1, 2, 3])[2], 0.66524095577, 1e-6) and close(sm([1000, 1001, 1002])[2], 0.66524095577, 1e-6)
    assert close(sm([-1000, -1001, -1002])[0], 0.66524095577, 1e-6)
    m = sm([-np.inf, 0.5, -np.inf])
    assert m[0] == 0.0 and m[1] == 1.0 and m[2] == 0.0
    assert np.all(sm([-np.inf, -np.inf]) == 0.0) and sm([42.0])[0] == 1.0
    assert L.efo_silu(0.0) == 0.0 and close(L.efo_silu(1.0), 0.7310585786, 1e-6) and L.efo_silu(100.0) == 100.0
    neg = L.efo_silu(-100.0)
    assert not np.isnan(neg) and abs(neg) < 1e-30


def rope_tables(max_pos, hd, theta):
    inv = np.empty(hd // 2, np.float32)
    c = np.empty((max_pos, hd // 2), np.float32)
    s = np.empty_like(c)
    L.efo_rope_table(O.ptr(inv, F), O.ptr(c, F), O.ptr(s, F), max_pos, hd, theta)
    return inv, c, s


def test_rope_half_split_formula_and_relative_positions():  # tests/test_kernels.cpp:183-224
    hd, H = 64, 3
    inv, c, s = rope_tables(64, hd, 10000.0)
    assert inv[0] == 1.0 and all(close(inv[i], 10000.0 ** (-2.0 * i / hd), 2e-6) for i in range(hd // 2))
    x0 = np.random.default_rng(5).standard_normal(H * hd).astype(np.float32)
    x = x0.copy()
    L.efo_rope_apply(O.ptr(x, F), H, hd, O.ptr(c[0], F), O.ptr(s[0], F))
    assert np.array_equal(x, x0)
    x = x0.copy()
    L.efo_rope_apply(O.ptr(x, F), H, hd, O.ptr(c[7], F), O.ptr(s[7], F))
    for h in range(H):
        for i in range(hd // 2):
            ang = 7 * 10000.0 ** (-2.0 * i / hd)
            a, b = float(x0[h * hd + i]), float(x0[h * hd + i + hd // 2])
            assert close(x[h * hd + i], a * np.cos(ang) - b * np.sin(ang), 1e-5, 1e-6)
            assert close(x[h * hd + i + hd // 2], b * np.cos(ang) + a * np.sin(ang), 1e-5, 1e-6)


def attention(q, k, v, n_pos, H, KV, hd):
    out = np.empty(H * hd, np.float32)
    scores = np.empty(n_pos, np.float32)
    L.efo_attention_heads(O.ptr(out, F), O.ptr(q, F), O.ptr(k, F), O.ptr(v, F), n_pos, H, KV, hd,
                          O.ptr(scores, F), 0, H)
    return out


def test_attention_causal_gqa_against_float64():  # tests/test_kernels.cpp:226-244
    H, KV, hd, T = 4, 2, 8, 5
    g = np.random.default_rng(7)
    q, k, v = (g.standard_normal(n).astype(np.float32) for n in (H * hd, T * KV * hd, T * KV * hd))
    for n in range(1, T + 1):
        out = attention(q, k, v, n, H, KV, hd)
        for h in range(H):
            kv = h // (H // KV)
            sc = np.array([np.dot(q[h * hd:(h + 1) * hd].astype(np.float64),
                                  k[t * KV * hd + kv * hd:t * KV * hd + (kv + 1) * hd]) / np.sqrt(hd) for t in range(n)])
            p = np.exp(sc - sc.max())
            p /= p.sum()
            ref = sum(p[t] * v[t * KV * hd + kv * hd:t * KV * hd + (kv + 1) * hd].astype(np.float64) for t in range(n))
            assert np.allclose(out[h * hd:(h + 1) * hd], ref, rtol=1e-5, atol=1e-6)
    first = attention(q, k, v, 1, H, KV, hd)
    for h in range(H):
        assert np.array_equal(first[h * hd:(h + 1) * hd], v[(h // 2) * hd:(h // 2 + 1) * hd])


@needs_ref
def test_glue_kernels_bit_identical_to_reference_build():
    g = np.random.default_rng(9)
    x = g.standard_normal(2048).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(2048)).astype(np.float32)
    a, b = np.empty_like(x), np.empty_like(x)
    L.efo_rmsnorm(O.ptr(a, F), O.ptr(x, F), O.ptr(w, F), 2048, 1e-5)
    O.ref().ref_rmsnorm(O.ptr(b, F), O.ptr(x, F), O.ptr(w, F), 2048, 1e-5)
    assert np.array_equal(a, b)
    for v in g.standard_normal(200).astype(np.float32) * 20:
        assert np.float32(L.efo_silu(float(v))) == np.float32(O.ref().ref_silu(float(v)))
    inv, c, s = rope_tables(64, 64, 10000.0)
    inv2, c2, s2 = np.empty_like(inv), np.empty_like(c), np.empty_like(s)
    O.ref().ref_rope_table(O.ptr(inv2, F), O.ptr(c2, F), O.ptr(s2, F), 64, 64, 10000.0)
    assert np.array_equal(inv, inv2) and np.array_equal(c, c2) and np.array_equal(s, s2)
    H, KV, hd, T = 32, 4, 64, 40
    q, k, v = (g.standard_normal(n).astype(np.float32) for n in (H * hd, T * KV * hd, T * KV * hd))
    out_ref, sc = np.empty(H * hd, np.float32), np.empty(T, np.float32)
    O.ref().ref_attention(O.ptr(out_ref, F), O.ptr(q, F), O.ptr(k, F), O.ptr(v, F), T, H, KV, hd, O.ptr(sc, F))
    assert np.array_equal(attention(q, k, v, T, H, KV, hd), out_ref)


TINY = Config(D=64, F=128, H=4, KV=2, hd=16, V=96, L=2, max_pos=32)


@needs_ref
@pytest.mark.parametrize("backend", [O.SCALAR, O.AVX2])
def test_transformer_logits_bit_identical_to_reference_engine(backend):
    hm = HostModel(TINY, seed=21, q8={(1, "w_down"), (0, "wv")})
    om = OracleModel(hm)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.efq")
        write_efq(path, TINY, hm.efq_tensors())
        e = O.ref().ref_engine_open(path.encode(), 16, 3, backend)
        assert e, "reference engine rejected the .efq file"
        bpt = O.ref().ref_engine_bytes_per_token(e)
        ot = om.transformer(16, threads=2, backend=backend)
        ids = [1, 5, 9, 33, 2, 17, 17, 4, 30, 12]
        for p, t in enumerate(ids):
            want = np.empty(TINY.V, np.float32)
            assert O.ref().ref_engine_forward(e, t, p, 1, O.ptr(want, F)) == 0
            got = ot.forward(t, p)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), p
        assert O.ref().ref_engine_forward(e, TINY.V, 0, 1, None) == -1  # token out of range throws
        assert O.ref().ref_engine_forward(e, 1, 12, 1, None) == -1  # skipping ahead throws
        O.ref().ref_engine_close(e)
        ot.close()
    assert bpt == sum(hm.host_bytes(k).nbytes for k in hm.weights if k != "embed") + (2 * TINY.L + 1) * TINY.D * 4


def test_quantized_engine_matches_its_dequantized_copy():
    """tests/test_qinfer.cpp:313-344: packed kernels only change the summation order."""
    hm = HostModel(TINY, seed=22, q8={(1, "w_down")})
    deq = HostModel(TINY, seed=22, q8={(1, "w_down")})
    for k, w in hm.weights.items():  # F32 copy of every packed matrix
        if w.qtype in (O.Q4_0, O.Q8_0):
            deq._bytes[k] = O.dequantize(w.qtype, hm.host_bytes(k), w.cols).view(np.uint8).reshape(w.rows, -1)
            deq.weights[k] = type(w)(O.F32, w.rows, w.cols)
    a, b = OracleModel(hm).transformer(12, threads=1), OracleModel(deq).transformer(12, threads=1)
    ids = [1, 5, 9, 33, 2, 17, 17, 4, 30, 12]
    for p, t in enumerate(ids):
        la, lb = a.forward(t, p), b.forward(t, p)
        assert np.abs(la - lb).max() / np.abs(lb).max() < 1e-4
        assert int(np.argmax(la)) == int(np.argmax(lb))


def test_greedy_tokens_match_golden_reference_engine():
    fx = GOLDEN["engine"]
    hm = HostModel(TINY, seed=fx["seed"], q8={(1, "w_down"), (0, "wv")})
    toks, logits, _, _ = OracleModel(hm).run_once(fx["prompt"], fx["n"], threads=2)
    assert toks.tolist() == fx["tokens"]
    assert logits[0].view(np.uint32).tolist()[:8] == fx["first_logits_bits"]
