"""The oracle's glue kernels against the reference's own golden vectors: PyTorch FP32 layer-0
internals of TinyLlama-1.1B on prompt p0_factual (a slice of /root/reference/tests/golden committed
as tests/golden/p0_layer0_math.npz), with verify-math's weight-free checks and tolerances
(src/verify_math.cpp:60-62, 131-185): 1e-5 relative (max|err| / max|ref|) elementwise, 1e-4 and
cosine 0.99999 for the attention reduction, and argmax(logits_last) == the greedy token."""
import os

import numpy as np

import oracle as O

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "p0_layer0_math.npz"))
L = O.lib()
F = O._f32p
S, D, H, KV, HD = 23, 2048, 32, 4, 64


def rel(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def cosine(a, b):
    a, b = a.astype(np.float64).ravel(), b.astype(np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


def tables():
    inv = np.empty(HD // 2, np.float32)
    c = np.empty((S, HD // 2), np.float32)
    s = np.empty_like(c)
    L.efo_rope_table(O.ptr(inv, F), O.ptr(c, F), O.ptr(s, F), S, HD, 10000.0)
    return c, s


def roped():
    c, s = tables()
    q, k = G["q"].copy(), G["k"].copy()
    for p in range(S):
        L.efo_rope_apply(O.ptr(q[p], F), H, HD, O.ptr(c[p], F), O.ptr(s[p], F))
        L.efo_rope_apply(O.ptr(k[p], F), KV, HD, O.ptr(c[p], F), O.ptr(s[p], F))
    return q, k


def test_rope_tables_and_rotation_match_pytorch():
    c, s = tables()
    assert rel(np.concatenate([c, c], 1), G["rope_cos"]) <= 1e-5
    assert rel(np.concatenate([s, s], 1), G["rope_sin"]) <= 1e-5
    q, k = roped()
    assert rel(q, G["q_rope"]) <= 1e-5 and rel(k, G["k_rope"]) <= 1e-5


def test_causal_gqa_attention_matches_pytorch_context():
    q, k = roped()
    v = G["v"]
    out = np.empty((S, D), np.float32)
    scores = np.empty(S, np.float32)
    for p in range(S):
        L.efo_attention_heads(O.ptr(out[p], F), O.ptr(q[p], F), O.ptr(k, F), O.ptr(np.ascontiguousarray(v), F),
                              p + 1, H, KV, HD, O.ptr(scores, F), 0, H)
        assert rel(out[p], G["attn_context"][p]) <= 1e-4 and cosine(out[p], G["attn_context"][p]) >= 0.99999


def test_swiglu_and_residual_match_pytorch():
    gate, up = np.ascontiguousarray(G["gate"]), np.ascontiguousarray(G["up"])
    act = np.empty_like(gate)
    L.efo_swiglu(O.ptr(act, F), O.ptr(gate, F), O.ptr(up, F), gate.size)
    assert rel(act, G["mlp_act"]) <= 1e-5
    x = np.ascontiguousarray(G["embed"]).copy()
    L.efo_add_inplace(O.ptr(x, F), O.ptr(np.ascontiguousarray(G["attn_out"]), F), x.size)
    assert rel(x, G["resid"]) <= 1e-5


def test_argmax_of_golden_logits_is_the_greedy_token():
    lg = np.ascontiguousarray(G["logits_last"])
    assert L.efo_argmax(O.ptr(lg, F), lg.size) == int(G["greedy_first"][0])
