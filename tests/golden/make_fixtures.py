"""Regenerate the committed golden fixtures (run in the build container, where /root/reference and
the reference build oracle/_ref/libefref.so exist):

    python tests/golden/make_fixtures.py

Writes
  tests/golden/fixtures.json       outputs of the REFERENCE BUILD (its quantize_row, matvec in both
                                   backends, Sampler, and Model::load_efq + Transformer greedy
                                   decode) on seeded inputs that the tests regenerate;
  tests/golden/p0_layer0_math.npz  a slice of the reference's own golden data
                                   (tests/golden/prompts/p0_factual: PyTorch FP32 layer-0 internals
                                   used by verify-math's weight-free checks, src/verify_math.cpp:131-185).
Both are data only: inputs are regenerated from seeds by the tests, expected values come from the
reference.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from edgeforge_amd.model import Config  # noqa: E402
from oracle.efq import write_efq  # noqa: E402
from oracle.model import HostModel  # noqa: E402
from tests import _data as D  # noqa: E402
from tests.test_oracle_codec import special_rows  # noqa: E402
from tests.test_oracle_sampler import CONFIGS, sampler_inputs  # noqa: E402

REF_GOLDEN = "/root/reference/tests/golden/prompts/p0_factual"


def ref_quantize(qtype, w, search=True):
    R = O.ref()
    out = np.empty((w.shape[0], O.row_bytes(qtype, w.shape[1])), np.uint8)
    for r in range(w.shape[0]):
        assert R.ref_quantize_row(qtype, O.ptr(np.ascontiguousarray(w[r]), O._f32p), w.shape[1], O.ptr(out[r]),
                                  int(search)) == 0
    return out


def main() -> None:
    R = O.ref()
    assert R is not None, "build the reference first: make -C oracle ref"
    fx = {"note": "expected values produced by the reference build (oracle/_ref) by tests/golden/make_fixtures.py"}

    fx["quant"] = {}
    for name, qtype, search in (("q4_search", O.Q4_0, True), ("q4_plain", O.Q4_0, False), ("q8", O.Q8_0, True)):
        sums = {}
        for seed in range(4):
            sums[str(seed)] = hashlib.sha256(ref_quantize(qtype, special_rows(seed), search).tobytes()).hexdigest()
        fx["quant"][name] = {"sha256": sums, "row0_seed0_hex": ref_quantize(qtype, special_rows(0), search)[0].tobytes().hex()}

    fx["gemv"] = {}
    for case, qt, n, seed in (("q4_2048", O.Q4_0, 2048, 101), ("q8_2048", O.Q8_0, 2048, 102), ("q4_5632", O.Q4_0, 5632, 103)):
        W = D.random_rows(qt, 16, n, seed=seed)
        x = D.activations_with_outliers(seed + 1, n)
        entry = {"rows": 16, "seed": seed}
        for backend, key in ((O.SCALAR, "scalar_bits"), (O.AVX2, "avx2_bits")):
            entry[key] = O.ref_matvec_jobs([(qt, W, x)], backend=backend)[0].view(np.uint32).tolist()
        fx["gemv"][case] = entry

    fx["sampler"] = {}
    for ci, (T, k, p, rep) in enumerate(CONFIGS):
        s = O.RefSampler(T, k, p, rep, seed=77)
        fx["sampler"][str(ci)] = [s.sample(*sampler_inputs(ci, step)) for step in range(10)]

    # tiny model quantized by the reference's quantizer, run by the reference's own engine
    tiny = Config(D=64, F=128, H=4, KV=2, hd=16, V=96, L=2, max_pos=32)
    seed, prompt, n = 31, [1, 5, 9, 33, 2, 17], 12
    hm = HostModel(tiny, seed=seed, q8={(1, "w_down"), (0, "wv")}, keep_floats=True)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.efq")
        t = hm.efq_tensors()
        for key, w in hm.weights.items():  # bytes re-made by the reference quantizer from the same floats
            if w.qtype in (O.Q4_0, O.Q8_0):
                floats = hm._floats[key]
                t[key] = (w.qtype, ref_quantize(w.qtype, floats))
        write_efq(path, tiny, t)
        e = R.ref_engine_open(path.encode(), len(prompt) + n, 1, O.AVX2)
        assert e
        logits = np.empty(tiny.V, np.float32)
        for pp in range(len(prompt)):
            assert R.ref_engine_forward(e, prompt[pp], pp, int(pp + 1 == len(prompt)), O.ptr(logits, O._f32p)) == 0
        first = logits.view(np.uint32)[:8].tolist()
        toks = []
        for kk in range(n):
            tok = int(R.ref_argmax(O.ptr(logits, O._f32p), tiny.V))
            toks.append(tok)
            if kk + 1 < n:
                assert R.ref_engine_forward(e, tok, len(prompt) + kk, 1, O.ptr(logits, O._f32p)) == 0
        R.ref_engine_close(e)
    fx["engine"] = {"seed": seed, "prompt": prompt, "n": n, "tokens": toks, "first_logits_bits": first}
    json.dump(fx, open(os.path.join(HERE, "fixtures.json"), "w"), indent=0)

    # slice of the reference's PyTorch golden data (weight-free layer-0 checks)
    def f32(name, shape):
        return np.fromfile(os.path.join(REF_GOLDEN, name), dtype=np.float32).reshape(shape)
    S = 23
    man = json.load(open(os.path.join(REF_GOLDEN, "manifest.json")))
    np.savez_compressed(
        os.path.join(HERE, "p0_layer0_math.npz"),
        rope_cos=f32("rope_cos.f32", (S, 64)), rope_sin=f32("rope_sin.f32", (S, 64)),
        q=f32("layer0/q.f32", (S, 2048)), k=f32("layer0/k.f32", (S, 256)), v=f32("layer0/v.f32", (S, 256)),
        q_rope=f32("layer0/q_rope.f32", (S, 2048)), k_rope=f32("layer0/k_rope.f32", (S, 256)),
        attn_context=f32("layer0/attn_context.f32", (S, 2048)),
        gate=f32("layer0/gate.f32", (S, 5632))[:3], up=f32("layer0/up.f32", (S, 5632))[:3],
        mlp_act=f32("layer0/mlp_act.f32", (S, 5632))[:3],
        embed=f32("embed_all.f32", (S, 2048))[:3], attn_out=f32("layer0/attn_out.f32", (S, 2048))[:3],
        resid=f32("layer0/resid_after_attn.f32", (S, 2048))[:3],
        logits_last=f32("logits_last.f32", (32000,)), greedy_first=np.array([man["greedy"]["ids"][0]], np.int32))
    print("wrote fixtures.json and p0_layer0_math.npz")


if __name__ == "__main__":
    main()
