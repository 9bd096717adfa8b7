"""GPU parity of the engine run from an .efq file (Model::load_efq, src/model.cpp:66-111, then
Transformer::forward) against the CPU oracle's engine on the same packed bytes.

Files are written by oracle/efq.py from oracle-quantized weights (the reference quantizer's bytes,
pinned in the CPU suite); the reference build itself accepts them (tests/test_efq_reader.py).  Cases:
the default policy (Q4_0 layers with Q8_0 overrides, Q8_0 lm_head, BF16 embedding), a lossless
BF16 file (every product on the unquantized-weight GEMV), tied embeddings (the BF16 embedding is
the lm_head), and several sequences at once.  Gates: logits within 1e-4 relative at every position,
identical greedy tokens, the uploaded bytes equal to the file's, and the model's description and
bytes per token as the reference computes them.
"""
import ctypes as C
import os
import tempfile

import numpy as np
import pytest

import oracle as O
from edgeforge_amd import _lib as EL
from edgeforge_amd.model import Config
from edgeforge_amd.qfile import EfqModel, QuantFile
from oracle.efq import write_efq
from oracle.model import HostModel, OracleModel
from tests import _data as D

pytestmark = pytest.mark.gpu

SMALL = Config(D=256, F=512, H=4, KV=2, hd=64, V=500, L=2, max_pos=64)


def _logit_err(a, b):
    return float(np.abs(a - b).max() / max(1.0, np.abs(b).max()))


def _check_engine(path, hm, prompt_len=7, n=12, batch=1):
    m = EfqModel.load_efq(path)
    om = OracleModel(hm)
    prompts = [[int(v) for v in D.rng(100 + b).integers(0, hm.cfg.V, prompt_len)] for b in range(batch)]
    eng = m.engine(max_seq=prompt_len + n, batch=batch)
    got, _, _ = eng.generate(prompts, n)
    for b in range(batch):
        want, want_logits, _, _ = om.run_once(prompts[b], n, threads=2)
        assert got[b].tolist() == want.tolist(), b
    # logits position by position for the first sequence
    ot = om.transformer(prompt_len + n, threads=2)
    seq = prompts[0] + got[0].tolist()[:-1]
    for p, t in enumerate(seq[:prompt_len + 3]):
        eng.forward([t] * batch, p)
        want = ot.forward(t, p)
        assert _logit_err(eng.logits()[0], want) < 1e-4, p
    ot.close()
    with pytest.raises(EL.HipError, match="destroy the engines"):
        m.free()  # an engine still uses the weights
    eng.close()
    return m


def test_default_policy_file(hip):
    print("[case] efq Q4_0 + Q8_0 overrides, Q8_0 lm_head, BF16 embed", flush=True)
    hm = HostModel(SMALL, seed=51, q8={(0, "wk"), (0, "wv"), (1, "w_down")})
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.efq")
        write_efq(path, SMALL, hm.efq_tensors())
        m = _check_engine(path, hm)
        f = QuantFile.open(path)
        assert m.bytes_per_token == f.bytes_per_token()
        assert m.description == "efq, policy custom: 11 Q4_0 + 4 Q8_0 matrices, embedding BF16"
        assert m.cfg.D == SMALL.D and m.cfg.V == SMALL.V and not m.tied
        # the device arena holds the file's bytes
        lay = m.layer_handles(1)
        qt, rows, cols, dev = C.c_int(), C.c_size_t(), C.c_size_t(), C.c_void_p()
        EL.call("ef_hip_weight_info", lay.w_down, C.byref(qt), C.byref(rows), C.byref(cols), C.byref(dev))
        t = f.at("model.layers.1.mlp.down_proj.weight")
        host = np.empty(t.bytes, np.uint8)
        EL.call("ef_hip_memcpy_d2h", host.ctypes.data, dev.value, t.bytes, None)
        assert (qt.value, rows.value, cols.value) == (O.Q8_0, SMALL.D, SMALL.F)
        assert np.array_equal(host, f.data(t))
        f.close()
        m.free()


def test_batched_sequences_from_file(hip):
    print("[case] efq engine, 3 sequences", flush=True)
    hm = HostModel(SMALL, seed=52, q8={(1, "wv")})
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.efq")
        write_efq(path, SMALL, hm.efq_tensors())
        _check_engine(path, hm, batch=3).free()


def test_lossless_bf16_file(hip):
    print("[case] efq layers BF16, lm_head BF16", flush=True)
    hm = HostModel(SMALL, seed=53, layer_type=O.BF16, lm_type=O.BF16)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "bf16.efq")
        write_efq(path, SMALL, hm.efq_tensors(), layer_type=O.BF16, lm_type=O.BF16)
        m = _check_engine(path, hm)
        assert m.description == "efq, policy custom: 0 Q4_0 + 0 Q8_0 + 15 other matrices, embedding BF16"
        m.free()


def test_tied_embeddings_file(hip):
    print("[case] efq tied embeddings", flush=True)
    hm = HostModel(SMALL, seed=54)
    hm._bytes["lm_head"], hm.weights["lm_head"] = hm._bytes["embed"], hm.weights["embed"]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tied.efq")
        write_efq(path, SMALL, hm.efq_tensors(), tied=True)
        m = _check_engine(path, hm)
        assert m.tied
        emb = SMALL.V * SMALL.D * 2
        f = QuantFile.open(path)
        assert m.bytes_per_token == sum(t.bytes for t in f.tensors())  # the embedding is streamed as lm_head
        assert f.at("model.embed_tokens.weight").bytes == emb
        f.close()
        m.free()
