"""Decode at the reference's full context (max_position_embeddings = 2048, src/model.cpp:165-167):
attention over every cached position (src/kernels.cpp:153-174) through position 2047 at the
TinyLlama-1.1B shapes of config 5, at B=1 and B=16, against the CPU oracle's Transformer
(src/model.cpp:184-304).  At these cache lengths the decode step splits each (sequence, KV group)'s
positions over several workgroups and combines their partial softmax sums in a fixed order, so
logits are checked within the GEMV tolerance (1e-4 relative) and greedy ids must be identical."""
import numpy as np
import pytest

from edgeforge_amd.model import TINYLLAMA, Config, DeviceModel, Engine
from oracle.model import OracleModel
from tests import _data as D
from tests.test_gpu_engine import _logit_err, assert_greedy_identical

pytestmark = pytest.mark.gpu

MAX = 2048
PROMPT = 2000
STEPS = MAX - PROMPT  # decode forwards at positions 2000..2047
CHECK = (PROMPT - 1, 2024, 2040, 2046, MAX - 1)  # positions whose logits are checked


@pytest.fixture(scope="module")
def tinyllama(hip):
    print("[case] building config-5 synthetic TinyLlama-1.1B on the device", flush=True)
    dm = DeviceModel.synthetic(TINYLLAMA, seed=2024)
    return dm, OracleModel(dm)


def _oracle_greedy(om, prompt):
    """The reference decode loop (src/bench_decode.cpp:30-49) on the oracle's Transformer with a
    2048-position cache, through the forward at position 2047: (ids [STEPS + 1], logits by
    position)."""
    ot = om.transformer(MAX)
    lg = None
    for p, t in enumerate(prompt):
        lg = ot.forward(int(t), p, compute_logits=p == len(prompt) - 1)
    toks, by_pos = [], {}
    for k in range(STEPS + 1):
        by_pos[PROMPT - 1 + k] = lg.copy()
        toks.append(int(np.argmax(lg)))  # kern::argmax: first maximum
        if k < STEPS:
            lg = ot.forward(toks[-1], PROMPT + k)
    ot.close()
    return np.array(toks), by_pos


@pytest.mark.parametrize("B", [1, 16])
def test_decode_through_position_2047_matches_oracle(tinyllama, B):
    dm, om = tinyllama
    prompts = D.rng(2047 + B).integers(0, 32000, size=(B, PROMPT)).astype(np.int32)
    print(f"[case] config-5 decode to position 2047 at B={B}", flush=True)
    eng = Engine(dm, max_seq=MAX, batch=B)
    got, pre, dec = eng.generate(prompts, STEPS)  # picks from the forwards at 1999..2046
    print(f"B={B}: prefill {PROMPT} positions {pre:.3f}s, {STEPS - 1} steps at 2000..2046 "
          f"{dec / (STEPS - 1) * 1e6:.1f} us/step", flush=True)
    seqs = np.concatenate([prompts, got], axis=1)  # MAX tokens: positions 0..2047
    tf = {}
    for p in range(PROMPT - 1, MAX):  # teacher forced from 1999 (a forward at p drops the cache past p)
        eng.forward(seqs[:, p], p, compute_logits=p in CHECK)
        if p in CHECK:
            tf[p] = eng.logits()
    eng.close()
    last = np.argmax(tf[MAX - 1], axis=1)
    for b in sorted({0, B - 1}):
        print(f"[case] oracle run, sequence {b} of {B}", flush=True)
        toks, logits = _oracle_greedy(om, prompts[b])
        ours = np.append(got[b], last[b])
        assert_greedy_identical(ours, toks, [logits[PROMPT - 1 + k] for k in range(STEPS + 1)],
                                f"2047 B={B} seq {b}:")
        for p in CHECK:
            e = _logit_err(tf[p][b], logits[p])
            assert e < 1e-4, (b, p, e)


SPLITS = Config(D=512, F=768, H=8, KV=1, hd=64, V=512, L=2, max_pos=512)  # 8 query heads per KV head


@pytest.mark.parametrize("B", [1, 3])
def test_position_split_equals_single_pass_within_tolerance(hip, B, monkeypatch):
    """A 400-position cache, 8 query heads per KV head: every step's logits from the position-split
    kernel (up to 7 splits, combined by the last to arrive) match the oracle's at every decode
    position and the single-pass kernel's within 1e-5 relative; both runs give identical greedy
    ids, and a second run of the split kernel reproduces its logits bit for bit."""
    dm = DeviceModel.synthetic(SPLITS, seed=41)
    om = OracleModel(dm)
    prompts = D.rng(43 + B).integers(0, SPLITS.V, size=(B, 380)).astype(np.int32)
    out = {}
    for kind in ("split", "head", "split"):
        monkeypatch.setenv("EF_HIP_ATTENTION", kind)
        print(f"[case] 400-position cache, attention={kind}, B={B}", flush=True)
        eng = Engine(dm, max_seq=400, batch=B)
        toks, _, _ = eng.generate(prompts, 20)
        seqs = np.concatenate([prompts, toks], axis=1)
        lg = []
        for p in range(379, 399):
            eng.forward(seqs[:, p], p)
            lg.append(eng.logits())
        eng.close()
        if kind in out:
            assert np.array_equal(np.array(lg).view(np.uint32), np.array(out[kind][1]).view(np.uint32))
        out[kind] = (toks, lg)
    assert np.array_equal(out["split"][0], out["head"][0])
    worst = max(_logit_err(a, b) for a, b in zip(out["split"][1], out["head"][1]))
    assert worst < 1e-5, worst
    want, want_logits, _, _ = om.run_once(prompts[0], 20)
    assert out["split"][0][0].tolist() == want.tolist()
    for k in range(20):
        assert _logit_err(out["split"][1][k][0], want_logits[k]) < 1e-4, k
