"""GPU chat turns (ef_hip_engine_reply): the token-level ChatSession::reply (src/chat.cpp:174-259).

1. The reference's own scripted-model cases (tests/test_chat.cpp:186-300): every layer matrix zero,
   a one-hot embedding and an lm_head that makes the greedy next token a fixed function of the
   current one, so the exact reply is known: a reply ending in EOS, a loop stopped by max-new, the
   context limit, and EOS as a close second stopped only by eos_min_p -- with the reference's
   expected replies, stop reasons and P(EOS) figures.  The model is an .efq file of BF16 tensors.
2. Sampled multi-turn conversations on a random model against the oracle's ChatSession
   restatement (oracle/model.py OracleChat): identical ids turn after turn (so the RNG advances
   exactly as the reference's Sampler even though the device runs ahead in windows of steps),
   identical prefix reuse, P(EOS) per step within the logits' tolerance, and equal to prob_of of the
   device's own logits to 1e-12 relative (the fused computation itself).
"""
import os
import tempfile

import numpy as np
import pytest

from edgeforge_amd import _lib as EL
from edgeforge_amd import hip as H
from edgeforge_amd.model import Config, DeviceModel, Engine
from edgeforge_amd.qfile import EfqModel
from oracle.efq import write_efq
from oracle.model import OracleChat, OracleModel, prob_of
from tests import _data as D

pytestmark = pytest.mark.gpu

K_A, K_B, K_C, K_EOS = 265, 266, 267, 2
NL = 3 + ord("\n")
LT, SL, S_, GT = 3 + ord("<"), 3 + ord("/"), 3 + ord("s"), 3 + ord(">")
TINY = Config(D=16, F=24, H=4, KV=2, hd=4, V=272, L=2, max_pos=256)  # tests/tiny_model.h:23 with the mini vocab


def bf16(a):
    a = np.ascontiguousarray(a, np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)  # the values used here are exact in BF16


def scripted(path, nxt: dict, eos_second=()):
    """tests/test_chat.cpp:54-84: next[token] is the greedy successor; EOS a close second after
    the tokens in eos_second."""
    cfg = TINY
    dim = {src: i for i, src in enumerate(nxt)}
    emb = np.zeros((cfg.V, cfg.D), np.float32)
    for r in range(cfg.V):
        emb[r, dim.get(r, cfg.D - 1)] = 1.0
    lm = np.zeros((cfg.V, cfg.D), np.float32)
    for src, dst in nxt.items():
        lm[dst, dim[src]] = 10.0
        if src in eos_second:
            lm[K_EOS, dim[src]] = 9.9
    t = {"embed": (2, bf16(emb)), "lm_head": (2, bf16(lm)), "final": np.ones(cfg.D, np.float32)}
    kvd = cfg.KV * cfg.hd
    shapes = {"wq": (cfg.D, cfg.D), "wk": (kvd, cfg.D), "wv": (kvd, cfg.D), "wo": (cfg.D, cfg.D),
              "w_gate": (cfg.F, cfg.D), "w_up": (cfg.F, cfg.D), "w_down": (cfg.D, cfg.F)}
    for l in range(cfg.L):
        for k, shp in shapes.items():
            t[(l, k)] = (2, np.zeros(shp, np.uint16))
        t[(l, "attn")] = np.ones(cfg.D, np.float32)
        t[(l, "ffn")] = np.ones(cfg.D, np.float32)
    write_efq(path, cfg, t, layer_type=2, lm_type=2)
    return EfqModel.load_efq(path)


PROMPT = [1, 260, 261, 262, NL]  # BOS, a few user ids, the template's closing newline


def test_scripted_eos_max_new_and_context(hip):
    with tempfile.TemporaryDirectory() as d:
        m = scripted(os.path.join(d, "a.efq"), {NL: K_A, K_A: K_B, K_B: K_EOS})
        eng = m.engine(max_seq=256)
        reply, peos, st = eng.reply(PROMPT, 64, eos_id=K_EOS)
        assert reply.tolist() == [K_A, K_B] and st.reason == EL.STOP_EOS
        assert st.eos_p_max > 0.9 and st.eos_p_max_step == 2 and st.steps == 3
        assert st.prompt_tokens == len(PROMPT) and st.reused_tokens == 0
        eng.close()
        m.free()
        loop = scripted(os.path.join(d, "b.efq"), {NL: K_A, K_A: K_B, K_B: K_C, K_C: K_A})
        eng = loop.engine(max_seq=256)
        reply, _, st = eng.reply(PROMPT, 20, eos_id=K_EOS, steps_per_check=3)
        assert st.reason == EL.STOP_MAX_NEW and st.generated == 20
        assert reply.tolist() == ([K_A, K_B, K_C] * 7)[:20]
        eng.close()
        eng = loop.engine(max_seq=len(PROMPT) + 5)  # the context runs out before max_new
        _, _, st = eng.reply(PROMPT, 64, eos_id=K_EOS)
        assert st.reason == EL.STOP_CONTEXT and st.generated == 5
        eng.close()
        loop.free()


@pytest.mark.parametrize("window", [1, 3, 8])
def test_scripted_eos_min_p(hip, window):
    with tempfile.TemporaryDirectory() as d:
        m = scripted(os.path.join(d, "c.efq"), {NL: K_A, K_A: K_B, K_B: K_C, K_C: K_C}, eos_second=(K_B,))
        eng = m.engine(max_seq=256)
        reply, peos, st = eng.reply(PROMPT, 8, eos_id=K_EOS, steps_per_check=window)
        assert st.reason == EL.STOP_MAX_NEW  # greedy continues past the close second
        assert 0.3 < st.eos_p_max < 0.5 and st.eos_p_max_step == 2
        eng.reset()
        reply, _, st = eng.reply(PROMPT, 8, eos_id=K_EOS, eos_min_p=0.3, steps_per_check=window)
        assert reply.tolist() == [K_A, K_B] and st.reason == EL.STOP_EOS_MIN_P
        eng.close()
        m.free()


SMALL = Config(D=256, F=512, H=4, KV=2, hd=64, V=512, L=2, max_pos=128)


@pytest.mark.parametrize("sampler,window", [
    ({"temperature": 0.8, "top_k": 40, "top_p": 0.95, "repetition_penalty": 1.1, "seed": 5}, 4),
    ({"temperature": 1.0, "top_k": 0, "top_p": 1.0, "repetition_penalty": 1.0, "seed": 9}, 1),
    ({"temperature": 0.0, "repetition_penalty": 1.3}, 8),
])
def test_multi_turn_matches_oracle_chat(hip, sampler, window):
    print(f"[case] chat multi-turn {sampler} window={window}", flush=True)
    dm = DeviceModel.synthetic(SMALL, seed=71, q8={(1, "wk")})
    om = OracleModel(dm)
    max_seq = 120
    # find an EOS id the first turn will meet: the 4th token of a free run (same RNG path)
    free = OracleChat(om, max_seq, sampler)
    first = [int(v) for v in D.rng(80).integers(3, SMALL.V, 9)]
    g0, _, _, _ = free.reply(first, 12)
    free.close()
    eos = g0[3]
    ref = OracleChat(om, max_seq, sampler)
    eng = Engine(dm, max_seq=max_seq)
    rng = H.RngStates([sampler.get("seed", 0)]) if sampler["temperature"] > 0 else None
    ids = first
    for turn in range(3):
        want, want_p, want_reason, want_lcp = ref.reply(ids, 12, eos_id=eos)
        got, got_p, st = eng.reply(ids, 12, sampler=sampler, rng=rng, eos_id=eos, steps_per_check=window)
        assert got.tolist() == want, turn
        assert st.reason == want_reason and st.reused_tokens == want_lcp, turn
        # P(EOS) from the device's own logits: to the logits' 1e-4 tolerance against the oracle's
        assert np.allclose(got_p, want_p, rtol=1e-4, atol=0), turn
        if window == 1:  # no steps past the stop: the engine's logits are the last step's
            assert abs(got_p[-1] - prob_of(eng.logits()[0], eos)) <= 1e-12 * got_p[-1], turn
        ids = ids + want + [int(v) for v in D.rng(90 + turn).integers(3, SMALL.V, 4)]  # the next user message
    assert st.reused_tokens > 0
    ref.close()
    eng.close()
