"""GPU parity of the device decode engine against the CPU oracle's Transformer (src/model.cpp:184-304)
on the same packed weights: logits within the GEMV tolerance at every position, identical greedy
token sequences (32 steps at the TinyLlama-1.1B shapes of config 5), batch = independent sequences,
sampled generation bit-exact given the same logits and seeds, and the reference's error checks."""
import numpy as np
import pytest

import oracle as O
from edgeforge_amd import _lib as L
from edgeforge_amd.model import TINYLLAMA, Config, DeviceModel, Engine
from tests import _data as D
from oracle.model import OracleModel

pytestmark = pytest.mark.gpu

SMALL = Config(D=256, F=512, H=4, KV=2, hd=64, V=512, L=3, max_pos=64)
ODD = Config(D=96, F=160, H=3, KV=1, hd=32, V=200, L=2, max_pos=32)  # generic (cols % 64 != 0) GEMV path
WIDE = Config(D=512, F=768, H=4, KV=2, hd=128, V=300, L=2, max_pos=64)  # head_dim 128


def _logit_err(a, b):
    return float(np.abs(a - b).max() / max(1.0, np.abs(b).max()))


def _top2_margin(l):
    s = np.sort(l)
    return float(s[-1] - s[-2])


# The reference's checker tolerates a greedy difference where its own top-1 / top-2 logit margin
# at the first differing step is below 1e-3 (README.md:603-607, src/verify_chat.cpp:193-216).  The
# committed seeds are held to the stricter bar: identical ids at every step, no tolerated flip.
# The smallest oracle margin over the compared steps is printed (pytest -s) and returned, so a
# run shows how close the closest call came.
NEAR_TIE = 1e-3


def assert_greedy_identical(got, want, want_logits, label=""):
    """Identical greedy ids over every step.  Returns the minimum top-2 margin of the oracle's
    logits over the steps.  A difference fails, and the message says whether the reference's
    near-tie rule would have tolerated it."""
    got = [int(v) for v in got]
    want = [int(v) for v in want]
    margins = [_top2_margin(l) for l in want_logits[:len(want)]]
    k = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
    assert k is None, (f"{label} greedy ids differ at step {k} ({got[k]} vs {want[k]}); the oracle's "
                       f"top-2 margin there is {margins[k]:.3e}"
                       + (" (a near-tie the reference's checker would tolerate)" if margins[k] < NEAR_TIE else ""))
    print(f"{label} greedy ids identical over {len(want)} steps; min top-2 margin {min(margins):.3e}", flush=True)
    return min(margins)


@pytest.mark.parametrize("cfg,q8", [(SMALL, {(0, "wk"), (1, "wv"), (2, "w_down")}), (ODD, {(1, "wq")}),
                                    (WIDE, {(0, "wo")})])
def test_forward_logits_match_oracle_each_position(hip, cfg, q8):
    print(f"[case] engine forward {cfg}", flush=True)
    dm = DeviceModel.synthetic(cfg, seed=7, q8=q8)
    om = OracleModel(dm)
    ids = [int(v) for v in D.rng(3).integers(0, cfg.V, 12)]
    eng = Engine(dm, max_seq=len(ids))
    ot = om.transformer(len(ids))
    for p, t in enumerate(ids):
        eng.forward([t], p)
        want = ot.forward(t, p)
        got = eng.logits()[0]
        assert _logit_err(got, want) < 1e-4, p
        assert np.abs(eng.hidden()[0] - ot.hidden()).max() < 1e-4
    # rewinding to an earlier position overwrites the cache from there (include/ef/model.h:103-104)
    for p, t in [(3, ids[5]), (4, ids[4])]:
        eng.forward([t], p)
        assert _logit_err(eng.logits()[0], ot.forward(t, p)) < 1e-4
    ot.close()
    eng.close()


def test_generate_greedy_small_matches_oracle(hip):
    dm = DeviceModel.synthetic(SMALL, seed=11, q8={(0, "wv")})
    om = OracleModel(dm)
    prompt = [int(v) for v in D.rng(5).integers(0, SMALL.V, 9)]
    want, want_logits, _, _ = om.run_once(prompt, 20)
    eng = Engine(dm, max_seq=len(prompt) + 20)
    got, pre, dec = eng.generate([prompt], 20)
    assert got[0].tolist() == want.tolist()
    assert pre > 0 and dec > 0
    eng.close()


@pytest.fixture(scope="module")
def tinyllama(hip):
    print("[case] building config-5 synthetic TinyLlama-1.1B on the device", flush=True)
    dm = DeviceModel.synthetic(TINYLLAMA, seed=2024)
    return dm, OracleModel(dm)


def test_config5_greedy_32_steps_identical(tinyllama):
    """Config 5: 23-token prompt of uniform ids, 32 greedy steps, token sequence identical to the
    CPU oracle's (src/bench_decode.cpp:30-49); logits within 1e-4 relative at every step."""
    dm, om = tinyllama
    prompt = [int(v) for v in D.rng(23).integers(0, 32000, 23)]
    want, want_logits, _, _ = om.run_once(prompt, 32)
    eng = Engine(dm, max_seq=23 + 32)
    got, pre, dec = eng.generate([prompt], 32)
    print(f"greedy tokens {got[0].tolist()}", flush=True)
    assert_greedy_identical(got[0], want, want_logits, "config 5 B=1:")
    # logits of every decode step (teacher-forced on the same tokens)
    seq = prompt + want.tolist()
    for p in range(len(prompt) + 31):
        eng.forward([seq[p]], p, compute_logits=p >= len(prompt) - 1)
        if p >= len(prompt) - 1:
            k = p - (len(prompt) - 1)
            assert _logit_err(eng.logits()[0], want_logits[k]) < 1e-4, k
    eng.close()


def test_config5_batch_of_sequences_matches_single(tinyllama):
    """Config 5 at B=4: independent prompts decode exactly as they do alone (B=1)."""
    dm, om = tinyllama
    B = 4
    prompts = D.rng(40).integers(0, 32000, size=(B, 23)).astype(np.int32)
    eng = Engine(dm, max_seq=23 + 16, batch=B)
    got, _, _ = eng.generate(prompts, 16)
    eng.close()
    one = Engine(dm, max_seq=23 + 16, batch=1)
    for b in range(B):
        single, _, _ = one.generate(prompts[b:b + 1], 16)
        assert got[b].tolist() == single[0].tolist(), b
    one.close()
    want, _, _, _ = om.run_once(prompts[1], 16)
    assert got[1].tolist() == want.tolist()


def test_config5_sampled_generation_replays_on_cpu(tinyllama, hip):
    """Sampled decode (T=0.8, top-k 40, top-p 0.95, penalty 1.1 over the context): every id the device
    picks equals the CPU sampler's pick on the device's own logits with the same seed."""
    dm, _ = tinyllama
    cfg = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    prompt = [int(v) for v in D.rng(77).integers(0, 32000, 23)]
    n = 24
    eng = Engine(dm, max_seq=23 + n)
    got, _, _ = eng.generate([prompt], n, sampler=cfg, rng=hip.RngStates([99]))
    cpu = O.Sampler(seed=99, **cfg)
    seq = list(prompt)
    for p in range(len(prompt) + n - 1):
        eng.forward([seq[p]], p, compute_logits=p >= len(prompt) - 1)
        if p >= len(prompt) - 1:
            tok = cpu.sample(eng.logits()[0], seq)
            k = p - (len(prompt) - 1)
            assert tok == int(got[0][k]), k
            seq.append(tok)
    eng.close()


# Sequences checked against the oracle in the batched config-5 runs: spread over the batch,
# including the first and the last.
def _checked(B):
    return sorted({0, B - 1, *range(0, B, max(1, B // 8))})


def _teacher_forced_logits(eng, toks_by_pos, first):
    """Logits of every sequence at positions first .. len(toks_by_pos)-1, each position run through
    the engine's one-position batched step on the given tokens: {position: [B][V]}."""
    out = {}
    for p, t in enumerate(toks_by_pos):
        eng.forward(t, p, compute_logits=p >= first)
        if p >= first:
            out[p] = eng.logits()
    return out


@pytest.mark.parametrize("B", [16, 64])
def test_config5_batched_greedy_32_steps_match_oracle(tinyllama, B):
    """Config 5 at B=16 and B=64 (config 4's shapes: the matrix-core GEMV with the K split, the
    KV-group attention, the batched argmax): independent prompts, 32 greedy steps.  Spread sequences
    (first and last included) match the oracle's run_once token for token (src/bench_decode.cpp:30-49,
    src/model.cpp:184-276), and their logits at every decode step are within 1e-4 relative."""
    dm, om = tinyllama
    n = 32
    prompts = D.rng(500 + B).integers(0, 32000, size=(B, 23)).astype(np.int32)
    print(f"[case] config-5 greedy decode at B={B}", flush=True)
    eng = Engine(dm, max_seq=23 + n, batch=B)
    got, _, _ = eng.generate(prompts, n)
    check = _checked(B)
    want = {}
    for b in check:
        toks, logits, _, _ = om.run_once(prompts[b], n)
        want[b] = (toks, logits)
        assert_greedy_identical(got[b], toks, logits, f"config 5 B={B} seq {b}:")
    # every decode step's logits on the generated tokens (teacher forced, all sequences at once)
    seqs = np.concatenate([prompts, got], axis=1)
    tf = _teacher_forced_logits(eng, [seqs[:, p] for p in range(23 + n - 1)], 22)
    worst = 0.0
    for b in check:
        toks, logits = want[b]
        for k in range(n):
            e = _logit_err(tf[22 + k][b], logits[k])
            worst = max(worst, e)
            assert e < 1e-4, (b, k, e)
    print(f"B={B}: worst relative logit error over {len(check)} sequences x {n} steps {worst:.2e}", flush=True)
    eng.close()


def test_config5_batched_sampled_replays_on_cpu(tinyllama, hip, monkeypatch):
    """Config 5 at B=64 with config 3's sampler (T 0.8, top-k 40, top-p 0.95, penalty 1.1 over the
    context), one seed per sequence: every id of every sequence equals the CPU Sampler's pick
    (src/sampler.cpp:13-70, one Sampler per sequence) on the device's own logits of that step.
    The prompt goes through the decode step too (EF_HIP_PREFILL=serial), so the teacher-forced
    replay recomputes exactly the logits the generation sampled from: the batched prefill agrees
    with the decode step to the products' rounding only, and a sampled id whose uniform draw falls
    that close to a boundary of the cumulative distribution would move."""
    monkeypatch.setenv("EF_HIP_PREFILL", "serial")
    dm, _ = tinyllama
    B, n = 64, 32
    cfg = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    prompts = D.rng(700).integers(0, 32000, size=(B, 23)).astype(np.int32)
    seeds = [9000 + 31 * b for b in range(B)]
    print("[case] config-5 sampled decode at B=64", flush=True)
    eng = Engine(dm, max_seq=23 + n, batch=B)
    got, _, _ = eng.generate(prompts, n, sampler=cfg, rng=hip.RngStates(seeds))
    seqs = np.concatenate([prompts, got], axis=1)
    tf = _teacher_forced_logits(eng, [seqs[:, p] for p in range(23 + n - 1)], 22)
    eng.close()
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    for k in range(n):
        for b in range(B):
            hist = seqs[b, :23 + k]
            tok = cpu[b].sample(tf[22 + k][b], hist)
            assert tok == int(got[b][k]), (b, k)


def test_engine_rejects_bad_tokens_and_positions(tinyllama):
    dm, _ = tinyllama
    eng = Engine(dm, max_seq=8)
    with pytest.raises(L.HipError, match="outside"):
        eng.forward([32000], 0)
    with pytest.raises(L.HipError, match="skips ahead"):
        eng.forward([1], 1)
    with pytest.raises(L.HipError, match="exceeds the KV-cache"):
        eng.generate([[1, 2, 3, 4, 5]], 4)
    with pytest.raises(L.HipError, match="empty prompt"):
        eng.generate(np.zeros((1, 0), np.int32), 2)
    eng.forward([1], 0)
    eng.close()


@pytest.mark.parametrize("cfg", [SMALL, ODD, WIDE])
def test_group_attention_forward_matches_oracle(hip, cfg, monkeypatch):
    """The KV-group decode attention (one workgroup per KV group and sequence, forced here at B=1;
    ODD has three query heads per group) against the oracle's Transformer at every position."""
    print(f"[case] group attention forward {cfg}", flush=True)
    monkeypatch.setenv("EF_HIP_ATTENTION", "group")
    dm = DeviceModel.synthetic(cfg, seed=13)
    om = OracleModel(dm)
    ids = [int(v) for v in D.rng(8).integers(0, cfg.V, 12)]
    eng = Engine(dm, max_seq=len(ids))
    ot = om.transformer(len(ids))
    for p, t in enumerate(ids):
        eng.forward([t], p)
        assert _logit_err(eng.logits()[0], ot.forward(t, p)) < 1e-4, p
    ot.close()
    eng.close()


@pytest.mark.parametrize("cfg,B", [(ODD, 3), (WIDE, 2), (TINYLLAMA, 8)])
def test_group_attention_bit_identical_to_per_head(hip, cfg, B, monkeypatch):
    """Both decode attention kernels keep the reference's operation order per head, so a batch
    decoded with either gives identical logits and tokens."""
    print(f"[case] group vs per-head attention {cfg.D}x{cfg.L} B={B}", flush=True)
    dm = DeviceModel.synthetic(cfg, seed=17)
    prompts = D.rng(41).integers(0, cfg.V, size=(B, 9)).astype(np.int32)
    out = {}
    for kind in ("head", "group"):
        monkeypatch.setenv("EF_HIP_ATTENTION", kind)
        eng = Engine(dm, max_seq=9 + 12, batch=B)
        toks, _, _ = eng.generate(prompts, 12)
        out[kind] = (toks, eng.logits())
        eng.close()
    assert np.array_equal(out["head"][0], out["group"][0])
    assert np.array_equal(out["head"][1], out["group"][1])


LONG = Config(D=256, F=512, H=4, KV=2, hd=64, V=512, L=2, max_pos=512)


def test_long_context_decode_matches_oracle(hip):
    """Decode past a 280-token prompt: the per-head attention stages the positions after its first
    64 in one LDS-DMA chunk; greedy tokens and the last logits match the oracle."""
    print("[case] long-context decode, 280-token prompt", flush=True)
    dm = DeviceModel.synthetic(LONG, seed=19)
    om = OracleModel(dm)
    prompt = [int(v) for v in D.rng(9).integers(0, LONG.V, 280)]
    want, want_logits, _, _ = om.run_once(prompt, 12)
    eng = Engine(dm, max_seq=300)
    got, _, _ = eng.generate([prompt], 12)
    assert got[0].tolist() == want.tolist()
    assert _logit_err(eng.logits()[0], want_logits[-1]) < 1e-4
    eng.close()


@pytest.mark.parametrize("kind", ["wave", "head", "split"])
def test_decode_attention_across_the_first_chunk_matches_oracle(hip, kind, monkeypatch):
    """Greedy decode from a 58-token prompt through positions 58..69, across the 64-position
    boundary where the one-wave kernel moves from the rows it loads at entry to loaded chunks (and
    the position-split kernel from one split to two, combined by the last to arrive); forced per
    kernel, tokens and every step's logits match the oracle."""
    print(f"[case] decode across position 64, attention={kind}", flush=True)
    monkeypatch.setenv("EF_HIP_ATTENTION", kind)
    dm = DeviceModel.synthetic(LONG, seed=31)
    om = OracleModel(dm)
    prompt = [int(v) for v in D.rng(12).integers(0, LONG.V, 58)]
    want, want_logits, _, _ = om.run_once(prompt, 12)
    eng = Engine(dm, max_seq=80)
    got, _, _ = eng.generate([prompt], 12)
    assert got[0].tolist() == want.tolist()
    assert _logit_err(eng.logits()[0], want_logits[-1]) < 1e-4
    eng.close()


def test_wave_attention_short_cache_matches_oracle(hip, monkeypatch):
    """max_seq below 64: the one-wave kernel's entry loads past the cache's last row read zeros
    through the buffer range and are never used; every position's logits match the oracle."""
    print("[case] wave attention, max_seq 12", flush=True)
    monkeypatch.setenv("EF_HIP_ATTENTION", "wave")
    dm = DeviceModel.synthetic(SMALL, seed=37)
    om = OracleModel(dm)
    ids = [int(v) for v in D.rng(10).integers(0, SMALL.V, 12)]
    eng = Engine(dm, max_seq=len(ids))
    ot = om.transformer(len(ids))
    for p, t in enumerate(ids):
        eng.forward([t], p)
        assert _logit_err(eng.logits()[0], ot.forward(t, p)) < 1e-4, p
    ot.close()
    eng.close()


def test_long_context_group_and_head_attention_identical(hip, monkeypatch):
    """Positions 250..261: the per-head kernel (large LDS-DMA chunks) and the KV-group kernel
    (64-row chunks) give identical logits and tokens."""
    print("[case] long-context group vs per-head attention", flush=True)
    dm = DeviceModel.synthetic(LONG, seed=23)
    prompts = D.rng(43).integers(0, LONG.V, size=(2, 250)).astype(np.int32)
    out = {}
    for kind in ("head", "group"):
        monkeypatch.setenv("EF_HIP_ATTENTION", kind)
        eng = Engine(dm, max_seq=300, batch=2)
        toks, _, _ = eng.generate(prompts, 12)
        out[kind] = (toks, eng.logits())
        eng.close()
    assert np.array_equal(out["head"][0], out["group"][0])
    assert np.array_equal(out["head"][1], out["group"][1])


@pytest.mark.parametrize("B", [1, 3])
def test_engine_profile_groups_and_state(hip, B):
    """ef_hip_engine_profile times every kernel group of a step and puts the position back: each
    group has a positive time, the groups add up to about one step, and decoding afterwards from
    the same state gives the same tokens as before."""
    print(f"[case] engine profile B={B}", flush=True)
    dm = DeviceModel.synthetic(SMALL, seed=29)
    prompts = D.rng(47).integers(0, SMALL.V, size=(B, 9)).astype(np.int32)
    eng = Engine(dm, max_seq=9 + 12, batch=B)
    first, _, dec = eng.generate(prompts, 12)
    prof = eng.profile(reps=5)
    assert set(prof) == set(Engine.PROFILE_GROUPS)
    assert all(v > 0.0 and np.isfinite(v) for v in prof.values()), prof
    again, _, _ = eng.generate(prompts, 12)
    assert np.array_equal(first, again)
    prof_s = eng.profile(reps=5, sampler=dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),
                         rng=hip.RngStates(list(range(B))))
    assert prof_s["pick"] > 0.0
    eng.close()


# ---- several-sequence steps over producer-staged product inputs ----

TWO_LAYER = Config(D=2048, F=5632, H=32, KV=4, hd=64, V=1024, L=2, max_pos=128)  # TinyLlama's layer shapes


@pytest.mark.parametrize("cfg,B,q8,attn", [
    (SMALL, 3, {(0, "wk"), (1, "wv"), (2, "w_down")}, None),  # per-head attention: o's input prepared
    (ODD, 5, {(1, "wq")}, "group"),  # KV-group attention stages o's input; K = 96, three heads per group
    (TWO_LAYER, 64, frozenset(), None),  # TinyLlama's layer shapes at B=64 (KV-group attention, K split)
    (TWO_LAYER, 16, frozenset({(0, "wk"), (0, "wv"), (1, "w_down")}), None),
])
def test_staged_tables_match_per_product_preparation(hip, cfg, B, q8, attn, monkeypatch):
    """A several-sequence engine stages every product's input in the producing kernel (embedding,
    attention, o / gate-up / down epilogues); its logits at every position equal those of the
    per-product preparation (EF_HIP_DECODE_TABLES=prep) to float rounding, and the first and last
    sequences match the oracle's Transformer."""
    print(f"[case] staged tables vs preparation D={cfg.D} L={cfg.L} B={B} q8={sorted(q8)} attn={attn}", flush=True)
    if attn is not None:
        monkeypatch.setenv("EF_HIP_ATTENTION", attn)
    dm = DeviceModel.synthetic(cfg, seed=51, q8=q8)
    n = 10
    ids = D.rng(52).integers(0, cfg.V, size=(B, n)).astype(np.int32)
    logits = {}
    for kind in ("staged", "prep"):
        if kind == "prep":
            monkeypatch.setenv("EF_HIP_DECODE_TABLES", "prep")
        else:
            monkeypatch.delenv("EF_HIP_DECODE_TABLES", raising=False)
        eng = Engine(dm, max_seq=n, batch=B)
        on, why = eng.staged_tables()
        assert on == (kind == "staged"), why
        logits[kind] = _teacher_forced_logits(eng, [ids[:, p] for p in range(n)], 0)
        eng.close()
    worst = max(_logit_err(logits["staged"][p][b], logits["prep"][p][b]) for p in range(n) for b in range(B))
    print(f"staged vs prep: worst relative logit difference {worst:.2e}", flush=True)
    assert worst < 1e-5
    om = OracleModel(dm)
    for b in (0, B - 1):
        ot = om.transformer(n)
        for p in range(n):
            assert _logit_err(logits["staged"][p][b], ot.forward(int(ids[b, p]), p)) < 1e-4, (b, p)
        ot.close()


def test_staged_tables_off_where_they_do_not_apply(hip, monkeypatch):
    """One sequence, or EF_HIP_DECODE_TABLES=prep at creation: the engine says why it prepares each
    product's input itself."""
    dm = DeviceModel.synthetic(SMALL, seed=3)
    eng = Engine(dm, max_seq=16)
    on, why = eng.staged_tables()
    assert not on and "one sequence" in why
    eng.close()
    monkeypatch.setenv("EF_HIP_DECODE_TABLES", "prep")
    eng = Engine(dm, max_seq=16, batch=4)
    on, why = eng.staged_tables()
    assert not on and "EF_HIP_DECODE_TABLES" in why
    eng.close()
