"""eval-quant on the GPU (src/eval_quant.cpp): chunking of the text (CPU), compare_dist and
neg_log_prob on device logits against a float64 restatement (pinned by closed forms), teacher-forced
scoring against the oracle's Transformer, and the harness's invariants (a model against itself:
KL 0, every top-1 agreeing, perplexity ratio 1)."""
import math

import numpy as np
import pytest

from edgeforge_amd.eval_quant import run_text_eval, text_chunks


def np_lse(x):
    x = x.astype(np.float64)
    m = x.max()
    s = 0.0
    for v in np.exp(x - m):
        s += v
    return m + math.log(s)


def np_compare(ref, ours):
    """compare_dist (src/eval_quant.cpp:60-75) in float64, sums left to right."""
    if not np.all(np.isfinite(ours)):
        return None
    lr, lq = np_lse(ref), np_lse(ours)
    a, b = ref.astype(np.float64) - lr, ours.astype(np.float64) - lq
    kl = 0.0
    for x, y in zip(a, b):
        kl += math.exp(x) * (x - y)
    ar, aq = int(np.argmax(ref)), int(np.argmax(ours))  # first maximum, as kern::argmax without NaNs
    return max(kl, 0.0), ar == aq, math.exp(float(ref[ar]) - lr) >= 0.5


def test_restatement_closed_forms():
    p = np.array([0.0, math.log(3.0)], np.float32)  # P = (1/4, 3/4)
    q = np.array([0.0, 0.0], np.float32)            # Q = (1/2, 1/2)
    kl, top1, conf = np_compare(p, q)
    want = 0.25 * math.log(0.5) + 0.75 * math.log(1.5)
    assert abs(kl - want) < 1e-7 and conf and not top1  # argmax(q) = 0: ties go to the first index
    assert np_compare(p, p)[0] == 0.0
    assert np_compare(p, np.array([0, np.inf], np.float32)) is None


def test_text_chunks_follow_the_reference_scheme():
    ids = list(range(100, 150))
    assert text_chunks(ids, 0, max_text_tokens=20) == [(ids[:20], 0)]
    ch = text_chunks(ids, 16, bos_id=1)
    assert len(ch) == 3 and all(len(c) == 16 and c[0] == 1 and f == 8 for c, f in ch)
    assert ch[1][0][1:] == ids[17:32]
    assert len(text_chunks(ids, 16, max_chunks=2)) == 2
    with pytest.raises(ValueError, match="at least 4"):
        text_chunks(ids, 3)
    assert text_chunks([5], 0) == []


@pytest.mark.gpu
def test_compare_dist_on_device_matches_float64(hip):
    from edgeforge_amd.eval_quant import compare_dist
    V, n = 1000, 9
    g = np.random.default_rng(3)
    ref = (g.standard_normal((n, V)) * 3).astype(np.float32)
    ours = ref + (g.standard_normal((n, V)) * 0.3).astype(np.float32)
    ours[1] = ref[1]                        # identical: KL 0
    ref[2, 17] = 40.0                       # confident reference
    ours[3, 5] = np.nan                     # non-finite
    ref[4, :] = 0.0
    ref[4, [7, 9]] = 5.0                    # tie: the first index is the reference's top-1
    ours[4, :] = 0.0
    ours[4, [9, 7]] = [5.0, 4.0]
    kl, agg = compare_dist(hip.DeviceArray.from_host(ref), hip.DeviceArray.from_host(ours), V, n)
    want = [np_compare(ref[p], ours[p]) for p in range(n)]
    fin = [w for w in want if w is not None]
    assert agg.n == n and agg.nonfinite == 1
    for p, w in enumerate(want):
        if w is not None:
            assert abs(kl[p] - w[0]) <= 1e-12 + 1e-10 * w[0], p
    assert kl[1] == 0.0
    assert agg.top1 == sum(w[1] for w in fin) and agg.confident == sum(w[2] for w in fin)
    assert agg.confident_top1 == sum(w[1] and w[2] for w in fin)
    assert abs(agg.kl_mean - np.mean([w[0] for w in fin])) < 1e-12
    assert not want[4][1]  # ref picks 7, ours 9


@pytest.fixture(scope="module")
def models(hip):
    from edgeforge_amd import _lib as L
    from edgeforge_amd.model import Config, DeviceModel
    cfg = Config(D=256, F=512, H=4, KV=2, hd=64, V=512, L=2, max_pos=128)
    q = DeviceModel.synthetic(cfg, seed=81)
    bf = DeviceModel.synthetic(cfg, seed=81, layer_type=L.BF16, lm_type=L.BF16)  # the same floats, lossless
    return cfg, q, bf


@pytest.mark.gpu
@pytest.mark.parametrize("first,rows", [(0, None), (20, None), (5, "7")])
def test_score_matches_oracle(models, monkeypatch, first, rows):
    from edgeforge_amd.model import Engine
    from oracle.model import OracleModel
    cfg, q, _ = models
    if rows:
        monkeypatch.setenv("EF_HIP_PREFILL_ROWS", rows)
    ids = [int(v) for v in np.random.default_rng(5).integers(0, cfg.V, 40)]
    eng = Engine(q, max_seq=64)
    got = eng.score(ids, first)
    ot = OracleModel(q).transformer(64, threads=2)
    want = []
    for p in range(len(ids) - 1):
        lg = ot.forward(ids[p], p, p >= first)
        if p >= first:
            want.append(np_lse(lg) - float(lg[ids[p + 1]]))
    assert np.abs(got - np.array(want)).max() < 2e-4
    ot.close()
    eng.close()


@pytest.mark.gpu
def test_harness_invariants(models):
    cfg, q, bf = models
    ids = [int(v) for v in np.random.default_rng(6).integers(0, cfg.V, 70)]
    same = run_text_eval(q, q, ids, window=32, bos_id=1)
    assert same.positions == same.n_scored == 2 * 15
    assert same.kl_mean == 0.0 and same.top1 == same.positions and same.ppl_q == same.ppl_ref
    assert same.failed == 0
    r = run_text_eval(q, bf, ids, window=0, max_text_tokens=64)
    assert r.positions == r.n_scored == 63 and r.kl_mean > 0 and r.ppl_q > 0 and r.ppl_ref > 0
    print(f"Q4_0 vs BF16 (random weights): KL mean {r.kl_mean:.4f}, top-1 {r.top1}/{r.positions}, "
          f"PPL {r.ppl_ref:.2f} -> {r.ppl_q:.2f}", flush=True)
