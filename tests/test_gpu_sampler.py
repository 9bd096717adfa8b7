"""GPU parity of argmax and the sampler: token ids bit-identical to the reference's, on identical
logits and seeds (src/sampler.cpp:13-70; oracle/efo_sampler.c pinned to the reference build)."""
import numpy as np
import pytest

import oracle as O
from edgeforge_amd import _lib as EL
from tests import _data as D

pytestmark = pytest.mark.gpu


def _argmax(H, x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, x.shape[-1])
    out = H.DeviceArray((x.shape[0],), np.int32)
    H.argmax(H.DeviceArray.from_host(x), x.shape[1], out, batch=x.shape[0])
    return out.numpy()


def test_argmax_first_max_ties_nan(hip):
    assert _argmax(hip, np.array([0.5, 3.0, -1.0, 3.0], np.float32))[0] == 1  # tests/test_kernels.cpp:251
    x = np.full(32000, -np.inf, np.float32)
    assert _argmax(hip, x)[0] == 0
    x[31999] = 0.0
    x[17] = 0.0
    assert _argmax(hip, x)[0] == 17
    y = D.normal(1, 32000)
    y[5] = np.nan
    assert _argmax(hip, y)[0] == O.lib().efo_argmax(O.ptr(y, O._f32p), 32000)
    y[0] = np.nan  # a NaN first element is never replaced in the sequential scan
    assert _argmax(hip, y)[0] == 0
    many = D.normal(2, (64, 32000), 3.0)
    got = _argmax(hip, many)
    assert [int(v) for v in got] == [int(np.argmax(r)) for r in many]


def _exp_sweep_points():
    """Arguments of the sweep, all in [-746, 0]: every 64th float (the sampler's exp arguments are
    float differences w - max, widened), 2^22 uniform doubles, and the boundaries (0, -0, the
    subnormal-result and underflow thresholds and their neighbours)."""
    top = np.float32(-746.0).view(np.uint32)
    floats = np.arange(0x80000000, int(top) + 1, 64, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rand = -D.rng(4242).uniform(0.0, 746.0, 1 << 22)
    edges = np.array([0.0, -0.0, -1e-300, -708.3964185322641, -708.39641853226419, -709.782712893384,
                      -744.44007192138122, -745.13321910194110, -745.1332191019412, -745.13321910194122], np.float64)
    near = np.concatenate([np.nextafter(edges, -np.inf), np.nextafter(edges, np.inf)])
    x = np.concatenate([floats.astype(np.float64), rand, edges, near])
    return x[(x <= 0.0) & (x >= -746.0)]


def test_device_exp_matches_host_libm(hip):
    """The sampler's one libm call, exp(double) of the softmax terms (src/sampler.cpp:46, std::exp
    from glibc on the reference's host): the device's exp_libm is bit-identical to the host's over
    every sweep point (about 2^24.4 of them).  (The device libm's own exp differed by one ulp on
    362,788 of these points, 1.6%.)"""
    x = _exp_sweep_points()
    n = x.size
    print(f"[case] exp(double) sweep over {n} points in [-746, 0]", flush=True)
    assert n >= 1 << 20
    dx = hip.DeviceArray.from_host(x)
    dy = hip.DeviceArray((n,), np.float64)
    hip.sampler_exp(dx, dy, n)
    got = dy.numpy()
    want = O.exp_array(x)
    diff = got.view(np.int64) - want.view(np.int64)  # both non-negative: ulp distance
    bad = np.flatnonzero(diff)
    print(f"exp sweep: {bad.size} of {n} differ, max {np.abs(diff).max() if n else 0} ulp", flush=True)
    assert bad.size == 0, (f"{bad.size} of {n} arguments differ (max {np.abs(diff).max()} ulp), e.g. "
                           + ", ".join(f"exp({x[i]!r}) = {got[i]!r} vs {want[i]!r}" for i in bad[:5]))


CONFIGS = [
    dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),  # config 3
    dict(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0),  # CLI defaults with --temp 1
    dict(temperature=0.7, top_k=0, top_p=0.9, repetition_penalty=1.3),
    dict(temperature=1.5, top_k=1000, top_p=1.0, repetition_penalty=1.0),
    dict(temperature=0.0, top_k=0, top_p=1.0, repetition_penalty=1.2),  # greedy with penalty
    dict(temperature=5.0, top_k=1, top_p=1.0, repetition_penalty=1.0),
    dict(temperature=1.0, top_k=0, top_p=1e-6, repetition_penalty=1.0),
    dict(temperature=2.0, top_k=2000, top_p=0.5, repetition_penalty=1.0),  # k above the LDS path
]


@pytest.mark.parametrize("batch", [4, 16, 64])
@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_sampler_ids_bit_exact_over_steps(hip, ci, batch):
    """One Sampler per sequence (config 4's per-sequence sampling on [B, 32000] at B = 16 and 64):
    every sequence's id equals its own CPU Sampler's, step after step (the RNG states advance
    independently).  Configurations without top-k (or k above 1024) take the split full sort."""
    cfg = CONFIGS[ci]
    V, steps = 32000, 12 if batch <= 16 else 6
    print(f"[case] sampler B={batch} {cfg}", flush=True)
    seeds = [1234 + 17 * b for b in range(batch)]
    rng = hip.RngStates(seeds)
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    ws = hip.DeviceArray((EL.lib().ef_hip_sample_workspace_bytes(V, batch),), np.uint8)
    g = D.rng(100 + ci)
    for step in range(steps):
        scale = 3.0 if step % 2 == 0 else 1.0
        logits = (g.standard_normal((batch, V), dtype=np.float32) * np.float32(scale)).astype(np.float32)
        if step == 3:
            logits[:, 100:110] = logits[:, 100:101]  # exact ties resolved by lower id
        hist = g.integers(0, V, size=(batch, 64)).astype(np.int32)
        hist[:, 0] = -1  # out-of-range ids are skipped
        hist[:, 1] = hist[:, 2]  # repeated ids penalised once
        hist[:, 3], hist[:, 4], hist[:, 5] = V, V - 1, 32767  # past the vocabulary; the last id
        hlen = np.array([64 - 13 * (b % 5) for b in range(batch)], np.int32)
        out = hip.DeviceArray((batch,), np.int32)
        hip.sample(hip.DeviceArray.from_host(logits), V, cfg, out, batch=batch, hist=hip.DeviceArray.from_host(hist),
                   hist_len=hip.DeviceArray.from_host(hlen), hist_ld=64, rng=rng, ws=ws)
        got = out.numpy()
        want = [cpu[b].sample(logits[b], hist[b][:hlen[b]]) for b in range(batch)]
        assert [int(v) for v in got] == want, (step, cfg)


def test_sampler_reference_kats(hip):
    """tests/test_tokenizer.cpp:152-172 on the device."""
    def one(logits, cfg, hist=(), seed=0):
        logits = np.asarray(logits, np.float32)
        n = len(logits)
        h = np.asarray(list(hist) or [0], np.int32)
        out = hip.DeviceArray((1,), np.int32)
        rng = hip.RngStates([seed])
        hip.sample(hip.DeviceArray.from_host(logits), n, cfg, out, hist=hip.DeviceArray.from_host(h),
                   hist_len=hip.DeviceArray.from_host(np.array([len(hist)], np.int32)), hist_ld=len(h), rng=rng)
        return int(out.numpy()[0])

    l = [1.0, 3.0, 2.0, -1.0]
    assert one(l, {}) == 1
    assert one(l, dict(temperature=5.0, top_k=1)) == 1
    assert one(l, dict(temperature=1.0, top_p=1e-6)) == 1
    assert one(l, dict(repetition_penalty=2.0), hist=[1, 1]) == 2
    assert one([-1.0, -1.5], dict(repetition_penalty=2.0), hist=[0]) == 1


def test_sampler_seeded_distribution(hip):
    """0.7 / 0.2 / 0.1 within 0.02 over 20000 draws, and the GPU sequence equals the CPU one
    (tests/test_tokenizer.cpp:174-191)."""
    l = np.log(np.array([0.7, 0.2, 0.1], np.float32)).astype(np.float32)
    n = 4000
    cfg = dict(temperature=1.0, seed=42)
    rng = hip.RngStates([42])
    cpu = O.Sampler(temperature=1.0, seed=42)
    dl = hip.DeviceArray.from_host(l)
    out = hip.DeviceArray((1,), np.int32)
    counts = np.zeros(3)
    for i in range(n):
        hip.sample(dl, 3, cfg, out, rng=rng)
        t = int(out.numpy()[0])
        assert t == cpu.sample(l)
        counts[t] += 1
    assert np.all(np.abs(counts / n - [0.7, 0.2, 0.1]) < 0.03)


@pytest.mark.parametrize("layout", ["one_thread", "two_waves", "all_equal", "few_finite"])
@pytest.mark.parametrize("top_k", [1, 16, 40, 128, 129])
def test_sampler_topk_floor_layouts(hip, layout, top_k):
    """The radix select's key floor (each wave's m-th largest lane maximum, the smallest over the
    waves) on layouts that put the k largest logits in few lanes: the kept set, and so the ids,
    must still equal the reference's (src/sampler.cpp:26-43).  Thread t of the 1024-thread
    workgroup holds ids t + 1024 j."""
    V, batch = 32000, 4
    print(f"[case] sampler floor layout={layout} k={top_k}", flush=True)
    g = D.rng(7 + top_k)
    logits = (g.standard_normal((batch, V), dtype=np.float32)).astype(np.float32)
    if layout == "one_thread":  # the 31 largest in thread 5, the next in thread 900
        logits[:, 5::1024] += np.float32(20.0)
        logits[:, 900::1024] += np.float32(10.0)
    elif layout == "two_waves":  # every large logit in waves 3 and 11
        for w in (3, 11):
            for t in range(64 * w, 64 * w + 64):
                logits[:, t::1024] += np.float32(8.0)
    elif layout == "all_equal":  # ties everywhere: keys differ only by id
        logits[:] = np.float32(0.25)
    else:  # only 50 finite logits above -inf
        logits[:] = -np.inf
        idx = g.choice(V, size=50, replace=False)
        logits[:, idx] = g.standard_normal(50).astype(np.float32)
    cfg = dict(temperature=0.9, top_k=top_k, top_p=0.97, repetition_penalty=1.0)
    seeds = [11 + b for b in range(batch)]
    rng = hip.RngStates(seeds)
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    hist = np.zeros((batch, 1), np.int32)
    out = hip.DeviceArray((batch,), np.int32)
    for step in range(3):
        hip.sample(hip.DeviceArray.from_host(logits), V, cfg, out, batch=batch, hist=hip.DeviceArray.from_host(hist),
                   hist_len=hip.DeviceArray.from_host(np.zeros(batch, np.int32)), hist_ld=1, rng=rng)
        want = [cpu[b].sample(logits[b], []) for b in range(batch)]
        assert [int(v) for v in out.numpy()] == want, (layout, top_k, step)


@pytest.mark.parametrize("layout", ["peaked", "all_equal", "two_levels", "plus_inf", "minus_inf_tail", "tiny_tail"])
@pytest.mark.parametrize("top_p", [1.0, 0.9, 0.5, 1e-6])
def test_sampler_full_sort_sums(hip, layout, top_p):
    """Sampling without top-k (the sorted softmax, nucleus and CDF sums over every id): ids equal
    the reference's for distributions whose running sums cross many binades, stop at the first
    term, tie everywhere, or are NaN (+inf logits: the reference then takes the last sorted id)
    (src/sampler.cpp:42-69)."""
    V, batch = 32000, 4
    print(f"[case] sampler full-sort layout={layout} top_p={top_p}", flush=True)
    g = D.rng(900 + len(layout))
    logits = g.standard_normal((batch, V), dtype=np.float32)
    if layout == "peaked":  # one id carries almost all the mass: the cut and the draw stop at term 0
        logits[:, 77] = np.float32(40.0)
    elif layout == "all_equal":
        logits[:] = np.float32(-1.5)
    elif layout == "two_levels":
        logits[:] = np.float32(0.0)
        logits[:, ::3] = np.float32(2.0)
    elif layout == "plus_inf":
        logits[:, 5] = np.float32(np.inf)
    elif layout == "minus_inf_tail":
        logits[:, 1000:] = np.float32(-np.inf)
    else:  # terms down to the smallest doubles
        logits = (logits * np.float32(80.0)).astype(np.float32)
    cfg = dict(temperature=1.0, top_k=0, top_p=top_p, repetition_penalty=1.0)
    seeds = [31 + b for b in range(batch)]
    rng = hip.RngStates(seeds)
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    hist = np.zeros((batch, 1), np.int32)
    out = hip.DeviceArray((batch,), np.int32)
    for step in range(4):
        hip.sample(hip.DeviceArray.from_host(logits), V, cfg, out, batch=batch, hist=hip.DeviceArray.from_host(hist),
                   hist_len=hip.DeviceArray.from_host(np.zeros(batch, np.int32)), hist_ld=1, rng=rng)
        want = [cpu[b].sample(logits[b], []) for b in range(batch)]
        assert [int(v) for v in out.numpy()] == want, (layout, top_p, step)


@pytest.mark.parametrize("V,top_k,top_p", [(40000, 0, 0.9), (40000, 2000, 0.95), (50000, 30000, 1.0), (5000, 0, 0.9),
                                           (32768, 0, 0.8), (33, 0, 0.5)])
def test_sampler_other_vocab_sizes(hip, V, top_k, top_p):
    """Vocabularies other than TinyLlama's: above the 32768 ids the parallel sums take (the
    sequential fallback), top-k above the LDS path with a large vocabulary (the parallel sums over
    k ids), and small ones (src/sampler.cpp:13-70)."""
    batch = 3
    print(f"[case] sampler V={V} top_k={top_k} top_p={top_p}", flush=True)
    g = D.rng(V + top_k)
    cfg = dict(temperature=0.9, top_k=top_k, top_p=top_p, repetition_penalty=1.2)
    seeds = [5 + b for b in range(batch)]
    rng = hip.RngStates(seeds)
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    ws = hip.DeviceArray((EL.lib().ef_hip_sample_workspace_bytes(V, batch),), np.uint8)
    out = hip.DeviceArray((batch,), np.int32)
    for step in range(3):
        logits = (g.standard_normal((batch, V), dtype=np.float32) * np.float32(2.0 + step)).astype(np.float32)
        hist = g.integers(0, V, size=(batch, 16)).astype(np.int32)
        hip.sample(hip.DeviceArray.from_host(logits), V, cfg, out, batch=batch, hist=hip.DeviceArray.from_host(hist),
                   hist_len=hip.DeviceArray.from_host(np.full(batch, 16, np.int32)), hist_ld=16, rng=rng, ws=ws)
        want = [cpu[b].sample(logits[b], hist[b]) for b in range(batch)]
        assert [int(v) for v in out.numpy()] == want, (V, top_k, top_p, step)


HEAD = 4096  # the sorted head of the top-p-only path (nucleus_kernel)


def _nucleus_facts(logits, cfg, hist=()):
    """What decides the top-p-only path for one sequence, restated on the host in the reference's
    operations (src/sampler.cpp:16-61: penalty and temperature in float, descending sort with ties
    by id, exp(double(l - max)) from the host libm, left-to-right double sums): the number of kept
    ids, and how many binades the softmax sum enters after the head's 4096 terms."""
    lv = np.asarray(logits, np.float32).copy()
    V = lv.size
    pen = np.float32(cfg["repetition_penalty"])
    if pen != np.float32(1.0):
        for t in sorted({int(h) for h in hist if 0 <= h < V}):
            lv[t] = lv[t] / pen if lv[t] > 0 else lv[t] * pen
    lv = (lv / np.float32(cfg["temperature"])).astype(np.float32)
    order = np.lexsort((np.arange(V), -lv))
    ls = lv[order]
    t = O.exp_array((ls - ls[0]).astype(np.float32).astype(np.float64)).tolist()
    s, s_head = 0.0, None
    for i, v in enumerate(t):
        s += v
        if i == HEAD - 1:
            s_head = s
    cum, keep = 0.0, V
    for i, v in enumerate(t):
        cum += v / s
        if cum >= cfg["top_p"]:
            keep = i + 1
            break
    exits = int(np.floor(np.log2(s))) - int(np.floor(np.log2(s_head)))
    return keep, exits


def _designed_tail(g, V, c, decay, lo, hi):
    """Logits whose sorted softmax terms are 1, then c exp(-i / decay) for the other 4095 head ids,
    then V - 4096 tail terms uniform in [lo, hi) (below the head's last), ids shuffled."""
    i = np.arange(1, HEAD)
    head = c * np.exp(-i / decay)
    assert hi < head[-1]
    tail = g.uniform(lo, hi, V - HEAD)
    vals = np.concatenate([[1.0], head, tail])
    return np.log(vals).astype(np.float32)[g.permutation(V)]


def _check_against_oracle(H, logits, cfg, steps, seeds, hist=None):
    batch, V = logits.shape
    rng = H.RngStates(seeds)
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    if hist is None:
        hist = np.zeros((batch, 1), np.int32)
        hlen = np.zeros(batch, np.int32)
    else:
        hlen = np.full(batch, hist.shape[1], np.int32)
    ws = H.DeviceArray((EL.lib().ef_hip_sample_workspace_bytes(V, batch),), np.uint8)
    out = H.DeviceArray((batch,), np.int32)
    dl, dh, dn = H.DeviceArray.from_host(logits), H.DeviceArray.from_host(hist), H.DeviceArray.from_host(hlen)
    for step in range(steps):
        H.sample(dl, V, cfg, out, batch=batch, hist=dh, hist_len=dn, hist_ld=hist.shape[1], rng=rng, ws=ws)
        want = [cpu[b].sample(logits[b], hist[b][:hlen[b]]) for b in range(batch)]
        assert [int(v) for v in out.numpy()] == want, step


@pytest.mark.parametrize("layout", ["one_tail_exit", "two_tail_exits", "no_tail_exit", "crowded_bin"])
def test_sampler_nucleus_head_tail_exits(hip, layout):
    """Top-p without top-k from the sorted head of at most 4096 keys: the rest of the vocabulary
    joins the softmax sum unsorted, and when the sum enters a new binade after the head the next
    keys are sorted and added in order first (a second exit goes to the full sort); a crowded bin of
    equal logits takes the head's bitonic sort (src/sampler.cpp:36-48).  The logits are built so
    that the host restatement shows the intended number of exits and a nucleus inside the head;
    ids must equal the reference's over several draws."""
    V, batch = 32000, 6
    print(f"[case] sampler nucleus head layout={layout}", flush=True)
    g = D.rng(4100 + len(layout))
    if layout == "one_tail_exit":  # head sum about 14 in [8, 16), the tail takes it past 16
        rows = [_designed_tail(g, V, 0.0133, 1000.0, 1.0e-4, 2.2e-4) for _ in range(batch)]
        cfg, want_exits = dict(temperature=1.0, top_k=0, top_p=0.7, repetition_penalty=1.0), 1
    elif layout == "two_tail_exits":  # head sum about 6 in [4, 8), the tail takes it past 8 and 16
        rows = [_designed_tail(g, V, 0.00195, 4000.0, 3.0e-4, 7.0e-4) for _ in range(batch)]
        cfg, want_exits = dict(temperature=1.0, top_k=0, top_p=0.25, repetition_penalty=1.0), 2
    elif layout == "crowded_bin":  # 300 equal logits inside the nucleus: the head's bitonic sort
        rows = []
        for _ in range(batch):
            r = (g.standard_normal(V, dtype=np.float32) * np.float32(3.0)).astype(np.float32)
            r[g.choice(V, size=300, replace=False)] = np.sort(r)[-40]
            rows.append(r)
        cfg, want_exits = dict(temperature=0.8, top_k=0, top_p=0.95, repetition_penalty=1.0), 0
    else:  # peaked: the sum settles inside the head
        rows = [(g.standard_normal(V, dtype=np.float32) * np.float32(4.0)).astype(np.float32) for _ in range(batch)]
        cfg, want_exits = dict(temperature=0.8, top_k=0, top_p=0.95, repetition_penalty=1.0), 0
    logits = np.stack(rows)
    for b in range(batch):
        keep, exits = _nucleus_facts(logits[b], cfg)
        assert keep < HEAD and exits == want_exits, (b, keep, exits)
    _check_against_oracle(hip, logits, cfg, 4, [71 + b for b in range(batch)])


def test_sampler_nucleus_mixed_batch(hip):
    """One call whose sequences split between the head path and the full sort (flat rows whose
    nucleus reaches past 4096 ids, a row with a +inf logit, peaked rows), with penalties: every
    sequence's id equals its own reference Sampler's, call after call (src/sampler.cpp:13-70)."""
    V, batch = 32000, 8
    print("[case] sampler nucleus mixed batch", flush=True)
    g = D.rng(4242)
    scales = [3.0, 1.0, 4.0, 0.5, 3.0, 1.0, 2.5, 3.0]
    logits = np.stack([(g.standard_normal(V, dtype=np.float32) * np.float32(sc)).astype(np.float32)
                       for sc in scales])
    logits[6, 123] = np.float32(np.inf)
    hist = g.integers(0, V, size=(batch, 32)).astype(np.int32)
    cfg = dict(temperature=0.8, top_k=0, top_p=0.95, repetition_penalty=1.1)
    heads = []
    for b in range(batch):
        if b != 6:
            keep, _ = _nucleus_facts(logits[b], cfg, hist[b])
            heads.append(keep < HEAD)
    assert any(heads) and not all(heads), heads
    _check_against_oracle(hip, logits, cfg, 4, [300 + b for b in range(batch)], hist=hist)


def test_sampler_nucleus_bucket_edges(hip):
    """Logits that sit on the head's bucket edges: many ids exactly k / 4 below the maximum (the
    order-bit threshold of the head's last bucket must keep or drop each of them as the bucket
    formula does), values near +-3e38 whose distance to the maximum overflows to infinity, large
    offsets where the float spacing is coarse (many equal logits), and a maximum repeated.  Ids equal
    the reference's call after call (src/sampler.cpp:13-70)."""
    V, batch = 32000, 6
    print("[case] sampler nucleus bucket edges", flush=True)
    g = D.rng(4343)
    rows = []
    r = (g.standard_normal(V, dtype=np.float32) * np.float32(2.0)).astype(np.float32)
    r[:] = np.minimum(r, np.float32(9.0))
    ids = g.permutation(V)
    r[ids[0]] = np.float32(10.0)
    for k in range(1, 60):  # 60 ids at each quarter step below the maximum
        r[ids[k * 60:(k + 1) * 60]] = np.float32(10.0 - k / 4.0)
    rows.append(r)
    r = (g.standard_normal(V, dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    r[ids[:3000]] = np.float32(-3.0e38)
    r[ids[3000:3005]] = np.float32(3.0e38) - np.float32(2.0 ** 103) * np.arange(5, dtype=np.float32)
    rows.append(r)
    rows.append((np.float32(1.0e6) + g.standard_normal(V, dtype=np.float32) * np.float32(4.0)).astype(np.float32))
    r = (g.standard_normal(V, dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    r[ids[100:140]] = r.max()
    rows.append(r)
    r = (g.standard_normal(V, dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    r[ids[:5000]] = np.float32(-np.inf)
    rows.append(r)
    rows.append(np.float32(-1.0e6) + (g.standard_normal(V, dtype=np.float32) * np.float32(3.0)).astype(np.float32))
    logits = np.stack(rows).astype(np.float32)
    for temperature in (1.0, 0.8):  # at 0.8 the 3e38 logits overflow to +inf: the full sort's rule
        cfg = dict(temperature=temperature, top_k=0, top_p=0.9, repetition_penalty=1.0)
        if temperature == 1.0:
            print("[case]   nucleus sizes", [_nucleus_facts(logits[b], cfg)[0] for b in range(batch)], flush=True)
        _check_against_oracle(hip, logits, cfg, 3, [910 + b for b in range(batch)])


@pytest.mark.parametrize("top_k", [0, 40])
def test_sampler_long_history(hip, top_k):
    """Histories longer than a workgroup (2000 entries, hist_ld 2048, some past the vocabulary and
    many repeated): the penalty marks take several passes per thread; ids equal the reference's on
    the register path with and without top-k (src/sampler.cpp:16-24)."""
    V, batch, L = 32000, 4, 2048
    print(f"[case] sampler long history top_k={top_k}", flush=True)
    g = D.rng(5150 + top_k)
    logits = (g.standard_normal((batch, V), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    hist = g.integers(-10, V + 10, size=(batch, L)).astype(np.int32)
    hist[:, 1500:] = hist[:, :L - 1500]  # repeats
    hlen = np.array([2000, 1025, 1024, 1], np.int32)
    cfg = dict(temperature=0.8, top_k=top_k, top_p=0.95, repetition_penalty=1.3)
    seeds = [60 + b for b in range(batch)]
    rng = hip.RngStates(seeds)
    cpu = [O.Sampler(seed=s, **cfg) for s in seeds]
    ws = hip.DeviceArray((EL.lib().ef_hip_sample_workspace_bytes(V, batch),), np.uint8)
    out = hip.DeviceArray((batch,), np.int32)
    dl, dh, dn = hip.DeviceArray.from_host(logits), hip.DeviceArray.from_host(hist), hip.DeviceArray.from_host(hlen)
    for step in range(3):
        hip.sample(dl, V, cfg, out, batch=batch, hist=dh, hist_len=dn, hist_ld=L, rng=rng, ws=ws)
        want = [cpu[b].sample(logits[b], hist[b][:hlen[b]]) for b in range(batch)]
        assert [int(v) for v in out.numpy()] == want, step


def test_sampler_nucleus_bench_logits(hip):
    """The bench's top-p-only sampler input (seeded N(0, 3) logits, T 0.8, repetition penalty 1.1,
    64-token histories, B = 64): some rows' sums enter their last binade after the head.  Ids equal
    the reference's (src/sampler.cpp:13-70)."""
    V, batch = 32000, 64
    print("[case] sampler nucleus bench logits B=64", flush=True)
    g = np.random.default_rng(5)
    logits = (g.standard_normal((batch, V), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    hist = g.integers(0, V, size=(batch, 64)).astype(np.int32)
    cfg = dict(temperature=0.8, top_k=0, top_p=0.95, repetition_penalty=1.1)
    facts = [_nucleus_facts(logits[b], cfg, hist[b]) for b in range(batch)]
    assert all(k < HEAD for k, _ in facts) and any(e > 0 for _, e in facts)
    _check_against_oracle(hip, logits, cfg, 3, [7 + b for b in range(batch)], hist=hist)
