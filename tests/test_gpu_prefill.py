"""GPU parity of the batched prefill (ef_hip_engine_prefill): the prompt through every product once
for all positions (matrix-core GEMV over batch x positions rows), RoPE + cache writes, then causal
attention per (head, row).  The reference feeds the prompt one position at a time
(src/model.cpp:290, Transformer::forward); the gates are the engine's: logits within 1e-4 relative
of the CPU oracle's Transformer at the last prompt position and at every later decode position (so
the KV cache the prefill wrote is right), identical greedy tokens, prefill at a non-zero start
position, chunked prompts, and several sequences."""
import os

import numpy as np
import pytest

from edgeforge_amd.model import Config, DeviceModel, Engine
from oracle.model import OracleModel
from tests import _data as D

pytestmark = pytest.mark.gpu

SMALL = Config(D=256, F=512, H=4, KV=2, hd=64, V=512, L=3, max_pos=64)
ODD = Config(D=96, F=160, H=3, KV=1, hd=32, V=200, L=2, max_pos=32)  # vector-ALU GEMVs (cols % 256 != 0)


def _err(a, b):
    return float(np.abs(a - b).max() / max(1.0, np.abs(b).max()))


@pytest.fixture(params=["small", "odd"])
def model(request, hip):
    cfg = SMALL if request.param == "small" else ODD
    dm = DeviceModel.synthetic(cfg, seed=61, q8={(0, "wk"), (1, "w_down")})
    return cfg, dm, OracleModel(dm)


@pytest.mark.parametrize("start,n", [(0, 9), (3, 6), (0, 1)])
def test_prefill_logits_and_cache_match_serial(model, start, n):
    cfg, dm, om = model
    print(f"[case] prefill {cfg.D} start={start} n={n}", flush=True)
    ids = [int(v) for v in D.rng(7).integers(0, cfg.V, start + n + 4)]
    eng = Engine(dm, max_seq=len(ids))
    ot = om.transformer(len(ids), threads=2)
    for p in range(start):  # cached positions before the prefill
        eng.forward([ids[p]], p, compute_logits=False)
        ot.forward(ids[p], p, compute_logits=False)
    eng.prefill([ids[start:start + n]], start)
    want = None
    for p in range(start, start + n):
        want = ot.forward(ids[p], p, compute_logits=p == start + n - 1)
    assert _err(eng.logits()[0], want) < 1e-4
    assert np.abs(eng.hidden()[0] - ot.hidden()).max() < 1e-4
    for p in range(start + n, len(ids)):  # decode on the cache the prefill wrote
        eng.forward([ids[p]], p)
        assert _err(eng.logits()[0], ot.forward(ids[p], p)) < 1e-4, p
    ot.close()
    eng.close()


def test_chunked_prefill_and_batch(hip, monkeypatch):
    """Prompts longer than one launch's rows go in chunks; each sequence of a batch matches the
    oracle run alone."""
    monkeypatch.setenv("EF_HIP_PREFILL_ROWS", "10")  # 3 sequences -> chunks of 3 positions
    dm = DeviceModel.synthetic(SMALL, seed=62, q8={(2, "wv")})
    om = OracleModel(dm)
    prompts = [[int(v) for v in D.rng(20 + b).integers(0, SMALL.V, 11)] for b in range(3)]
    eng = Engine(dm, max_seq=11 + 8, batch=3)
    got, _, _ = eng.generate(prompts, 8)
    for b in range(3):
        want, _, _, _ = om.run_once(prompts[b], 8, threads=2)
        assert got[b].tolist() == want.tolist(), b
    eng.close()


def test_generate_batched_equals_serial_prefill(hip, monkeypatch):
    dm = DeviceModel.synthetic(SMALL, seed=63)
    prompt = [[int(v) for v in D.rng(30).integers(0, SMALL.V, 17)]]
    eng = Engine(dm, max_seq=17 + 12)
    fast, pre_fast, _ = eng.generate(prompt, 12)
    monkeypatch.setenv("EF_HIP_PREFILL", "serial")
    slow, pre_slow, _ = eng.generate(prompt, 12)
    assert fast.tolist() == slow.tolist()
    print(f"prefill of 17 positions: batched {pre_fast * 1e3:.2f} ms, serial {pre_slow * 1e3:.2f} ms", flush=True)
    eng.close()


TILE = Config(D=512, F=768, H=8, KV=1, hd=64, V=512, L=2, max_pos=512)  # 8 query heads per KV head
TILE4 = Config(D=256, F=512, H=4, KV=2, hd=64, V=512, L=2, max_pos=512)  # 2 per KV head


@pytest.mark.parametrize("cfg,B,rows", [(TILE, 1, 0), (TILE, 3, 0), (TILE4, 2, 0), (TILE, 1, 150)])
def test_tiled_prefill_attention_matches_rows_kernel_and_oracle(hip, monkeypatch, cfg, B, rows):
    """Prompts of 300 positions take the tiled prefill attention (16 rows of a sequence x one KV
    group per workgroup, two passes over 64-position chunks): the logits after the prefill and at
    later decode positions match the per-(head, row) kernel's within 1e-5 relative and the oracle's
    serial forward within 1e-4; several sequences per launch, a partial last row block, and a
    prompt in launches of 150 positions (the second starting at position 150)."""
    print(f"[case] tiled prefill D={cfg.D} H={cfg.H} KV={cfg.KV} B={B} rows={rows}", flush=True)
    if rows:
        monkeypatch.setenv("EF_HIP_PREFILL_ROWS", str(rows))
    dm = DeviceModel.synthetic(cfg, seed=71)
    n = 300
    prompts = D.rng(72 + B).integers(0, cfg.V, size=(B, n)).astype(np.int32)
    got = {}
    for kind in ("tiled", "rows"):
        monkeypatch.setenv("EF_HIP_PREFILL_ATTENTION", kind)
        eng = Engine(dm, max_seq=n + 4, batch=B)
        eng.prefill(prompts, 0)
        lg = [eng.logits().copy()]
        nxt = np.argmax(lg[0], axis=1).astype(np.int32)
        for k in range(3):
            eng.forward(nxt, n + k)
            lg.append(eng.logits().copy())
            nxt = np.argmax(lg[-1], axis=1).astype(np.int32)
        eng.close()
        got[kind] = lg
    for a, b in zip(got["tiled"], got["rows"]):
        assert _err(a, b) < 1e-5
    om = OracleModel(dm)
    ot = om.transformer(n + 4, threads=2)
    want = None
    for p in range(n):
        want = ot.forward(int(prompts[0][p]), p, compute_logits=p == n - 1)
    assert _err(got["tiled"][0][0], want) < 1e-4
    ot.close()
