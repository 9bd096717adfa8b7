"""The CPU oracle's transformer over the packed bytes of a device model (TEST INFRASTRUCTURE ONLY:
tests, smoke() and bench.py's cpu_baseline leg)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

import oracle as O
LAYER_MATS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


class OracleModel:
    """efo_model over host copies of a model's packed weights and norms (DeviceModel or HostModel)."""

    def __init__(self, dm):
        cfg = dm.cfg
        self.cfg = cfg
        self.keep = []
        layers = (O.efo_layer * cfg.L)()
        for l in range(cfg.L):
            ws = []
            for n in LAYER_MATS:
                b = dm.host_bytes((l, n))
                w = dm.weights[(l, n)]
                self.keep.append(b)
                ws.append(O.weight(w.qtype, b, w.rows, w.cols))
            an, fn = dm.host_norm((l, "attn")), dm.host_norm((l, "ffn"))
            self.keep += [an, fn]
            layers[l] = O.efo_layer(*ws, O.ptr(an, O._f32p), O.ptr(fn, O._f32p))
        eb, lb, fnorm = dm.host_bytes("embed"), dm.host_bytes("lm_head"), dm.host_norm("final")
        self.keep += [eb, lb, fnorm, layers]
        e, lm = dm.weights["embed"], dm.weights["lm_head"]
        c = O.efo_config(cfg.D, cfg.F, cfg.H, cfg.KV, cfg.hd, cfg.V, cfg.L, cfg.max_pos, cfg.eps, cfg.rope_theta)
        self.m = O.efo_model(c, O.weight(e.qtype, eb, e.rows, e.cols), O.weight(lm.qtype, lb, lm.rows, lm.cols),
                             O.ptr(fnorm, O._f32p), layers)

    def run_once(self, prompt, n: int, threads: int | None = None, backend: int = O.AVX2):
        """Reference decode protocol: (tokens [n], logits [n][V], prefill_s, decode_s)."""
        prompt = np.ascontiguousarray(np.asarray(prompt, np.int32))
        toks = np.empty(n, np.int32)
        logits = np.empty((n, self.cfg.V), np.float32)
        pre, dec = C.c_double(), C.c_double()
        pool = O.Pool(threads or cpu_threads())
        rc = O.lib().efo_run_once(C.byref(self.m), O.ptr(prompt, O._i32p), prompt.size, n, pool.h, backend,
                                  O.ptr(toks, O._i32p), O.ptr(logits, O._f32p), C.byref(pre), C.byref(dec))
        pool.close()
        assert rc == 0
        return toks, logits, pre.value, dec.value

    def transformer(self, max_seq: int, threads: int | None = None, backend: int = O.AVX2):
        return OracleTransformer(self, max_seq, threads or cpu_threads(), backend)


class OracleTransformer:
    def __init__(self, om: OracleModel, max_seq: int, threads: int, backend: int):
        self.om = om
        self.pool = O.Pool(threads)
        self.t = O.lib().efo_transformer_create(C.byref(om.m), max_seq, self.pool.h, backend)
        assert self.t

    def forward(self, token: int, pos: int, compute_logits: bool = True):
        err = C.c_int()
        p = O.lib().efo_transformer_forward(self.t, token, pos, int(compute_logits), C.byref(err))
        if err.value:
            raise ValueError("forward rejected the token or position")
        if not compute_logits:
            return None
        return np.ctypeslib.as_array(p, shape=(self.om.cfg.V,)).copy()

    def hidden(self) -> np.ndarray:
        p = O.lib().efo_transformer_hidden(self.t)
        return np.ctypeslib.as_array(p, shape=(self.om.cfg.D,)).copy()

    def close(self):
        if self.t:
            O.lib().efo_transformer_destroy(self.t)
            self.t = None
        self.pool.close()


class _W:
    def __init__(self, qtype, rows, cols):
        self.qtype, self.rows, self.cols = qtype, rows, cols


class HostModel:
    """A synthetic model built on the host with the oracle's quantizer (CPU-only tests): the same
    accessors as edgeforge_amd.model.DeviceModel (weights[key] -> qtype/rows/cols, host_bytes,
    host_norm).  Weights N(0, std), norms 1 + 0.1 N(0, 1), from numpy's PCG64 with `seed`."""

    def __init__(self, cfg, seed: int, q8=(), std: float = 0.02, layer_type: int = O.Q4_0,
                 lm_type: int = O.Q8_0, embed_type: int = O.BF16, keep_floats: bool = False):
        g = np.random.default_rng(seed)
        self.cfg = cfg
        self.weights, self._bytes, self._norms, self._floats = {}, {}, {}, {}

        def pack(key, qt, rows, cols):
            w = (g.standard_normal((rows, cols), dtype=np.float32) * np.float32(std)).astype(np.float32)
            if keep_floats:
                self._floats[key] = w
            self._bytes[key] = O.quantize(qt, w)
            self.weights[key] = _W(qt, rows, cols)

        pack("embed", embed_type, cfg.V, cfg.D)
        for l in range(cfg.L):
            for n in LAYER_MATS:
                rows, cols = cfg.shape(n)
                pack((l, n), O.Q8_0 if (l, n) in set(q8) else layer_type, rows, cols)
            for nn in ("attn", "ffn"):
                self._norms[(l, nn)] = (1.0 + 0.1 * g.standard_normal(cfg.D)).astype(np.float32)
        self._norms["final"] = (1.0 + 0.1 * g.standard_normal(cfg.D)).astype(np.float32)
        pack("lm_head", lm_type, cfg.V, cfg.D)

    def host_bytes(self, key):
        return self._bytes[key]

    def host_norm(self, key):
        return self._norms[key]

    def efq_tensors(self):
        t = {k: (self.weights[k].qtype, self._bytes[k]) for k in self._bytes}
        t.update(self._norms)
        return t


def prob_of(logits: np.ndarray, token: int) -> float:
    """P(token) under softmax(logits) in double, summed left to right (src/chat.cpp:35-42)."""
    import math
    if token < 0 or token >= logits.size:
        return 0.0
    l64 = logits.astype(np.float64)
    m = -math.inf
    for v in l64:
        m = max(m, float(v))
    s = 0.0
    for v in l64:
        s += math.exp(float(v) - m)
    return math.exp(float(l64[token]) - m) / s


STOP_EOS, STOP_EOS_MIN_P, STOP_MAX_NEW, STOP_CONTEXT = 1, 2, 5, 6


class OracleChat:
    """ChatSession::reply at the token level (src/chat.cpp:174-259) over the oracle's Transformer and
    Sampler, TEST INFRASTRUCTURE ONLY: cached-prefix reuse (at least the last id recomputed),
    prob_of(EOS) every step, and the EOS / EOS-probability / max-new / context stops in the
    reference's order.  The Sampler (and its RNG) lives across turns, as ChatSession's does."""

    def __init__(self, om: OracleModel, max_seq: int, sampler: dict, threads: int = 2):
        self.t = om.transformer(max_seq, threads=threads)
        self.s = O.Sampler(**sampler)
        self.cached: list[int] = []
        self.max_seq = max_seq

    def reply(self, ids, max_new: int, eos_id: int = -1, eos_min_p: float = 0.0):
        ids = [int(v) for v in ids]
        lcp = 0
        while lcp < len(self.cached) and lcp < len(ids) and self.cached[lcp] == ids[lcp]:
            lcp += 1
        if lcp == len(ids):
            lcp -= 1
        logits = None
        for p in range(lcp, len(ids)):
            logits = self.t.forward(ids[p], p, p + 1 == len(ids))
        self.cached = list(ids)
        limit = min(max_new, self.max_seq - len(ids))
        history, gen, peos, reason = list(ids), [], [], 0
        min_p = float(np.float32(eos_min_p))
        for step in range(limit):
            tok = self.s.sample(logits, history)
            pe = prob_of(logits, eos_id)
            peos.append(pe)
            if tok == eos_id:
                reason = STOP_EOS
                break
            if min_p > 0.0 and pe >= min_p:
                reason = STOP_EOS_MIN_P
                break
            gen.append(tok)
            history.append(tok)
            if step + 1 == limit:
                reason = STOP_CONTEXT if limit < max_new else STOP_MAX_NEW
                break
            logits = self.t.forward(tok, len(self.cached))
            self.cached.append(tok)
        return gen, peos, reason, lcp

    def close(self):
        self.t.close()
