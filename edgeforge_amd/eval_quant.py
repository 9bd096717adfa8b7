"""eval-quant on the GPU: how far a quantized model's next-token distributions are from a reference
model's (src/eval_quant.cpp:180-471, text perplexity and the verdict).

Both models run on the device engine; every chunk is scored teacher-forced in batched prefills
with the logits of every position (ef_hip_engine_score), and the distributions are compared on the
device (ef_hip_compare_dist: KL(P_ref || P_quantized) in double, top-1 agreement, confident
reference).  The reference model is whatever the caller loads: a lossless BF16 .efq file stands in
for the reference's BF16 safetensors checkpoint.  Targets are the reference's, fixed in
src/eval_quant.cpp:31-35.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from . import _lib as EL
from . import hip as H
from .model import Engine

TARGET_MEAN_KL = 0.10          # nats per position
CONFIDENT_P = 0.5              # the reference puts >= 50% on its top-1 token ...
TARGET_CONFIDENT_TOP1 = 0.95   # ... and the quantized model agrees there at least 95% of the time
TARGET_PPL_RATIO = 1.15        # perplexity(quantized) / perplexity(reference)


@dataclass
class EvalQuantReport:
    """The text part of ef::EvalQuantReport (include/ef/eval_quant.h:23-39)."""
    passed: int = 0
    failed: int = 0
    failed_checks: list = field(default_factory=list)
    positions: int = 0
    top1: int = 0
    confident: int = 0
    confident_top1: int = 0
    nonfinite: int = 0
    kl_mean: float = 0.0
    kl_max: float = 0.0
    ppl_ref: float = 0.0
    ppl_q: float = 0.0
    worst_chunk_ratio: float = 0.0
    n_scored: int = 0

    def check(self, ok: bool, what: str) -> None:
        if ok:
            self.passed += 1
        else:
            self.failed += 1
            self.failed_checks.append(what)


def text_chunks(text_ids, window: int = 0, max_chunks: int = 0, max_text_tokens: int = 128, bos_id: int = -1):
    """(ids, first scored position) per chunk (src/eval_quant.cpp:305-331): window 0 is one window
    from the start with every prediction scored; otherwise the llama-perplexity scheme, chunks of
    `window` tokens, the first token replaced by BOS, the second half scored."""
    ids = [int(t) for t in text_ids]
    if window == 0:
        ids = ids[:max_text_tokens]
        return [(ids, 0)] if len(ids) >= 2 else []
    if window < 4:
        raise ValueError("--window must be at least 4 tokens")
    n = len(ids) // window
    if max_chunks > 0:
        n = min(n, max_chunks)
    out = []
    for ci in range(n):
        ch = ids[ci * window:(ci + 1) * window]
        if bos_id >= 0:
            ch[0] = bos_id
        out.append((ch, window // 2))
    return out


def compare_dist(ref: H.DeviceArray, ours: H.DeviceArray, V: int, n: int):
    """Per-position KL and the DistAgg totals of n positions of [n][V] device logits."""
    kl = np.empty(n, np.float64)
    agg = EL.ef_hip_dist_stats()
    EL.call("ef_hip_compare_dist", ref.ptr, ours.ptr, V, n, V, V, kl.ctypes.data_as(C.POINTER(C.c_double)),
            C.byref(agg), None)
    return kl, agg


def run_text_eval(q_model, ref_model, text_ids, window: int = 0, max_chunks: int = 0, max_text_tokens: int = 128,
                  bos_id: int = -1) -> EvalQuantReport:
    """Text perplexity of both models, the per-position comparison, and the verdict checks."""
    R = EvalQuantReport()
    chunks = text_chunks(text_ids, window, max_chunks, max_text_tokens, bos_id)
    if not chunks:
        return R
    V = q_model.cfg.V
    max_len = max(len(c) for c, _ in chunks)
    qe, re_ = Engine(q_model, max_seq=max_len), Engine(ref_model, max_seq=max_len)
    qlog = H.DeviceArray((max_len, V))
    rlog = H.DeviceArray((max_len, V))
    nll_q = nll_r = 0.0
    tot = dict(n=0, top1=0, confident=0, confident_top1=0, nonfinite=0, kl_sum=0.0, kl_max=0.0)
    for ids, first in chunks:
        S = len(ids) - 1 - first
        cq = cr = 0.0
        for v in qe.score(ids, first, logits=qlog):  # left to right, as the reference accumulates
            cq += float(v)
        for v in re_.score(ids, first, logits=rlog):
            cr += float(v)
        nll_q += cq
        nll_r += cr
        R.n_scored += S
        R.worst_chunk_ratio = max(R.worst_chunk_ratio, math.exp((cq - cr) / S))
        _, agg = compare_dist(rlog, qlog, V, S)
        for k in ("n", "top1", "confident", "confident_top1", "nonfinite"):
            tot[k] += getattr(agg, k)
        tot["kl_sum"] += agg.kl_sum
        tot["kl_max"] = max(tot["kl_max"], agg.kl_max)
    qe.close()
    re_.close()
    R.ppl_q = math.exp(nll_q / R.n_scored)
    R.ppl_ref = math.exp(nll_r / R.n_scored)
    R.positions, R.top1, R.confident = tot["n"], tot["top1"], tot["confident"]
    R.confident_top1, R.nonfinite, R.kl_max = tot["confident_top1"], tot["nonfinite"], tot["kl_max"]
    R.kl_mean = tot["kl_sum"] / (tot["n"] - tot["nonfinite"]) if tot["n"] > tot["nonfinite"] else 0.0
    # verdict (src/eval_quant.cpp:437-462)
    R.check(R.nonfinite == 0, f"no NaN/Inf logits ({R.positions} positions)")
    R.check(R.kl_mean <= TARGET_MEAN_KL, f"mean KL(reference || quantized) {R.kl_mean:.4f} <= {TARGET_MEAN_KL}")
    conf = R.confident_top1 / R.confident if R.confident else 1.0
    R.check(conf >= TARGET_CONFIDENT_TOP1, f"confident top-1 agreement {conf:.3f} >= {TARGET_CONFIDENT_TOP1}")
    R.check(R.ppl_q / R.ppl_ref <= TARGET_PPL_RATIO, f"perplexity ratio {R.ppl_q / R.ppl_ref:.4f} <= {TARGET_PPL_RATIO}")
    return R
