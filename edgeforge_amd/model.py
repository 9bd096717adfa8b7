"""Synthetic TinyLlama-shaped models on the device and the decode engine over them.

The model mirrors the reference's quantized file layout (src/model.cpp:66-111): every layer
matrix Q4_0 except the TinyLlama policy's six Q8_0 overrides (src/quantizer.cpp:75-80), a Q8_0
lm_head, a BF16 embedding and F32 norms.  Weights are random-init N(0, 0.02) and norms
1 + 0.1 N(0, 1) (tools/make_synthetic_checkpoint.py:92-95), generated on the device and packed by
the device quantizer, which is byte-identical to the reference's quantize_row.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib as EL
from . import hip as H

LAYER_MATS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
# model.layers.{l}.self_attn.{k,v}_proj stored Q8_0 by the tinyllama-1.1b-chat-v1.0 policy
TINYLLAMA_Q8 = frozenset({(0, "wk"), (0, "wv"), (1, "wv"), (2, "wv"), (17, "wv"), (18, "wv")})


def _packed_row_bytes(qtype: int, cols: int) -> int:  # src/quant.cpp:136-149
    return cols // 32 * (34 if qtype == EL.Q8_0 else 18)


@dataclass
class Config:
    D: int = 2048
    F: int = 5632
    H: int = 32
    KV: int = 4
    hd: int = 64
    V: int = 32000
    L: int = 22
    max_pos: int = 2048
    eps: float = 1e-5
    rope_theta: float = 10000.0

    def shape(self, name: str) -> tuple[int, int]:
        kvd = self.KV * self.hd
        return {"wq": (self.D, self.D), "wk": (kvd, self.D), "wv": (kvd, self.D), "wo": (self.D, self.D),
                "w_gate": (self.F, self.D), "w_up": (self.F, self.D), "w_down": (self.D, self.F)}[name]

    def c_struct(self) -> EL.ef_hip_model_config:
        return EL.ef_hip_model_config(self.D, self.F, self.H, self.KV, self.hd, self.V, self.L, self.max_pos,
                                     self.eps, self.rope_theta)

    def weight_bytes_per_token(self, q8=TINYLLAMA_Q8, lm_type=EL.Q8_0) -> int:
        """Bytes streamed per decoded token: layer matrices + norms + lm_head (QuantFile::bytes_per_token)."""
        total = 0
        for l in range(self.L):
            for m in LAYER_MATS:
                r, c = self.shape(m)
                total += r * _packed_row_bytes(EL.Q8_0 if (l, m) in q8 else EL.Q4_0, c)
            total += 2 * self.D * 4
        total += self.D * 4 + self.V * _packed_row_bytes(lm_type, self.D)
        return total


TINYLLAMA = Config()


@dataclass
class DeviceModel:
    cfg: Config
    seed: int
    q8: frozenset = TINYLLAMA_Q8
    weights: dict = field(default_factory=dict)  # (layer, name) -> H.Weight ; ("embed"|"lm_head") -> H.Weight
    packed: dict = field(default_factory=dict)   # same keys -> DeviceArray of packed bytes
    norms: dict = field(default_factory=dict)    # (layer, "attn"|"ffn") | "final" -> DeviceArray

    @classmethod
    def synthetic(cls, cfg: Config, seed: int = 1234, q8=TINYLLAMA_Q8, layer_type: int = EL.Q4_0,
                  lm_type: int = EL.Q8_0, embed_type: int = EL.BF16, std: float = 0.02) -> "DeviceModel":
        H.init()
        m = cls(cfg, seed, frozenset(q8))
        biggest = max(cfg.V * cfg.D, cfg.F * cfg.D)
        scratch = H.DeviceArray((biggest,), np.float32)
        tid = 0

        def gen(n, mean, scale):
            nonlocal tid
            EL.call("ef_hip_fill_normal", scratch.ptr, n, seed, tid, mean, scale, None)
            tid += 1

        def pack(key, qtype, rows, cols):
            gen(rows * cols, 0.0, std)
            buf = H.quantize(qtype, scratch, rows, cols, search=True)
            m.packed[key] = buf
            m.weights[key] = H.Weight(qtype, rows, cols, device=buf)

        pack("embed", embed_type, cfg.V, cfg.D)
        for l in range(cfg.L):
            for name in LAYER_MATS:
                r, c = cfg.shape(name)
                pack((l, name), EL.Q8_0 if (l, name) in m.q8 else layer_type, r, c)
            for nn in ("attn", "ffn"):
                gen(cfg.D, 1.0, 0.1)
                d = H.DeviceArray((cfg.D,), np.float32)
                EL.call("ef_hip_memcpy_d2d", d.ptr, scratch.ptr, cfg.D * 4, None)
                m.norms[(l, nn)] = d
        gen(cfg.D, 1.0, 0.1)
        d = H.DeviceArray((cfg.D,), np.float32)
        EL.call("ef_hip_memcpy_d2d", d.ptr, scratch.ptr, cfg.D * 4, None)
        m.norms["final"] = d
        pack("lm_head", lm_type, cfg.V, cfg.D)
        H.sync()
        scratch.free()
        return m

    def host_bytes(self, key) -> np.ndarray:
        w = self.weights[key]
        return self.packed[key].numpy().reshape(w.rows, w.row_bytes)

    def host_norm(self, key) -> np.ndarray:
        return self.norms[key].numpy()


class Engine:
    """ef_hip_engine: Transformer::forward on the device for `batch` sequences."""

    def __init__(self, model, max_seq: int, batch: int = 1):
        """model: a DeviceModel, or a device model handle holder with .h (qfile.EfqModel)."""
        self.model, self.max_seq, self.batch = model, max_seq, batch
        cfg = model.cfg
        if not isinstance(model, DeviceModel):
            h = C.c_void_p()
            EL.call("ef_hip_model_engine_create", model.h, max_seq, batch, C.byref(h))
            self.h = h.value
            return
        layers = (EL.ef_hip_layer * cfg.L)()
        for l in range(cfg.L):
            layers[l] = EL.ef_hip_layer(*[model.weights[(l, n)].handle for n in LAYER_MATS],
                                       model.norms[(l, "attn")].ptr, model.norms[(l, "ffn")].ptr)
        self._cfg = cfg.c_struct()
        h = C.c_void_p()
        EL.call("ef_hip_engine_create", C.byref(self._cfg), layers, model.weights["embed"].handle,
               model.weights["lm_head"].handle, model.norms["final"].ptr, max_seq, batch, C.byref(h))
        self.h = h.value

    def forward(self, tokens, pos: int, compute_logits: bool = True) -> None:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(self.batch))
        EL.call("ef_hip_engine_forward", self.h, t.ctypes.data_as(EL._i32p), pos, int(compute_logits))

    def prefill(self, tokens, pos: int, compute_logits: bool = True) -> None:
        """tokens [batch][n] at positions pos .. pos+n-1, all rows at once (ef_hip_engine_prefill)."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(self.batch, -1))
        EL.call("ef_hip_engine_prefill", self.h, t.ctypes.data_as(EL._i32p), t.shape[1], pos, int(compute_logits))

    def _fetch(self, fn: str, n: int) -> np.ndarray:
        p = C.c_void_p()
        EL.call(fn, self.h, C.byref(p))
        out = np.empty((self.batch, n), np.float32)
        EL.call("ef_hip_memcpy_d2h", out.ctypes.data, p.value, out.nbytes, None)
        return out

    def logits(self) -> np.ndarray:
        return self._fetch("ef_hip_engine_logits", self.model.cfg.V)

    def hidden(self) -> np.ndarray:
        return self._fetch("ef_hip_engine_hidden", self.model.cfg.D)

    def generate(self, prompt, n: int, sampler: dict | None = None, rng: H.RngStates | None = None):
        """prompt [batch][n_prompt] -> (tokens [batch][n], prefill_s, decode_s)."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32).reshape(self.batch, -1))
        out = np.empty((self.batch, n), np.int32)
        pre, dec = C.c_double(), C.c_double()
        cfg = None
        if sampler is not None:
            cfg = EL.ef_hip_sampler_config(sampler.get("temperature", 0.0), sampler.get("top_k", 0),
                                          sampler.get("top_p", 1.0), sampler.get("repetition_penalty", 1.0),
                                          sampler.get("seed", 0))
        EL.call("ef_hip_engine_generate", self.h, p.ctypes.data_as(EL._i32p), p.shape[1], n,
               C.byref(cfg) if cfg is not None else None, rng.buf.ptr if rng else None,
               out.ctypes.data_as(EL._i32p), C.byref(pre), C.byref(dec))
        return out, pre.value, dec.value

    def reply(self, ids, max_new: int, sampler: dict | None = None, rng: H.RngStates | None = None,
              eos_id: int = -1, eos_min_p: float = 0.0, steps_per_check: int = 8):
        """ChatSession::reply at the token level (batch 1): (reply ids, P(EOS) per step, stats)."""
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32).reshape(-1))
        sampler = sampler or {}
        cfg = EL.ef_hip_sampler_config(sampler.get("temperature", 0.0), sampler.get("top_k", 0),
                                      sampler.get("top_p", 1.0), sampler.get("repetition_penalty", 1.0),
                                      sampler.get("seed", 0))
        opts = EL.ef_hip_reply_options(max_new, eos_id, eos_min_p, steps_per_check)
        out = np.empty(max_new, np.int32)
        peos = np.empty(max_new, np.float64)
        st = EL.ef_hip_reply_stats()
        EL.call("ef_hip_engine_reply", self.h, ids.ctypes.data_as(EL._i32p), ids.size, C.byref(cfg),
               rng.buf.ptr if rng else None, C.byref(opts), out.ctypes.data_as(EL._i32p),
               peos.ctypes.data_as(C.POINTER(C.c_double)), C.byref(st))
        return out[:st.generated].copy(), peos[:st.steps].copy(), st

    PROFILE_GROUPS = ("embed", "qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "pick")

    def staged_tables(self) -> tuple[bool, str]:
        """Whether several-sequence steps run over producer-staged product inputs, and why not
        (ef_hip_engine_tables)."""
        on, why = C.c_int(0), C.c_char_p()
        EL.call("ef_hip_engine_tables", self.h, C.byref(on), C.byref(why))
        return bool(on.value), (why.value or b"").decode()

    def profile(self, reps: int = 20, sampler: dict | None = None, rng: H.RngStates | None = None) -> dict:
        """Milliseconds per step of each kernel group of a decode step (ef_hip_engine_profile)."""
        out = (C.c_double * len(self.PROFILE_GROUPS))()
        cfg = None
        if sampler is not None:
            cfg = EL.ef_hip_sampler_config(sampler.get("temperature", 0.0), sampler.get("top_k", 0),
                                          sampler.get("top_p", 1.0), sampler.get("repetition_penalty", 1.0),
                                          sampler.get("seed", 0))
        EL.call("ef_hip_engine_profile", self.h, C.byref(cfg) if cfg is not None else None,
               rng.buf.ptr if rng else None, reps, out)
        return {g: float(out[i]) for i, g in enumerate(self.PROFILE_GROUPS)}

    def reset(self) -> None:
        EL.call("ef_hip_engine_reset", self.h)

    def score(self, ids, first: int = 0, logits: H.DeviceArray | None = None) -> np.ndarray:
        """Teacher-forced NLL of ids[p+1] at positions p in [first, n-1) (batch 1); logits, when given,
        receives those positions' logits [(n-1-first)][V] on the device."""
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32).reshape(-1))
        nll = np.empty(ids.size - 1 - first, np.float64)
        EL.call("ef_hip_engine_score", self.h, ids.ctypes.data_as(EL._i32p), ids.size, first,
               nll.ctypes.data_as(C.POINTER(C.c_double)), logits.ptr if logits is not None else None)
        return nll

    def close(self) -> None:
        if getattr(self, "h", None):
            EL.call("ef_hip_engine_destroy", self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
