"""Writer of the reference's .efq container (include/ef/qfile.h:1-21), TEST INFRASTRUCTURE ONLY.

Lets the reference's own engine (oracle/_ref: Model::load_efq + Transformer) run on the exact
packed bytes the tests and the device use.  Layout: "EFQ1", u32 version 1, u64 header length,
space-padded JSON header, then every tensor 64-byte aligned in forward order (embed, layers,
norm, lm_head).  The header carries the quantization policy so the reader's per-tensor type check
(src/qfile.cpp:208-221) accepts the file.
"""
from __future__ import annotations

import json
import struct

import numpy as np

TYPE_NAMES = {0: "F32", 1: "F16", 2: "BF16", 3: "Q8_0", 4: "Q4_0"}
MATS = [("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"), ("wv", "self_attn.v_proj"),
        ("wo", "self_attn.o_proj"), ("w_gate", "mlp.gate_proj"), ("w_up", "mlp.up_proj"), ("w_down", "mlp.down_proj")]


def _glob(p: str, s: str) -> bool:
    """'*' matches any run of characters (include/ef/qfile.h:45-47), by recursion on the pattern."""
    if not p:
        return not s
    if p[0] == "*":
        return any(_glob(p[1:], s[i:]) for i in range(len(s) + 1))
    return bool(s) and s[0] == p[0] and _glob(p[1:], s[1:])


def _rule(name: str, cols: int, layer_type: int, lm_type: int, embed_type: int, overrides) -> tuple:
    """(type, rule) the reader re-derives for a tensor (src/qfile.cpp:66-78)."""
    if "norm" in name:
        return 0, "norm"
    t, r = layer_type, "layers"
    if name == "model.embed_tokens.weight":
        t, r = embed_type, "embed"
    if name == "lm_head.weight":
        t, r = lm_type, "lm_head"
    for pat, ot in overrides:
        if _glob(pat, name):
            t, r = ot, "override"
    if t in (3, 4) and cols % 32:
        t, r = 2, "fallback-bf16"
    return t, r


def write_efq(path: str, cfg, tensors: dict, layer_type: int = 4, lm_type: int = 3, embed_type: int = 2,
              overrides=None, policy: str = "custom", tied: bool = False, extra_config: dict | None = None) -> None:
    """tensors: 'embed', 'lm_head' -> (qtype, bytes[rows, row_bytes]); (l, mat) -> same;
    (l, 'attn') / (l, 'ffn') / 'final' -> float32 [D].  cfg: D, F, H, KV, hd, V, L, max_pos, eps, rope_theta.
    overrides: [(pattern, qtype)] written into the policy (None: one exact-name override per layer
    matrix whose type differs from layer_type).  tied: no lm_head tensor, tie_word_embeddings true."""
    order = [("model.embed_tokens.weight", "embed", [cfg.V, cfg.D])]
    auto = overrides is None
    overrides = [] if auto else list(overrides)
    for l in range(cfg.L):
        p = f"model.layers.{l}."
        for key, nm in MATS:
            rows, cols = {"wq": (cfg.D, cfg.D), "wk": (cfg.KV * cfg.hd, cfg.D), "wv": (cfg.KV * cfg.hd, cfg.D),
                          "wo": (cfg.D, cfg.D), "w_gate": (cfg.F, cfg.D), "w_up": (cfg.F, cfg.D),
                          "w_down": (cfg.D, cfg.F)}[key]
            name = p + nm + ".weight"
            order.append((name, (l, key), [rows, cols]))
            if auto and tensors[(l, key)][0] != layer_type:
                overrides.append((name, tensors[(l, key)][0]))
        order.append((p + "input_layernorm.weight", (l, "attn"), [cfg.D]))
        order.append((p + "post_attention_layernorm.weight", (l, "ffn"), [cfg.D]))
    order.append(("model.norm.weight", "final", [cfg.D]))
    if not tied:
        order.append(("lm_head.weight", "lm_head", [cfg.V, cfg.D]))

    blobs, entries = [], []
    for name, key, shape in order:
        v = tensors[key]
        if isinstance(v, tuple):
            qt, data = v
        else:
            qt, data = 0, np.ascontiguousarray(v, np.float32)
        _, rule = _rule(name, shape[-1], layer_type, lm_type, embed_type, overrides)
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes()
        blobs.append(raw)
        entries.append({"name": name, "type": TYPE_NAMES[qt], "rule": rule, "shape": shape, "bytes": len(raw)})
    config = {"model_type": "llama", "architectures": ["LlamaForCausalLM"], "hidden_act": "silu",
              "hidden_size": cfg.D, "intermediate_size": cfg.F, "num_hidden_layers": cfg.L,
              "num_attention_heads": cfg.H, "num_key_value_heads": cfg.KV, "vocab_size": cfg.V,
              "max_position_embeddings": cfg.max_pos, "rms_norm_eps": float(cfg.eps),
              "rope_theta": float(cfg.rope_theta), "tie_word_embeddings": bool(tied), "head_dim": cfg.hd}
    config.update(extra_config or {})
    quant = {"layers": TYPE_NAMES[layer_type], "lm_head": TYPE_NAMES[lm_type], "embed": TYPE_NAMES[embed_type],
             "norms": "F32", "block": 32, "scale": "F16", "policy": policy,
             "overrides": [{"pattern": p_, "type": TYPE_NAMES[t_]} for p_, t_ in overrides]}

    def header(offsets):
        for e, off in zip(entries, offsets):
            e["offset"] = off
        return json.dumps({"format": "edgeforge-quant", "version": 1, "quant": quant, "source": {},
                           "config": config, "tensors": entries}, separators=(",", ":"))

    # fixed point: header length depends on the offsets, which depend on the header length
    hlen = len(header([0] * len(entries))) + 64
    for _ in range(8):
        start = 16 + hlen
        start += (-start) % 64
        offs, cur = [], start
        for b in blobs:
            offs.append(cur)
            cur += len(b)
            cur += (-cur) % 64
        text = header(offs)
        if 16 + len(text) <= start:
            break
        hlen = len(text) + 64
    text = text + " " * (start - 16 - len(text))
    with open(path, "wb") as f:
        f.write(b"EFQ1" + struct.pack("<I", 1) + struct.pack("<Q", len(text)) + text.encode())
        for off, b in zip(offs, blobs):
            f.seek(off)
            f.write(b)
