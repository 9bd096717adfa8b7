"""The .efq reader of the HIP library (host code: no GPU needed) against the reference reader.

Follows the reference's own tests of the format (tests/test_quant.cpp:197-233 corruption,
:295-341 overrides) and pins every decision on the reference build (oracle/_ref: parse_efq and
Model::load_efq compiled from src/qfile.cpp, src/model.cpp): the same files are accepted or
rejected, with the same message, including a few hundred single-byte corruptions of a valid
header.  Files are written by oracle/efq.py from oracle-quantized weights.
"""
import ctypes as C
import os
import tempfile

import numpy as np
import pytest

import oracle as O
from edgeforge_amd import _lib as EL
from edgeforge_amd.model import Config
from edgeforge_amd.qfile import QuantFile
from oracle.efq import write_efq
from oracle.model import HostModel

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not present")

TINY32 = Config(D=32, F=64, H=4, KV=2, hd=8, V=40, L=2, max_pos=64)  # tests/test_qinfer.cpp:269-278
NAMES = ["model.embed_tokens.weight"] + [
    f"model.layers.{l}.{n}" for l in range(2) for n in (
        "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
        "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight", "input_layernorm.weight",
        "post_attention_layernorm.weight")] + ["model.norm.weight", "lm_head.weight"]


def ours(buf: bytes):
    """(tensor count, None) or (None, message) from the HIP library's parse_efq."""
    b = C.create_string_buffer(bytes(buf), len(buf))
    h = C.c_void_p()
    rc = EL.lib().ef_hip_efq_parse(b, len(buf), C.byref(h))
    if rc != 0:
        return None, EL.lib().ef_hip_last_error().decode()
    n = C.c_size_t()
    EL.call("ef_hip_efq_tensor_count", h, C.byref(n))
    EL.call("ef_hip_efq_close", h)
    return n.value, None


def theirs(buf: bytes):
    err = C.create_string_buffer(1024)
    n = O.ref().ref_efq_parse(bytes(buf), len(buf), err, 1024)
    return (n, None) if n >= 0 else (None, err.value.decode())


def written(tmp, name="m.efq", seed=23, q8=(), **kw):
    hm = HostModel(TINY32, seed=seed, q8=q8, layer_type=kw.pop("layer_type", O.Q4_0),
                   lm_type=kw.pop("lm_type", O.Q8_0))
    path = os.path.join(tmp, name)
    write_efq(path, TINY32, hm.efq_tensors(), **kw)
    return hm, path, open(path, "rb").read()


def test_reader_indexes_a_written_file():
    with tempfile.TemporaryDirectory() as d:
        hm, path, good = written(d, q8={(1, "w_down"), (0, "wv")})
        f = QuantFile.open(path)
        ts = f.tensors()
        assert [t.name for t in ts] == NAMES  # forward order
        assert all(t.offset % 64 == 0 for t in ts)
        cfg = f.config()
        assert (cfg["D"], cfg["F"], cfg["H"], cfg["KV"], cfg["hd"], cfg["V"], cfg["L"]) == (32, 64, 4, 2, 8, 40, 2)
        assert not cfg["tie_word_embeddings"]
        assert f.at("model.layers.1.mlp.down_proj.weight").type == O.Q8_0
        assert f.at("model.layers.1.mlp.down_proj.weight").rule == "override"
        assert f.at("model.layers.1.self_attn.k_proj.weight").rule == "layers"
        assert f.at("lm_head.weight").rule == "lm_head" and f.at("model.norm.weight").rule == "norm"
        assert f.at("model.embed_tokens.weight").type == O.BF16
        assert f.find("model.layers.2.mlp.up_proj.weight") is None
        with pytest.raises(EL.HipError, match="not found"):
            f.at("model.layers.2.mlp.up_proj.weight")
        assert np.array_equal(f.data(f.at("model.layers.0.self_attn.v_proj.weight")),
                              hm.host_bytes((0, "wv")).reshape(-1))
        assert np.array_equal(f.data(f.at("model.norm.weight")).view(np.float32), hm.host_norm("final"))
        want = sum(t.bytes for t in ts if t.name != "model.embed_tokens.weight")
        assert f.bytes_per_token() == want
        pol = f.policy()
        assert (pol["layers"], pol["lm_head"], pol["embed"], pol["n_overrides"], pol["name"]) == \
            (O.Q4_0, O.Q8_0, O.BF16, 2, "custom")
        f.close()
        if O.ref_available():
            bpt, desc = C.c_uint64(), C.create_string_buffer(512)
            assert O.ref().ref_model_load_efq(path.encode(), C.byref(bpt), desc, 512) == 0
            assert bpt.value == want
            assert desc.value.decode() == "efq, policy custom: 12 Q4_0 + 3 Q8_0 matrices, embedding BF16"


def test_reader_rejects_corruption():
    """tests/test_quant.cpp:207-233, message for message."""
    with tempfile.TemporaryDirectory() as d:
        _, path, good = written(d)
        assert ours(good) == (21, None)
        bad = bytearray(good)
        bad[0] = ord("X")
        assert "bad magic" in ours(bad)[1]
        bad = bytearray(good)
        bad[4] = 2
        assert "unsupported .efq version 2" in ours(bad)[1]
        assert "past the end" in ours(good[:-1])[1]
        assert "too small" in ours(good[:10])[1]
        text = good[16:16 + 4096].decode("latin-1")
        pos = text.find('"offset":') + 9
        bad = bytearray(good)
        bad[16 + pos] = ord("8") if bad[16 + pos] == ord("9") else bad[16 + pos] + 1
        assert "64-byte aligned" in ours(bad)[1]
        bpos = text.find('"bytes":', text.find('"tensors"')) + 8
        bad = bytearray(good)
        bad[16 + bpos] = ord("8") if bad[16 + bpos] == ord("9") else bad[16 + bpos] + 1
        assert "header says" in ours(bad)[1]
        with pytest.raises(EL.HipError, match="cannot open"):
            QuantFile.open(os.path.join(d, "missing.efq"))


def _swap(buf: bytes, old: str, new: str) -> bytes:
    """Same-length text edit inside the header."""
    assert len(old) == len(new)
    i = buf.find(old.encode())
    assert i > 0, old
    return buf[:i] + new.encode() + buf[i + len(old):]


def test_policy_overrides_are_enforced():
    """tests/test_quant.cpp:295-341: every stored type must follow from the header's policy."""
    with tempfile.TemporaryDirectory() as d:
        _, _, good = written(d, q8={(0, "wk"), (0, "wv")})
        assert ours(good)[0] == 21
        key = '"pattern":"model.layers.0.self_attn.k_proj.weight","type":"Q8_0"'
        bad = _swap(good, key, key.replace("Q8_0", "Q4_0"))
        assert "policy gives Q4_0" in ours(bad)[1]
        bad = _swap(good, '"overrides":', '"overridez":')
        assert "re-run edgeforge quantize" in ours(bad)[1]


@pytest.mark.parametrize("patterns,msg", [
    ([("model.layers.*.mlp.down_proj.weight", O.Q8_0)], None),           # glob override, accepted
    ([("model.layers.1.*_proj.weight", O.Q8_0)], None),
    ([("model.layers.9.self_attn.v_proj.weight", O.Q8_0)], "matches no tensor"),
    ([("model.norm.weight", O.Q8_0)], "norms are always F32"),
    ([("", O.Q8_0)], "empty tensor pattern"),
])
def test_glob_overrides(patterns, msg):
    with tempfile.TemporaryDirectory() as d:
        hm = HostModel(TINY32, seed=31)
        t = hm.efq_tensors()
        for (l, n) in [(l, n) for l in range(2) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")]:
            name = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj",
                    "wo": "self_attn.o_proj", "w_gate": "mlp.gate_proj", "w_up": "mlp.up_proj",
                    "w_down": "mlp.down_proj"}[n]
            full = f"model.layers.{l}.{name}.weight"
            from oracle.efq import _glob
            if any(_glob(p, full) for p, _ in patterns if p):
                w = np.frombuffer(O.dequantize(O.Q4_0, t[(l, n)][1], hm.weights[(l, n)].cols).tobytes(), np.float32)
                w = w.reshape(hm.weights[(l, n)].rows, -1)
                t[(l, n)] = (O.Q8_0, O.quantize(O.Q8_0, w))
        path = os.path.join(d, "g.efq")
        write_efq(path, TINY32, t, overrides=patterns)
        buf = open(path, "rb").read()
        got = ours(buf)
        if msg is None:
            assert got == (21, None)
            f = QuantFile.open(path)
            ov = [x for x in f.tensors() if x.rule == "override"]
            assert ov and all(x.type == O.Q8_0 for x in ov)
        else:
            assert got[0] is None and msg in got[1]
        if O.ref_available():
            assert theirs(buf) == got


def test_tied_embeddings_and_bf16_fallback():
    """Tied: no lm_head tensor, the embedding counts per token (src/qfile.cpp:238-239).  Rows not a
    multiple of 32 fall back to BF16 (tests/test_quant.cpp:197-205)."""
    with tempfile.TemporaryDirectory() as d:
        hm = HostModel(TINY32, seed=41)
        path = os.path.join(d, "tied.efq")
        write_efq(path, TINY32, hm.efq_tensors(), tied=True)
        f = QuantFile.open(path)
        assert f.config()["tie_word_embeddings"] and f.find("lm_head.weight") is None
        emb = f.at("model.embed_tokens.weight").bytes
        assert f.bytes_per_token() == sum(t.bytes for t in f.tensors()) - emb + emb
        odd = Config(D=16, F=48, H=2, KV=1, hd=8, V=24, L=1, max_pos=16)
        hm2 = HostModel(odd, seed=42, layer_type=O.BF16, lm_type=O.BF16)
        p2 = os.path.join(d, "odd.efq")
        write_efq(p2, odd, hm2.efq_tensors(), overrides=[])
        g = QuantFile.open(p2)
        q = g.at("model.layers.0.self_attn.q_proj.weight")
        assert q.type == O.BF16 and q.rule == "fallback-bf16"
        if O.ref_available():
            for p in (path, p2):
                buf = open(p, "rb").read()
                assert theirs(buf) == ours(buf)


@pytest.mark.parametrize("edit", [
    ('"hidden_act":"silu"', '"hidden_act":"gelu"'),
    ('"model_type":"llama"', '"model_type":"llamb"'),
    ('"num_key_value_heads":2', '"num_key_value_heads":3'),
    ('"tie_word_embeddings":false', '"tie_word_embeddings":0.000'),
    ('"format":"edgeforge-quant"', '"format":"edgeforge-quanx"'),
    ('"norms":"F32"', '"norms":"F16"'),
    ('"layers":"Q4_0"', '"layers":"Q5_0"'),
    ('"hidden_size":32', '"hidden_size":3.'),    # invalid number
    ('"hidden_size":32', '"hidden_size":1e'),    # invalid exponent
    ('"hidden_size":32,', '"hidden_size":32,,'), # syntax
    ('"rms_norm_eps":', '"rms_norm_eps" '),
])
def test_header_edits_match_the_reference(edit):
    with tempfile.TemporaryDirectory() as d:
        _, _, good = written(d)
        old, new = edit
        if len(new) > len(old):  # keep the padded header length: eat a padding space
            i = good.find(old.encode())
            pad = good.rfind(b" ", 0, 16 + int.from_bytes(good[8:16], "little"))
            bad = good[:i] + new.encode() + good[i + len(old):pad] + good[pad + 1:]
        else:
            bad = _swap(good, old, new)
        got = ours(bad)
        assert got[0] is None, edit
        if O.ref_available():
            want = theirs(bad)
            assert want[0] is None
            if not want[1].startswith("invalid .efq header"):
                assert got[1] == want[1]


@needs_ref
def test_single_byte_corruptions_agree_with_the_reference():
    """300 seeded single-byte edits of the header (printable ASCII): accept / reject and message agree."""
    with tempfile.TemporaryDirectory() as d:
        _, _, good = written(d, q8={(1, "w_down")})
        hlen = int.from_bytes(good[8:16], "little")
        g = np.random.default_rng(7)
        agree_reject = 0
        for k in range(300):
            pos = 16 + int(g.integers(0, hlen))
            bad = bytearray(good)
            bad[pos] = int(g.integers(0x20, 0x7F))
            got, want = ours(bytes(bad)), theirs(bytes(bad))
            assert (got[0] is None) == (want[0] is None), (k, pos, got, want)
            if got[0] is None:
                agree_reject += 1
                if not want[1].startswith("invalid .efq header"):
                    assert got[1] == want[1], (k, pos)
            else:
                assert got[0] == want[0]
        assert agree_reject > 50


@needs_ref
@pytest.mark.parametrize("seed", [11, 12, 13])
def test_double_byte_corruptions_agree_with_the_reference(seed):
    """500 seeded two-byte edits of the header per seed (printable ASCII): the first failing check,
    and so the message, is the same as the reference reader's."""
    with tempfile.TemporaryDirectory() as d:
        _, _, good = written(d, q8={(0, "wv")})
        hlen = int.from_bytes(good[8:16], "little")
        g = np.random.default_rng(seed)
        for k in range(500):
            bad = bytearray(good)
            for _ in range(2):
                bad[16 + int(g.integers(0, hlen))] = int(g.integers(0x20, 0x7F))
            got, want = ours(bytes(bad)), theirs(bytes(bad))
            assert (got[0] is None) == (want[0] is None), (k, got, want)
            if got[0] is None and not want[1].startswith("invalid .efq header"):
                assert got[1] == want[1], (k, got, want)


CONFIG_KEYS = ["model_type", "hidden_act", "hidden_size", "intermediate_size", "num_hidden_layers",
               "num_attention_heads", "num_key_value_heads", "vocab_size", "max_position_embeddings",
               "rms_norm_eps", "rope_theta", "tie_word_embeddings", "bos_token_id", "eos_token_id"]
VALUES = ['null', '"x"', '7', '-3', '0', '1.5', 'true', '[]', '{}', '1048577', '16777217', '1e400', '2']


@needs_ref
@pytest.mark.parametrize("key", CONFIG_KEYS + ["head_dim", "rope_scaling", "attention_bias", "mlp_bias", "dtype",
                                               "torch_dtype"])
def test_config_field_values_agree_with_the_reference(key):
    """Every config field set to each of a set of values (absent, wrong JSON type, out of range,
    inconsistent with the other fields): accepted or rejected with the same message as the
    reference's config parser (src/model_config.cpp:72-131)."""
    import json
    import re
    with tempfile.TemporaryDirectory() as d:
        _, _, good = written(d)
        hlen = int.from_bytes(good[8:16], "little")
        header = json.loads(good[16:16 + hlen].decode())
        for v in VALUES + ["DELETE"]:
            h = json.loads(json.dumps(header))
            if v == "DELETE":
                h["config"].pop(key, None)
            else:
                h["config"][key] = "__V__"
            text = json.dumps(h, separators=(",", ":")).replace('"__V__"', v)
            if len(text) > hlen:
                continue
            text = text + " " * (hlen - len(text))
            bad = good[:16] + text.encode() + good[16 + hlen:]
            got, want = ours(bad), theirs(bad)
            assert (got[0] is None) == (want[0] is None), (key, v, got, want)
            if got[0] is None and not want[1].startswith("invalid .efq header"):
                assert got[1] == want[1], (key, v, got, want)
