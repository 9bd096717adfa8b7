"""CPU pinning of the oracle's 16-bit float and Q4_0 / Q8_0 block codec (oracle/efo_codec.c).

Pinned by: the reference's known-answer tests (tests/test_fp16.cpp, tests/test_quant.cpp:52-153),
closed forms independent of the oracle (IEEE round-to-nearest-even via numpy float16, the block
layout decoded in numpy), invariants (search never worse, error bounds), the reference build
(oracle/_ref, when present) bit for bit, and committed golden fixtures made by that build.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

L = O.lib()
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not present")
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "fixtures.json")))


def f16_all():
    h = np.arange(65536, dtype=np.uint16)
    out = np.empty(65536, np.float32)
    L.efo_fp16_to_f32_n(O.ptr(h, O._u16p), O.ptr(out, O._f32p), 65536)
    return h, out


def to_fp16(f):
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.size, np.uint16)
    L.efo_f32_to_fp16_n(O.ptr(f, O._f32p), O.ptr(out, O._u16p), f.size)
    return out


def to_bf16(f):
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.size, np.uint16)
    L.efo_f32_to_bf16_n(O.ptr(f, O._f32p), O.ptr(out, O._u16p), f.size)
    return out


# ---------------------------------------------------------------------------------- fp16 / bf16

def test_fp16_known_values():  # tests/test_fp16.cpp:62-73
    assert L.efo_fp16_to_f32(0x3C00) == 1.0 and L.efo_fp16_to_f32(0xC000) == -2.0
    assert L.efo_fp16_to_f32(0x7BFF) == 65504.0
    assert L.efo_fp16_to_f32(0x0001) == 2.0 ** -24 and L.efo_fp16_to_f32(0x03FF) == 1023 * 2.0 ** -24
    assert L.efo_fp16_to_f32(0x0400) == 2.0 ** -14
    assert np.isinf(L.efo_fp16_to_f32(0x7C00)) and np.isnan(L.efo_fp16_to_f32(0x7E00))
    assert L.efo_f32_to_fp16(65519.0) == 0x7BFF and L.efo_f32_to_fp16(65520.0) == 0x7C00
    assert L.efo_f32_to_fp16(1.0 + 2.0 ** -11) == 0x3C00 and L.efo_f32_to_fp16(1.0 + 3 * 2.0 ** -11) == 0x3C02
    assert L.efo_f32_to_fp16(2.0 ** -25) == 0 and L.efo_f32_to_fp16(1.5 * 2.0 ** -25) == 1
    assert L.efo_f32_to_fp16(3 * 2.0 ** -25) == 2 and L.efo_f32_to_fp16(-(2.0 ** -30)) == 0x8000


def test_fp16_decode_exhaustive_matches_ieee():
    """All 65,536 patterns against numpy's IEEE binary16 widening (exact), NaN as NaN."""
    h, got = f16_all()
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    back = to_fp16(got)
    assert np.array_equal(back[~nan], h[~nan])  # round trip of every non-NaN pattern
    assert np.all((back[nan] & 0x7C00) == 0x7C00) and np.all(back[nan] & 0x3FF)


def test_fp16_encode_matches_ieee_round_to_nearest_even():
    """2M random floats (a quarter in the fp16 exponent range) against numpy's RNE conversion."""
    g = np.random.default_rng(7)
    u = g.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    u[::4] = (u[::4] & 0x807FFFFF) | ((100 + g.integers(0, 60, u[::4].size, dtype=np.uint32)) << 23)
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(to_fp16(f), want)


def test_bf16_round_trip_and_rounding():  # tests/test_fp16.cpp:17-60
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = (h.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(f)
    back = to_bf16(f)
    assert np.array_equal(back[~nan], h[~nan])
    assert np.all((back[nan] & 0x7F80) == 0x7F80) and np.all(back[nan] & 0x7F)
    bits = lambda u: np.array([u], np.uint32).view(np.float32)  # noqa: E731
    assert to_bf16(bits(0x3F808000))[0] == 0x3F80 and to_bf16(bits(0x3F818000))[0] == 0x3F82
    assert to_bf16(bits(0x3F808001))[0] == 0x3F81 and to_bf16(bits(0x7F7FFFFF))[0] == 0x7F80


@needs_ref
def test_fp16_bf16_match_reference_build():
    h, got = f16_all()
    ref = np.array([O.ref().ref_fp16_to_f32(int(v)) for v in h], np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
    f = np.random.default_rng(3).integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert [O.ref().ref_f32_to_fp16(float(v)) for v in f] == to_fp16(f).tolist()
    assert [O.ref().ref_f32_to_bf16(float(v)) for v in f] == to_bf16(f).tolist()


# ---------------------------------------------------------------------------------- block codec

def qblock(x, search=True):
    out = np.empty(18, np.uint8)
    L.efo_quantize_block_q4_0(O.ptr(np.ascontiguousarray(x, np.float32), O._f32p), O.ptr(out, O._u8p), int(search))
    return out


def deq4(b):
    out = np.empty(32, np.float32)
    L.efo_dequantize_row(O.Q4_0, O.ptr(b, O._u8p), 32, O.ptr(out, O._f32p))
    return out


def deq8(b):
    out = np.empty(32, np.float32)
    L.efo_dequantize_row(O.Q8_0, O.ptr(b, O._u8p), 32, O.ptr(out, O._f32p))
    return out


L.efo_quantize_block_q4_0.argtypes = [O._f32p, O._u8p, O.C.c_int]
L.efo_quantize_block_q8_0.argtypes = [O._f32p, O._u8p]


def test_q4_grid_round_trip_and_nibble_layout():  # tests/test_quant.cpp:52-69
    x = np.array([(j % 16 - 8) * 0.25 for j in range(32)], np.float32)
    assert np.array_equal(deq4(qblock(x)), x)
    m = np.zeros(18, np.uint8)
    m[0:2] = np.array([1.0], np.float16).view(np.uint8)
    m[2] = 0x2F
    y = deq4(m)
    assert y[0] == 7.0 and y[16] == -6.0 and y[1] == -8.0
    z = qblock(np.zeros(32, np.float32))
    assert z[0] == 0 and z[1] == 0 and z[2] == 0x88 and deq4(z)[5] == 0.0


def test_block_decode_matches_closed_form():
    """Every code value and random fp16 scales against include/ef/quant.h:3-6 evaluated in numpy."""
    g = np.random.default_rng(5)
    raw = g.integers(0, 256, size=(500, 18), dtype=np.uint8)
    raw[:, 0:2] = g.uniform(-4, 4, 500).astype(np.float16).view(np.uint8).reshape(500, 2)
    got = O.dequantize(O.Q4_0, raw, 32)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32)
    codes = np.concatenate([(raw[:, 2:] & 15).astype(np.int32) - 8, (raw[:, 2:] >> 4).astype(np.int32) - 8], 1)
    assert np.array_equal(got, (codes.astype(np.float32) * d).astype(np.float32))
    raw8 = g.integers(0, 256, size=(500, 34), dtype=np.uint8)
    raw8[:, 0:2] = g.uniform(-4, 4, 500).astype(np.float16).view(np.uint8).reshape(500, 2)
    got8 = O.dequantize(O.Q8_0, raw8, 32)
    d8 = raw8[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(got8, (raw8[:, 2:].view(np.int8).astype(np.float32) * d8).astype(np.float32))


def test_q4_search_never_worse_and_absmax_error_bound():  # tests/test_quant.cpp:71-105
    g = np.random.default_rng(11)
    x = (g.standard_normal((20000, 32)) * 0.02).astype(np.float32)
    idx = np.arange(0, 20000, 7)
    x[idx, idx % 32] *= 6.0
    s = O.quantize(O.Q4_0, x.reshape(-1, 32), search=True)
    p = O.quantize(O.Q4_0, x.reshape(-1, 32), search=False)
    ds, dp = O.dequantize(O.Q4_0, s, 32), O.dequantize(O.Q4_0, p, 32)
    es = ((x.astype(np.float64) - ds) ** 2).sum(1)
    ep = ((x.astype(np.float64) - dp) ** 2).sum(1)
    assert np.all(es <= ep * (1 + 1e-12))
    step = np.abs(p[:, 0:2].copy().view(np.float16).astype(np.float32))
    assert np.all(np.abs(x - dp) <= step * 1.01)
    ref = (x.astype(np.float64) ** 2).sum()
    rel_s, rel_p = np.sqrt(es.sum() / ref), np.sqrt(ep.sum() / ref)
    assert rel_s < rel_p and rel_s < 0.11


def test_q8_error_bound():  # tests/test_quant.cpp:107-128
    x = np.random.default_rng(12).standard_normal((5000, 32)).astype(np.float32)
    q = O.quantize(O.Q8_0, x)
    y = O.dequantize(O.Q8_0, q, 32)
    d = q[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.abs(x - y) <= d * 0.5001 + 1e-7)
    assert np.sqrt(((x.astype(np.float64) - y) ** 2).sum() / (x.astype(np.float64) ** 2).sum()) < 0.01


def test_row_bytes_and_fake_group():  # tests/test_quant.cpp:130-153
    assert O.row_bytes(O.Q4_0, 2048) == 64 * 18 and O.row_bytes(O.Q8_0, 2048) == 64 * 34
    assert O.row_bytes(O.BF16, 2048) == 4096
    with pytest.raises(ValueError, match="divisible by 32"):
        O.row_bytes(O.Q4_0, 30)
    x = np.random.default_rng(13).standard_normal(256).astype(np.float32)
    for t in (O.F32, O.F16, O.BF16, O.Q8_0, O.Q4_0):
        y = O.dequantize(t, O.quantize(t, x.reshape(1, -1)), 256)[0]
        e = np.abs(x - y).max()
        assert (t != O.F32 or e == 0.0) and e < 0.6
    fake = np.empty(256, np.float32)
    for b in range(0, 256, 32):
        L.efo_fake_quant_q4_group(O.ptr(x[b:b + 32].copy(), O._f32p), 32, O.ptr(fake[b:b + 32], O._f32p), 1)
    y = O.dequantize(O.Q4_0, O.quantize(O.Q4_0, x.reshape(8, 32)), 32).reshape(-1)
    assert np.array_equal(y, fake)


def special_rows(seed):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((16, 256)) * 0.02).astype(np.float32)
    w[::3, 7] *= 6.0
    w[1, 32:64] = 0.0
    w[2, 64:96] = 1e-9
    w[3, 0] = 70000.0
    w[4, 100] = np.inf
    w[5, 200] = np.nan
    w[6, 0:32] = -0.5
    return w


@needs_ref
@pytest.mark.parametrize("qtype,search", [(O.Q4_0, True), (O.Q4_0, False), (O.Q8_0, True)])
def test_quantizer_bytes_match_reference_build(qtype, search):
    for seed in range(4):
        w = special_rows(seed)
        got = O.quantize(qtype, w, search=search)
        want = np.empty_like(got)
        for r in range(w.shape[0]):
            assert O.ref().ref_quantize_row(qtype, O.ptr(w[r], O._f32p), 256, O.ptr(want[r]), int(search)) == 0
        assert np.array_equal(got, want), seed


@pytest.mark.parametrize("name", ["q4_search", "q4_plain", "q8"])
def test_quantizer_bytes_match_golden_fixtures(name):
    fx = GOLDEN["quant"][name]
    qtype = {"q4_search": O.Q4_0, "q4_plain": O.Q4_0, "q8": O.Q8_0}[name]
    for seed, want in fx["sha256"].items():
        got = O.quantize(qtype, special_rows(int(seed)), search=name != "q4_plain")
        assert hashlib.sha256(got.tobytes()).hexdigest() == want, seed
    first = bytes.fromhex(fx["row0_seed0_hex"])
    assert O.quantize(qtype, special_rows(0), search=name != "q4_plain")[0].tobytes() == first
