"""GPU parity of the packed GEMV family, the quantizer and the row lookup (C-ABI calls).

Oracle: the CPU restatement (oracle/) of the reference kernels, plus float64 dequantize-then-dot.
Gates: max |gpu - cpu fp32| <= 1e-4 and |gpu - exact| <= 1e-5 * sum|w x|
(the reference's own kernel tolerance, tests/test_qinfer.cpp:95 and src/eval_quant.cpp:31);
packed bytes of the quantizer bit-identical.
"""
import numpy as np
import pytest

import oracle as O
from tests import _data as D

pytestmark = pytest.mark.gpu

ABS_TOL = 1e-4
REL_TOL = 1e-5


def _gemv(H, qtype, packed, x, batch=1):
    rows = packed.shape[0]
    cols = x.shape[-1]
    W = H.Weight(qtype, rows, cols, host=packed)
    dx = H.DeviceArray.from_host(x.reshape(batch, cols))
    dy = H.DeviceArray((batch, rows))
    H.matvec(W, dx, dy, batch=batch)
    return dy.numpy()


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("rows,cols", [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (24, 32), (24, 64),
                                       (7, 96), (40, 160), (37, 256)])
def test_gemv_random_codes_match_exact_dot(hip, qtype, rows, cols):
    print(f"[case] gemv qtype={qtype} {rows}x{cols}", flush=True)
    packed = D.random_rows(qtype, rows, cols, seed=rows * 7 + cols + qtype)
    x = D.activations_with_outliers(seed=cols + qtype, n=cols)
    got = _gemv(hip, qtype, packed, x)[0]
    w64 = D.dequant_exact(qtype, packed, cols)
    err = D.rel_dot_error(w64, x, got)
    assert err.max() < REL_TOL, err.max()
    cpu = O.matvec(qtype, packed.reshape(-1), x, backend=O.AVX2)
    assert np.abs(got - cpu).max() <= ABS_TOL + 1e-5 * np.abs(cpu).max()
    again = _gemv(hip, qtype, packed, x)[0]
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))  # reproducible bits


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0])
def test_gemv_config1_quantized_weights(hip, qtype):
    """Config 1: 2048x2048 N(0,0.02) quantized by the reference quantizer, x ~ N(0,1)."""
    w = D.normal(11, (2048, 2048), 0.02)
    packed = O.quantize(qtype, w)
    x = D.normal(12, 2048)
    got = _gemv(hip, qtype, packed, x)[0]
    cpu = O.matvec(qtype, packed.reshape(-1), x, backend=O.AVX2)
    scalar = O.matvec(qtype, packed.reshape(-1), x, backend=O.SCALAR)
    assert np.abs(got - cpu).max() <= ABS_TOL
    assert np.abs(got - scalar).max() <= ABS_TOL
    err = D.rel_dot_error(D.dequant_exact(qtype, packed, 2048), x, got)
    assert err.max() < REL_TOL


@pytest.fixture(scope="module")
def lm_head_q8():
    """Config 3's lm_head: 32000x2048 from N(0,0.02), quantized Q8_0 by the oracle's quantizer
    (src/quant.cpp:95-125), with its float64 decode."""
    packed = O.quantize(O.Q8_0, D.normal(31, (32000, 2048), 0.02))
    return packed, D.dequant_exact(O.Q8_0, packed, 2048)


@pytest.mark.parametrize("batch", [1, 16, 64])
def test_gemv_config3_lm_head_q8_0(hip, lm_head_q8, batch):
    """The Q8_0 lm_head product on its own (src/model.cpp:272-275 -> kern::matvec): hidden vectors
    from N(0,1), one sequence (config 3) and the batched decode's 16 and 64 (config 4).  Every
    sequence meets both gates against the oracle's AVX2 kernel and the exact dot."""
    packed, w64 = lm_head_q8
    print(f"[case] Q8_0 lm_head 32000x2048 B={batch}", flush=True)
    X = np.stack([D.normal(32 + b, 2048) for b in range(batch)])
    got = _gemv(hip, O.Q8_0, packed, X, batch=batch)
    x64 = X.T.astype(np.float64)
    exact = w64 @ x64
    mag = np.abs(w64) @ np.abs(x64)
    rel = np.abs(got.T.astype(np.float64) - exact) / np.maximum(mag, 1e-30)
    assert rel.max() < REL_TOL, rel.max()
    pool = O.Pool(8)
    for b in range(batch):
        cpu = O.matvec(O.Q8_0, packed.reshape(-1), X[b], backend=O.AVX2, pool=pool)
        assert np.abs(got[b] - cpu).max() <= ABS_TOL, b
    pool.close()


def test_gemv_edge_codes(hip):
    """tests/test_qinfer.cpp:100-122 on the device: nibble layout, zero scale, Q8 extremes."""
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:] = 0x88
    blk[2 + 3] = 0x0F
    x = np.zeros(32, np.float32)
    x[3], x[19] = 2.0, 0.5
    assert _gemv(hip, O.Q4_0, blk.reshape(1, 18), x)[0][0] == 7.0 * 2.0 + -8.0 * 0.5
    blk[0:2] = 0
    assert _gemv(hip, O.Q4_0, blk.reshape(1, 18), x)[0][0] == 0.0
    b8 = np.zeros(34, np.uint8)
    b8[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b8[2] = np.uint8(256 - 127)
    b8[2 + 31] = 127
    ones = np.ones(32, np.float32)
    assert _gemv(hip, O.Q8_0, b8.reshape(1, 34), ones)[0][0] == 0.0
    b8[2 + 5] = 3
    assert _gemv(hip, O.Q8_0, b8.reshape(1, 34), ones)[0][0] == 3.0


@pytest.mark.parametrize("batch", [2, 16, 64])
def test_gemv_batched_equals_per_sequence(hip, batch):
    qtype, rows, cols = O.Q4_0, 512, 2048
    packed = D.random_rows(qtype, rows, cols, seed=5)
    X = D.normal(6, (batch, cols))
    got = _gemv(hip, qtype, packed, X, batch=batch)
    w64 = D.dequant_exact(qtype, packed, cols)
    for b in range(batch):
        assert D.rel_dot_error(w64, X[b], got[b]).max() < REL_TOL
        one = _gemv(hip, qtype, packed, X[b])[0]
        assert np.abs(one - got[b]).max() <= 1e-6 * max(1.0, np.abs(one).max())


def test_gemv_jobs_mixed_types_match_single(hip):
    """q/k/v in one launch with k, v stored Q8_0 (layer 0 of the TinyLlama policy)."""
    cols = 2048
    x = D.normal(21, cols)
    shapes = [(O.Q4_0, 2048), (O.Q8_0, 256), (O.Q8_0, 256)]
    ws, outs, keep = [], [], []
    dx = hip.DeviceArray.from_host(x)
    for i, (qt, rows) in enumerate(shapes):
        packed = O.quantize(qt, D.normal(30 + i, (rows, cols), 0.02))
        keep.append(packed)
        ws.append(hip.Weight(qt, rows, cols, host=packed))
        outs.append(hip.DeviceArray((rows,)))
    hip.matvec_jobs([(ws[i], dx, outs[i]) for i in range(3)])
    for i, (qt, rows) in enumerate(shapes):
        single = _gemv(hip, qt, keep[i], x)[0]
        assert np.array_equal(outs[i].numpy(), single)
        cpu = O.matvec(qt, keep[i].reshape(-1), x)
        assert np.abs(single - cpu).max() <= ABS_TOL


def test_gemv_fused_rmsnorm_residual_swiglu(hip):
    """Transformer::forward chains (src/model.cpp:227-262) against the oracle's separate ops."""
    D_, F = 2048, 5632
    x = D.normal(40, D_)
    nw = (1.0 + 0.1 * D.normal(41, D_)).astype(np.float32)
    g = O.quantize(O.Q4_0, D.normal(42, (F, D_), 0.02))
    u = O.quantize(O.Q4_0, D.normal(43, (F, D_), 0.02))
    dn = O.quantize(O.Q4_0, D.normal(44, (D_, F), 0.02))
    # oracle chain
    L = O.lib()
    h = np.empty_like(x)
    L.efo_rmsnorm(O.ptr(h, O._f32p), O.ptr(x, O._f32p), O.ptr(nw, O._f32p), D_, 1e-5)
    gate, up = O.matvec_jobs([(O.Q4_0, g, h), (O.Q4_0, u, h)])
    act = np.empty_like(gate)
    L.efo_swiglu(O.ptr(act, O._f32p), O.ptr(gate, O._f32p), O.ptr(up, O._f32p), F)
    down = O.matvec(O.Q4_0, dn.reshape(-1), act)
    ref = x + down
    # device chain
    G, U, Dn = (hip.Weight(O.Q4_0, F, D_, host=g), hip.Weight(O.Q4_0, F, D_, host=u),
                hip.Weight(O.Q4_0, D_, F, host=dn))
    dx = hip.DeviceArray.from_host(x)
    dnw = hip.DeviceArray.from_host(nw)
    dact = hip.DeviceArray((F,))
    hip.matvec_swiglu(G, U, dx, dact, norm_w=dnw, eps=1e-5)
    got_act = dact.numpy()
    assert np.abs(got_act - act).max() <= ABS_TOL
    hip.matvec_residual(Dn, dact, dx)
    got = dx.numpy()
    assert np.abs(got - ref).max() <= ABS_TOL


@pytest.mark.parametrize("qtype,search", [(O.Q4_0, True), (O.Q4_0, False), (O.Q8_0, True), (O.BF16, True),
                                          (O.F16, True)])
def test_quantizer_bytes_match_reference_restatement(hip, qtype, search):
    rows, cols = 96, 2048
    w = D.normal(50, (rows, cols), 0.02)
    w[::7, 5] *= 6.0  # outliers
    w[3, 64:96] = 0.0  # all-zero block
    w[4, 96:128] = 1e-9  # underflows fp16 scales
    w[5, 0] = 70000.0  # scale clamp
    w[6, 100] = np.inf  # non-finite blocks follow the reference's x86-64 build
    w[7, 200] = np.nan
    dw = hip.DeviceArray.from_host(w)
    got = hip.quantize(qtype, dw, rows, cols, search=search).numpy()
    want = np.empty((rows, O.row_bytes(qtype, cols)), np.uint8)
    for r in range(rows):
        assert O.lib().efo_quantize_row(qtype, O.ptr(w[r], O._f32p), cols, O.ptr(want[r], O._u8p), int(search)) == 0
    assert np.array_equal(got.reshape(rows, -1), want)


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.BF16, O.F16, O.F32])
def test_rows_f32_is_exact_dequantization(hip, qtype):
    rows, cols = 40, 256
    w = D.normal(60, (rows, cols), 0.5)
    packed = O.quantize(qtype, w)
    W = hip.Weight(qtype, rows, cols, host=packed)
    ids = np.array([0, 39, 7, 7, 12], np.int32)
    out = hip.DeviceArray((len(ids), cols))
    hip.rows_f32(W, hip.DeviceArray.from_host(ids), out, batch=len(ids))
    got = out.numpy()
    ref = O.dequantize(qtype, packed, cols)
    for i, r in enumerate(ids):
        assert np.array_equal(got[i].view(np.uint32), ref[r].view(np.uint32))
