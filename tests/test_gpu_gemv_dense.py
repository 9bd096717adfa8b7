"""GPU parity of the GEMV over unquantized weights: F32, F16 and BF16 rows (C-ABI calls).

kern::matvec_rows dispatches all five storage types (src/qkernels.cpp:213-269); these three reach
the decode path through lossless .efq files, tied embeddings and the quantizer's BF16 fallback for
row lengths that are not a multiple of 32.  Gates as for the packed types (BASELINE.json
north_star, tests/test_qinfer.cpp:95): |gpu - exact| <= 1e-5 * sum|w x| per row against a float64
dot of the exactly decoded weights, and max |gpu - cpu| <= 1e-4 against the oracle's AVX2 kernels
(dot_bf16_avx2 / dot_f32_avx2 / the F16 loop, src/qkernels.cpp:182-234).  Shapes cover the 16-byte
vector path, odd row lengths (per-element path), a partial last tile, batches and every epilogue.
"""
import numpy as np
import pytest

import oracle as O
from tests import _data as D

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 0, 1, 2
ABS_TOL = 1e-4
REL_TOL = 1e-5


def dense_rows(qtype, rows, cols, seed, scale=0.02):
    """Raw row bytes [rows, row_bytes] and their exact float64 values."""
    w = D.normal(seed, (rows, cols), scale)
    if qtype == F32:
        raw = w
        exact = w.astype(np.float64)
    elif qtype == F16:
        h = w.astype(np.float16)
        h.reshape(-1)[::53] = np.float16(3e-6)  # subnormal fp16 values
        h.reshape(-1)[::71] = np.float16(-0.0)
        raw = h
        exact = h.astype(np.float64)
    else:
        bits = (w.view(np.uint32) >> 16).astype(np.uint16)  # truncated bf16: any finite pattern
        raw = bits
        exact = (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return np.ascontiguousarray(raw).view(np.uint8).reshape(rows, -1), exact


@pytest.mark.parametrize("qtype", [F32, F16, BF16])
@pytest.mark.parametrize("rows,cols,batch", [
    (300, 2048, 1),    # vector path, partial last tile
    (37, 33, 1),       # odd row length: per-element path
    (64, 5632, 3),     # batch
    (5, 16, 2),        # tiny rows (F32: one 16-byte step per row)
    (130, 40, 1),      # BF16 / F16 rows of 80 bytes
])
def test_dense_gemv_meets_the_gates(hip, qtype, rows, cols, batch):
    print(f"[case] dense gemv qtype={qtype} {rows}x{cols} B={batch}", flush=True)
    raw, w64 = dense_rows(qtype, rows, cols, seed=rows * 7 + cols + qtype)
    X = np.stack([D.activations_with_outliers(500 + b, cols) for b in range(batch)]).astype(np.float32)
    W = hip.Weight(qtype, rows, cols, host=raw)
    dx = hip.DeviceArray.from_host(X)
    dy = hip.DeviceArray((batch, rows))
    hip.matvec(W, dx, dy, batch=batch)
    got = dy.numpy()
    for b in range(batch):
        assert D.rel_dot_error(w64, X[b], got[b]).max() < REL_TOL, b
        cpu = O.matvec(qtype, raw.reshape(-1), X[b], backend=O.AVX2)
        assert np.abs(got[b] - cpu).max() <= ABS_TOL + 1e-5 * np.abs(cpu).max(), b
    hip.matvec(W, dx, dy, batch=batch)
    assert np.array_equal(dy.numpy().view(np.uint32), got.view(np.uint32))  # reproducible bits


def test_dense_swiglu_residual_and_norm(hip):
    """Transformer::forward's FFN chain (src/model.cpp:249-262) on BF16 matrices."""
    B, D_, F = 2, 256, 704
    X = np.stack([D.normal(80 + b, D_) for b in range(B)]).astype(np.float32)
    nw = (1.0 + 0.1 * D.normal(81, D_)).astype(np.float32)
    g, _ = dense_rows(BF16, F, D_, 82)
    u, _ = dense_rows(BF16, F, D_, 83)
    dn, _ = dense_rows(BF16, D_, F, 84)
    G, U, Dn = hip.Weight(BF16, F, D_, host=g), hip.Weight(BF16, F, D_, host=u), hip.Weight(BF16, D_, F, host=dn)
    dx = hip.DeviceArray.from_host(X)
    dact = hip.DeviceArray((B, F))
    hip.matvec_swiglu(G, U, dx, dact, norm_w=hip.DeviceArray.from_host(nw), eps=1e-5, batch=B)
    hip.matvec_residual(Dn, dact, dx, batch=B)
    got_act, got = dact.numpy(), dx.numpy()
    L = O.lib()
    for b in range(B):
        h = np.empty(D_, np.float32)
        L.efo_rmsnorm(O.ptr(h, O._f32p), O.ptr(X[b], O._f32p), O.ptr(nw, O._f32p), D_, 1e-5)
        gate, up = O.matvec_jobs([(BF16, g, h), (BF16, u, h)])
        act = np.empty_like(gate)
        L.efo_swiglu(O.ptr(act, O._f32p), O.ptr(gate, O._f32p), O.ptr(up, O._f32p), F)
        assert np.abs(got_act[b] - act).max() <= ABS_TOL, b
        ref = X[b] + O.matvec(BF16, dn.reshape(-1), got_act[b])
        assert np.abs(got[b] - ref).max() <= ABS_TOL, b


def test_mixed_packed_and_dense_jobs_in_one_call(hip):
    """q (Q4_0), k (BF16), v (F16) in one matvec_jobs call with the input norm fused: split into one
    launch per kind, each job equal to the oracle on the normalised input."""
    B, cols = 2, 512
    X = np.stack([D.normal(90 + b, cols) for b in range(B)]).astype(np.float32)
    nw = (1.0 + 0.05 * D.normal(91, cols)).astype(np.float32)
    q = O.quantize(O.Q4_0, D.normal(92, (512, cols), 0.02))
    k, _ = dense_rows(BF16, 64, cols, 93)
    v, _ = dense_rows(F16, 64, cols, 94)
    specs = [(O.Q4_0, 512, q), (BF16, 64, k), (F16, 64, v)]
    ws = [hip.Weight(qt, r, cols, host=p) for qt, r, p in specs]
    outs = [hip.DeviceArray((B, 512)) for _ in specs]
    dx = hip.DeviceArray.from_host(X)
    hip.matvec_jobs_rmsnorm([(ws[i], dx, outs[i]) for i in range(3)], hip.DeviceArray.from_host(nw), 1e-5,
                            batch=B, ldx=cols, ldy=512)
    L = O.lib()
    for b in range(B):
        h = np.empty(cols, np.float32)
        L.efo_rmsnorm(O.ptr(h, O._f32p), O.ptr(X[b], O._f32p), O.ptr(nw, O._f32p), cols, 1e-5)
        for i, (qt, rows, p) in enumerate(specs):
            cpu = O.matvec(qt, p.reshape(-1), h)
            assert np.abs(outs[i].numpy()[b, :rows] - cpu).max() <= ABS_TOL, (b, i)
