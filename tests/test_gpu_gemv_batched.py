"""GPU parity of the batched (2+ sequences) packed GEMV on the matrix cores (C-ABI calls).

Every sequence of a batch must meet the single-vector gates:
|gpu - exact| <= 1e-5 * sum|w x| per row (tests/test_qinfer.cpp:95) and max |gpu - cpu fp32| <= 1e-4
against the oracle's AVX2 kernel (src/qkernels.cpp:131-180) on that sequence alone.  Shapes cover
batches that are not a multiple of the 16-sequence tile, many tiles in one launch, more than 1024
sequences (several launches), row counts that leave a partial workgroup, Q8_0, a K split (K = 5632
at B = 64) and mixed-type launches; epilogues and the fused RMSNorm are checked against the oracle's separate operations.
"""
import numpy as np
import pytest

import oracle as O
from tests import _data as D

pytestmark = pytest.mark.gpu

ABS_TOL = 1e-4
REL_TOL = 1e-5


def _batch_x(seed, batch, cols):
    return np.stack([D.activations_with_outliers(seed + b, cols) for b in range(batch)]).astype(np.float32)



@pytest.mark.parametrize("qtype,rows,cols,batch", [
    (O.Q4_0, 512, 2048, 5),      # one partial sequence tile
    (O.Q8_0, 300, 2048, 16),     # Q8_0, rows leave a partial workgroup
    (O.Q4_0, 2048, 5632, 64),    # K split across workgroups
    (O.Q4_0, 37, 256, 70),       # tiny K, a partial last tile
    (O.Q4_0, 96, 512, 300),      # 19 sequence tiles in one launch
    (O.Q8_0, 37, 256, 1100),     # two launches (1024 + 76 sequences)
    (O.Q8_0, 64, 512, 2),
    (O.Q4_0, 5632, 2048, 16),    # config 4 at B = 16: gate / up shape
    (O.Q4_0, 2048, 5632, 16),    # down shape (K = 5632)
    (O.Q8_0, 256, 2048, 16),     # a Q8_0 k / v override
    (O.Q4_0, 2048, 2048, 16),    # q / o shape
    (O.Q4_0, 5632, 2048, 64),    # config 4 at B = 64
    (O.Q8_0, 256, 2048, 64),
])
def test_batched_gemv_each_sequence_meets_the_gates(hip, qtype, rows, cols, batch):
    print(f"[case] batched gemv qtype={qtype} {rows}x{cols} B={batch}", flush=True)
    packed = D.random_rows(qtype, rows, cols, seed=rows + cols + batch)
    X = _batch_x(1000 + batch, batch, cols)
    W = hip.Weight(qtype, rows, cols, host=packed)
    dx = hip.DeviceArray.from_host(X)
    dy = hip.DeviceArray((batch, rows))
    hip.matvec(W, dx, dy, batch=batch)
    got = dy.numpy()
    w64 = D.dequant_exact(qtype, packed, cols)
    for b in range(batch):
        assert D.rel_dot_error(w64, X[b], got[b]).max() < REL_TOL, b
        cpu = O.matvec(qtype, packed.reshape(-1), X[b], backend=O.AVX2)
        assert np.abs(got[b] - cpu).max() <= ABS_TOL + 1e-5 * np.abs(cpu).max(), b
    hip.matvec(W, dx, dy, batch=batch)
    assert np.array_equal(dy.numpy().view(np.uint32), got.view(np.uint32))  # reproducible bits


@pytest.mark.parametrize("B", [64, 300])  # 300: the many-sequence kernel (a batched prefill's shape)
def test_batched_swiglu_and_residual_chain(hip, B):
    """Transformer::forward's FFN chain (src/model.cpp:249-262) for 64 and 300 sequences at once."""
    print(f"[case] ffn chain B={B}", flush=True)
    D_, F = 2048, 5632
    X = np.stack([D.normal(40 + b, D_) for b in range(B)]).astype(np.float32)
    nw = (1.0 + 0.1 * D.normal(41, D_)).astype(np.float32)
    g = O.quantize(O.Q4_0, D.normal(42, (F, D_), 0.02))
    u = O.quantize(O.Q4_0, D.normal(43, (F, D_), 0.02))
    dn = O.quantize(O.Q4_0, D.normal(44, (D_, F), 0.02))
    G, U, Dn = (hip.Weight(O.Q4_0, F, D_, host=g), hip.Weight(O.Q4_0, F, D_, host=u),
                hip.Weight(O.Q4_0, D_, F, host=dn))
    dx = hip.DeviceArray.from_host(X)
    dnw = hip.DeviceArray.from_host(nw)
    dact = hip.DeviceArray((B, F))
    hip.matvec_swiglu(G, U, dx, dact, norm_w=dnw, eps=1e-5, batch=B)
    hip.matvec_residual(Dn, dact, dx, batch=B)  # K = 5632 at B = 64: split-K with a finalize pass
    got_act, got = dact.numpy(), dx.numpy()
    L = O.lib()
    for b in list(range(0, B, 9)) + [B - 1]:
        h = np.empty(D_, np.float32)
        L.efo_rmsnorm(O.ptr(h, O._f32p), O.ptr(X[b], O._f32p), O.ptr(nw, O._f32p), D_, 1e-5)
        gate, up = O.matvec_jobs([(O.Q4_0, g, h), (O.Q4_0, u, h)])
        act = np.empty_like(gate)
        L.efo_swiglu(O.ptr(act, O._f32p), O.ptr(gate, O._f32p), O.ptr(up, O._f32p), F)
        assert np.abs(got_act[b] - act).max() <= ABS_TOL, b
        ref = X[b] + O.matvec(O.Q4_0, dn.reshape(-1), got_act[b])
        assert np.abs(got[b] - ref).max() <= ABS_TOL, b


@pytest.mark.parametrize("B", [8, 270])
def test_batched_mixed_type_jobs_with_norm(hip, B):
    """q/k/v with k, v stored Q8_0 in one launch for 8 and 270 sequences, input RMSNorm fused."""
    print(f"[case] mixed q/k/v B={B}", flush=True)
    cols = 2048
    X = np.stack([D.normal(60 + b, cols) for b in range(B)]).astype(np.float32)
    nw = (1.0 + 0.05 * D.normal(61, cols)).astype(np.float32)
    shapes = [(O.Q4_0, 2048), (O.Q8_0, 256), (O.Q8_0, 256)]
    keep, ws, outs = [], [], []
    for i, (qt, rows) in enumerate(shapes):
        packed = O.quantize(qt, D.normal(70 + i, (rows, cols), 0.02))
        keep.append(packed)
        ws.append(hip.Weight(qt, rows, cols, host=packed))
        outs.append(hip.DeviceArray((B, 2048)))  # one output stride for the launch (the C-ABI's ldy)
    dx = hip.DeviceArray.from_host(X)
    hip.matvec_jobs_rmsnorm([(ws[i], dx, outs[i]) for i in range(3)], hip.DeviceArray.from_host(nw), 1e-5, batch=B,
                            ldx=cols, ldy=2048)
    L = O.lib()
    for b in range(0, B, 1 if B <= 16 else 7):
        h = np.empty(cols, np.float32)
        L.efo_rmsnorm(O.ptr(h, O._f32p), O.ptr(X[b], O._f32p), O.ptr(nw, O._f32p), cols, 1e-5)
        for i, (qt, rows) in enumerate(shapes):
            cpu = O.matvec(qt, keep[i].reshape(-1), h)
            assert np.abs(outs[i].numpy()[b, :rows] - cpu).max() <= ABS_TOL, (b, i)


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0])
def test_batched_gemv_dynamic_range(hip, qtype):
    """Sequences 12 decades apart, one block 1e5 above the rest of its sequence and an all-zero
    sequence in one launch: each sequence meets the gates on its own (every sequence has its own
    power-of-two scale), and the zero sequence gives exact zeros."""
    rows, cols, B = 96, 2048, 20
    print(f"[case] batched gemv dynamic range qtype={qtype}", flush=True)
    packed = D.random_rows(qtype, rows, cols, seed=91)
    X = _batch_x(500, B, cols) * (10.0 ** np.linspace(-6.0, 6.0, B))[:, None]
    X[3, 64:96] *= 1e5
    X[7, :] = 0.0
    X = X.astype(np.float32)
    W = hip.Weight(qtype, rows, cols, host=packed)
    dx = hip.DeviceArray.from_host(X)
    dy = hip.DeviceArray((B, rows))
    hip.matvec(W, dx, dy, batch=B)
    got = dy.numpy()
    w64 = D.dequant_exact(qtype, packed, cols)
    for b in range(B):
        assert D.rel_dot_error(w64, X[b], got[b]).max() < REL_TOL, b
    assert not got[7].any()


def test_batched_norm_long_rows(hip):
    """An RMSNorm fused into a product whose rows are longer than one workgroup's blocks (K = 4096,
    a K split): the results meet the gates against the oracle's norm + matvec."""
    B, cols, rows = 6, 4096, 128
    X = np.stack([D.normal(80 + b, cols) for b in range(B)]).astype(np.float32)
    nw = (1.0 + 0.05 * D.normal(81, cols)).astype(np.float32)
    packed = O.quantize(O.Q4_0, D.normal(82, (rows, cols), 0.02))
    W = hip.Weight(O.Q4_0, rows, cols, host=packed)
    out = hip.DeviceArray((B, rows))
    hip.matvec_jobs_rmsnorm([(W, hip.DeviceArray.from_host(X), out)], hip.DeviceArray.from_host(nw), 1e-5,
                            batch=B, ldx=cols, ldy=rows)
    L = O.lib()
    for b in range(B):
        h = np.empty(cols, np.float32)
        L.efo_rmsnorm(O.ptr(h, O._f32p), O.ptr(X[b], O._f32p), O.ptr(nw, O._f32p), cols, 1e-5)
        assert np.abs(out.numpy()[b] - O.matvec(O.Q4_0, packed.reshape(-1), h)).max() <= ABS_TOL, b


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0])
def test_refresh_after_rewriting_device_bytes(hip, qtype):
    """Batched products read a tile-order copy made on first use; ef_hip_weight_refresh rewrites it
    from the handle's current bytes, so a caller that rewrites the bytes sees the new matrix."""
    rows, cols, batch = 96, 512, 16
    print(f"[case] refresh qtype={qtype} {rows}x{cols} B={batch}", flush=True)
    first = D.random_rows(qtype, rows, cols, seed=11)
    second = D.random_rows(qtype, rows, cols, seed=12)
    buf = hip.DeviceArray.from_host(first.reshape(-1))
    W = hip.Weight(qtype, rows, cols, device=buf)
    X = _batch_x(77, batch, cols)
    dx = hip.DeviceArray.from_host(X)
    dy = hip.DeviceArray((batch, rows))
    hip.matvec(W, dx, dy, batch=batch)
    y_first = dy.numpy()
    buf.upload(second.reshape(-1))
    hip.matvec(W, dx, dy, batch=batch)
    assert np.array_equal(dy.numpy(), y_first)  # the copy still holds the former bytes
    W.refresh()
    hip.matvec(W, dx, dy, batch=batch)
    got = dy.numpy()
    w64 = D.dequant_exact(qtype, second, cols)
    for b in range(batch):
        assert D.rel_dot_error(w64, X[b], got[b]).max() < REL_TOL, b
    # batch 1 reads the bytes in place: the same matrix either way
    y1 = hip.DeviceArray((rows,))
    hip.matvec(W, hip.DeviceArray.from_host(X[0]), y1, batch=1)
    assert np.abs(y1.numpy() - got[0]).max() <= ABS_TOL + 1e-5 * np.abs(got[0]).max()
