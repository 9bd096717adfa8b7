"""Seeded synthetic inputs shared by the CPU and GPU tests (numpy PCG64 streams)."""
from __future__ import annotations

import numpy as np

QK = 32
BLOCK = {4: 18, 3: 34}  # Q4_0, Q8_0 block bytes


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(seed: int, shape, scale: float = 1.0) -> np.ndarray:
    return (rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def activations_with_outliers(seed: int, n: int) -> np.ndarray:
    """N(0,1) with ~2% of channels scaled by 30 (tests/test_qinfer.cpp:76)."""
    g = rng(seed)
    x = g.standard_normal(n, dtype=np.float32)
    big = g.standard_normal(n, dtype=np.float32) > 2.0
    return np.where(big, x * 30.0, x).astype(np.float32)


def random_rows(qtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Arbitrary packed bytes with finite fp16 scales of both signs in [-0.05, 0.05], including
    subnormal scales (tests/test_qinfer.cpp:26-40): every code value a kernel can meet."""
    bs = BLOCK[qtype]
    nb = rows * cols // QK
    g = rng(seed)
    raw = g.integers(0, 256, size=(nb, bs), dtype=np.uint8)
    d = g.uniform(-0.05, 0.05, size=nb).astype(np.float32)
    d[::97] = np.float32(3e-6)  # fp16 subnormal scales
    d[::89] = -np.float32(1e-7)
    raw[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return raw.reshape(rows, cols // QK * bs)


def dequant_exact(qtype: int, packed: np.ndarray, cols: int) -> np.ndarray:
    """Closed-form block decode in float64 (include/ef/quant.h:3-6), independent of the oracle."""
    bs = BLOCK[qtype]
    rows = packed.shape[0]
    b = packed.reshape(rows, cols // QK, bs)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)  # exact widening
    if qtype == 4:
        qs = b[:, :, 2:18].astype(np.int32)
        codes = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=2)
    else:
        codes = b[:, :, 2:34].view(np.int8).astype(np.int32)
    return (codes * d).reshape(rows, cols)


def rel_dot_error(w64: np.ndarray, x: np.ndarray, got: np.ndarray) -> np.ndarray:
    """|got - exact| / sum|w x| per row (tests/test_qinfer.cpp:57-67)."""
    x64 = x.astype(np.float64)
    exact = w64 @ x64
    mag = np.abs(w64) @ np.abs(x64)
    return np.abs(got.astype(np.float64) - exact) / np.maximum(mag, 1e-30)
