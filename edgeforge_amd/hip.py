"""Python view of the C-ABI: device buffers, weight handles and the hot-path calls.

Thin wrappers over include/ef_hip.h used by the tests, the smoke check and bench.py.  Arrays cross
the boundary as numpy (host) <-> DeviceArray (HIP device memory owned by the library allocator).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L
from ._lib import BF16, F16, F32, Q4_0, Q8_0, call, lib

__all__ = ["DeviceArray", "Weight", "Stream", "Event", "init", "row_bytes", "matvec", "matvec_jobs",
           "matvec_residual", "matvec_swiglu", "matvec_jobs_rmsnorm", "quantize", "rows_f32", "argmax", "sampler_exp",
           "RngStates", "sample", "F32", "F16", "BF16", "Q8_0", "Q4_0"]


def init(device: int = 0) -> None:
    L.init(device)


def row_bytes(qtype: int, cols: int) -> int:
    out = C.c_size_t()
    call("ef_hip_row_bytes", qtype, cols, C.byref(out))
    return out.value


class DeviceArray:
    """A contiguous device allocation with a numpy dtype and shape."""

    def __init__(self, shape, dtype=np.float32):
        init()
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        call("ef_hip_malloc", C.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray, stream=None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a, stream)
        return d

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        call("ef_hip_memcpy_h2d", self.ptr, a.ctypes.data, self.nbytes, _s(stream))

    def numpy(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        call("ef_hip_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes, _s(stream))
        return out

    def zero(self, stream=None) -> None:
        call("ef_hip_memset", self.ptr, 0, self.nbytes, _s(stream))

    def free(self) -> None:
        if getattr(self, "ptr", None):
            call("ef_hip_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def at(self, offset_elems: int) -> int:
        """Device address of element offset (for strided / sub-array calls)."""
        return self.ptr + offset_elems * self.dtype.itemsize


def _s(stream) -> int | None:
    if stream is None:
        return None
    return stream.ptr if isinstance(stream, Stream) else stream


class Stream:
    def __init__(self):
        init()
        p = C.c_void_p()
        call("ef_hip_stream_create", C.byref(p))
        self.ptr = p.value

    def sync(self) -> None:
        call("ef_hip_stream_sync", self.ptr)

    def __del__(self):
        try:
            if self.ptr:
                call("ef_hip_stream_destroy", self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self):
        init()
        p = C.c_void_p()
        call("ef_hip_event_create", C.byref(p))
        self.ptr = p.value

    def record(self, stream=None) -> None:
        call("ef_hip_event_record", self.ptr, _s(stream))

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        call("ef_hip_event_elapsed_ms", self.ptr, later.ptr, C.byref(ms))
        return ms.value

    def __del__(self):
        try:
            if self.ptr:
                call("ef_hip_event_destroy", self.ptr)
        except Exception:
            pass


def sync(stream=None) -> None:
    call("ef_hip_stream_sync", _s(stream))


class Weight:
    """A registered weight matrix (ef::WeightView on the device)."""

    def __init__(self, qtype: int, rows: int, cols: int, host: np.ndarray | None = None,
                 device: DeviceArray | None = None):
        init()
        self.qtype, self.rows, self.cols = qtype, rows, cols
        self.row_bytes = row_bytes(qtype, cols)
        h = C.c_void_p()
        self._keep = device
        if host is not None:
            host = np.ascontiguousarray(host)
            assert host.nbytes == self.row_bytes * rows, (host.nbytes, self.row_bytes * rows)
            call("ef_hip_weight_register_host", host.ctypes.data, qtype, rows, cols, C.byref(h))
        else:
            assert device is not None and device.nbytes >= self.row_bytes * rows
            call("ef_hip_weight_register_device", device.ptr, qtype, rows, cols, C.byref(h))
        self.handle = h.value

    def refresh(self, stream=None) -> None:
        """Rewrite the batched path's tile-order copy from the current bytes (after they changed)."""
        call("ef_hip_weight_refresh", self.handle, _s(stream))

    def release(self) -> None:
        if getattr(self, "handle", None):
            call("ef_hip_weight_release", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


def matvec(W: Weight, x: DeviceArray, y: DeviceArray, batch: int = 1, stream=None) -> None:
    call("ef_hip_matvec", W.handle, x.ptr, y.ptr, batch, W.cols, W.rows, _s(stream))


def matvec_residual(W: Weight, x: DeviceArray, y: DeviceArray, batch: int = 1, stream=None) -> None:
    call("ef_hip_matvec_residual", W.handle, x.ptr, y.ptr, batch, W.cols, W.rows, _s(stream))


def matvec_swiglu(G: Weight, U: Weight, x: DeviceArray, y: DeviceArray, norm_w: DeviceArray | None = None,
                  eps: float = 1e-5, batch: int = 1, stream=None) -> None:
    call("ef_hip_matvec_swiglu", G.handle, U.handle, x.ptr, norm_w.ptr if norm_w else None, eps, y.ptr, batch,
         G.cols, G.rows, _s(stream))


def _jobs(jobs):
    arr = (L.ef_hip_job * len(jobs))()
    for i, (W, x, y) in enumerate(jobs):
        arr[i] = L.ef_hip_job(y if isinstance(y, int) else y.ptr, W.handle, x if isinstance(x, int) else x.ptr)
    return arr


def matvec_jobs(jobs, batch: int = 1, ldx: int | None = None, ldy: int | None = None, stream=None) -> None:
    """jobs: list of (Weight, x, y) with DeviceArray or raw device addresses."""
    arr = _jobs(jobs)
    call("ef_hip_matvec_jobs", arr, len(jobs), batch, ldx or jobs[0][0].cols, ldy or jobs[0][0].rows, _s(stream))


def matvec_jobs_rmsnorm(jobs, norm_w: DeviceArray, eps: float, batch: int = 1, ldx: int | None = None,
                        ldy: int | None = None, stream=None) -> None:
    arr = _jobs(jobs)
    call("ef_hip_matvec_jobs_rmsnorm", arr, len(jobs), norm_w.ptr, eps, batch, ldx or jobs[0][0].cols,
         ldy or jobs[0][0].rows, _s(stream))


def quantize(qtype: int, w: DeviceArray, rows: int, cols: int, search: bool = True, stream=None) -> DeviceArray:
    out = DeviceArray((rows * row_bytes(qtype, cols),), np.uint8)
    call("ef_hip_quantize", qtype, w.ptr, rows, cols, int(search), out.ptr, _s(stream))
    return out


def rows_f32(W: Weight, ids: DeviceArray, out: DeviceArray, batch: int = 1, stream=None) -> None:
    call("ef_hip_rows_f32", W.handle, ids.ptr, batch, out.ptr, W.cols, _s(stream))


def sampler_exp(x: DeviceArray, y: DeviceArray, n: int, stream=None) -> None:
    """y[:n] = exp(x[:n]) on the device, as the sampler's softmax terms are computed (float64 arrays)."""
    call("ef_hip_sampler_exp", x.ptr, y.ptr, n, _s(stream))


def argmax(x: DeviceArray, n: int, out: DeviceArray, batch: int = 1, ld: int | None = None, stream=None) -> None:
    call("ef_hip_argmax", x.ptr, n, batch, ld or n, out.ptr, _s(stream))


class RngStates:
    """std::mt19937_64 states on the device, one per sequence."""

    def __init__(self, seeds):
        seeds = np.ascontiguousarray(np.asarray(seeds, dtype=np.uint64).reshape(-1))
        self.batch = seeds.size
        self.buf = DeviceArray((lib().ef_hip_rng_state_bytes() * self.batch,), np.uint8)
        call("ef_hip_rng_seed", self.buf.ptr, seeds.ctypes.data_as(L._u64p), self.batch, None)


def sample(logits: DeviceArray, vocab: int, cfg: dict, out: DeviceArray, batch: int = 1,
           hist: DeviceArray | None = None, hist_len: DeviceArray | None = None, hist_ld: int = 0,
           rng: RngStates | None = None, ld: int | None = None, ws: DeviceArray | None = None,
           stream=None) -> None:
    c = L.ef_hip_sampler_config(cfg.get("temperature", 0.0), cfg.get("top_k", 0), cfg.get("top_p", 1.0),
                                cfg.get("repetition_penalty", 1.0), cfg.get("seed", 0))
    call("ef_hip_sample", logits.ptr, vocab, batch, ld or vocab, C.byref(c), hist.ptr if hist else None,
         hist_len.ptr if hist_len else None, hist_ld, rng.buf.ptr if rng else None, out.ptr,
         ws.ptr if ws else None, _s(stream))
