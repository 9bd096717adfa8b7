"""ctypes binding of the CPU oracle (liboracle.so) and of the reference build (_ref/libefref.so).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or as the timed CPU
baseline; the product package ``edgeforge_amd`` never imports it.

``lib()`` is the plain-C restatement (oracle/efo_*.c, one reference file:line per function).
``ref()`` is the reference's own sources compiled from /root/reference (oracle/Makefile, target
``ref``); it is ``None`` where that library was not built (e.g. on the GPU box when
/root/reference was absent at build time).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 3, 4
SCALAR, AVX2 = 0, 1
QK = 32
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34}

_P = C.c_void_p
_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_i32p = C.POINTER(C.c_int32)
_u64p = C.POINTER(C.c_uint64)
_f64p = C.POINTER(C.c_double)
_sz = C.c_size_t


def build(with_ref: bool = True) -> None:
    """Compile liboracle.so (always) and _ref/libefref.so (when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if with_ref and os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def ptr(a: np.ndarray, t=C.c_void_p):
    return a.ctypes.data_as(t)


class efo_weight(C.Structure):
    _fields_ = [("qtype", C.c_int), ("data", _u8p), ("rows", _sz), ("cols", _sz)]


class efo_job(C.Structure):
    _fields_ = [("y", _f32p), ("W", C.POINTER(efo_weight)), ("x", _f32p)]


class efo_sampler_config(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float), ("seed", C.c_uint64)]


class efo_config(C.Structure):
    _fields_ = [(n, _sz) for n in ("D", "F", "H", "KV", "hd", "V", "L", "max_pos")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float)]


class efo_layer(C.Structure):
    _fields_ = [(n, efo_weight) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")] + \
               [("attn_norm", _f32p), ("ffn_norm", _f32p)]


class efo_model(C.Structure):
    _fields_ = [("cfg", efo_config), ("embed", efo_weight), ("lm_head", efo_weight),
                ("final_norm", _f32p), ("layers", C.POINTER(efo_layer))]


_LIB = None
_REF = None


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build(with_ref=False)
        L = C.CDLL(path)
        _sig(L, "efo_fp16_to_f32", C.c_float, C.c_uint16)
        _sig(L, "efo_f32_to_fp16", C.c_uint16, C.c_float)
        _sig(L, "efo_bf16_to_f32", C.c_float, C.c_uint16)
        _sig(L, "efo_f32_to_bf16", C.c_uint16, C.c_float)
        _sig(L, "efo_fp16_to_f32_n", None, _u16p, _f32p, _sz)
        _sig(L, "efo_f32_to_fp16_n", None, _f32p, _u16p, _sz)
        _sig(L, "efo_f32_to_bf16_n", None, _f32p, _u16p, _sz)
        _sig(L, "efo_row_bytes", C.c_int, C.c_int, C.c_uint64, _u64p)
        _sig(L, "efo_quantize_row", C.c_int, C.c_int, _f32p, _sz, _u8p, C.c_int)
        _sig(L, "efo_dequantize_row", C.c_int, C.c_int, _u8p, _sz, _f32p)
        _sig(L, "efo_quantize_matrix", C.c_int, C.c_int, _f32p, _sz, _sz, _u8p, C.c_int, C.c_int)
        _sig(L, "efo_fake_quant_q4_group", None, _f32p, _sz, _f32p, C.c_int)
        for n in ("efo_dot_q4_0", "efo_dot_q8_0", "efo_dot_q4_0_avx2", "efo_dot_q8_0_avx2"):
            _sig(L, n, C.c_float, _u8p, _f32p, _sz)
        _sig(L, "efo_dot_f32", C.c_float, _f32p, _f32p, _sz)
        _sig(L, "efo_pool_create", _P, C.c_uint)
        _sig(L, "efo_pool_destroy", None, _P)
        _sig(L, "efo_pool_size", C.c_uint, _P)
        _sig(L, "efo_pool_chunk_begin", _sz, _sz, C.c_uint, C.c_uint)
        _sig(L, "efo_matvec_rows", None, C.c_int, _f32p, C.POINTER(efo_weight), _f32p, _sz, _sz)
        _sig(L, "efo_matvec_jobs", None, C.c_int, C.POINTER(efo_job), _sz, _P)
        _sig(L, "efo_matvec", None, C.c_int, _f32p, C.POINTER(efo_weight), _f32p, _P)
        _sig(L, "efo_row_f32", None, _f32p, C.POINTER(efo_weight), _sz)
        _sig(L, "efo_rmsnorm", None, _f32p, _f32p, _f32p, _sz, C.c_float)
        _sig(L, "efo_softmax_inplace", None, _f32p, _sz)
        _sig(L, "efo_silu", C.c_float, C.c_float)
        _sig(L, "efo_swiglu", None, _f32p, _f32p, _f32p, _sz)
        _sig(L, "efo_embedding_bf16", None, _f32p, _u16p, _sz, _sz)
        _sig(L, "efo_argmax", _sz, _f32p, _sz)
        _sig(L, "efo_rope_table", None, _f32p, _f32p, _f32p, _sz, _sz, C.c_float)
        _sig(L, "efo_rope_apply", None, _f32p, _sz, _sz, _f32p, _f32p)
        _sig(L, "efo_attention_heads", None, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p, _sz, _sz)
        _sig(L, "efo_mt64_seed", None, _P, C.c_uint64)
        _sig(L, "efo_mt64_next", C.c_uint64, _P)
        _sig(L, "efo_canonical_double", C.c_double, _P)
        _sig(L, "efo_sampler_create", _P, C.POINTER(efo_sampler_config))
        _sig(L, "efo_sampler_destroy", None, _P)
        _sig(L, "efo_sampler_sample", C.c_int32, _P, _f32p, _sz, _i32p, _sz)
        _sig(L, "efo_sampler_last_keep", _sz, _P, _i32p, _f64p, _sz)
        _sig(L, "efo_sampler_last_r", C.c_double, _P)
        _sig(L, "efo_exp_array", None, _f64p, _f64p, _sz)
        _sig(L, "efo_transformer_create", _P, C.POINTER(efo_model), _sz, _P, C.c_int)
        _sig(L, "efo_transformer_destroy", None, _P)
        _sig(L, "efo_transformer_forward", _f32p, _P, C.c_int32, _sz, C.c_int, C.POINTER(C.c_int))
        _sig(L, "efo_transformer_hidden", _f32p, _P)
        _sig(L, "efo_run_once", C.c_int, C.POINTER(efo_model), _i32p, _sz, _sz, _P, C.c_int, _i32p, _f32p,
             _f64p, _f64p)
        _LIB = L
    return _LIB


def ref_available() -> bool:
    """Whether the reference build exists, without loading it (test collection stays load-free)."""
    return os.path.exists(os.path.join(HERE, "_ref", "libefref.so"))


def ref():
    """The reference build, or None when oracle/_ref/libefref.so is absent.  Loaded on first call."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libefref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        _sig(R, "ref_fp16_to_f32", C.c_float, C.c_uint16)
        _sig(R, "ref_f32_to_fp16", C.c_uint16, C.c_float)
        _sig(R, "ref_bf16_to_f32", C.c_float, C.c_uint16)
        _sig(R, "ref_f32_to_bf16", C.c_uint16, C.c_float)
        _sig(R, "ref_row_bytes", C.c_int, C.c_int, C.c_uint64, _u64p)
        _sig(R, "ref_quantize_row", C.c_int, C.c_int, _f32p, _sz, _P, C.c_int)
        _sig(R, "ref_dequantize_row", C.c_int, C.c_int, _P, _sz, _f32p)
        _sig(R, "ref_fake_quant_q4_group", None, _f32p, _sz, _f32p, C.c_int)
        for n in ("ref_dot_q4_0", "ref_dot_q8_0", "ref_dot_q4_0_avx2", "ref_dot_q8_0_avx2"):
            _sig(R, n, C.c_float, _u8p, _f32p, _sz)
        _sig(R, "ref_avx2_compiled", C.c_int)
        _sig(R, "ref_matvec_jobs", C.c_int, C.c_int, C.c_int, C.POINTER(_f32p), _i32p, C.POINTER(_u8p), C.POINTER(_sz),
             C.POINTER(_sz), C.POINTER(_f32p), C.c_uint)
        _sig(R, "ref_sampler_create", _P, C.c_float, C.c_int, C.c_float, C.c_float, C.c_uint64)
        _sig(R, "ref_sampler_destroy", None, _P)
        _sig(R, "ref_sampler_sample", C.c_int, _P, _f32p, _sz, _i32p, _sz, _i32p)
        _sig(R, "ref_mt64_words", None, C.c_uint64, _sz, _u64p)
        _sig(R, "ref_uniform_doubles", None, C.c_uint64, _sz, _f64p)
        _sig(R, "ref_rmsnorm", None, _f32p, _f32p, _f32p, _sz, C.c_float)
        _sig(R, "ref_softmax", None, _f32p, _sz)
        _sig(R, "ref_silu", C.c_float, C.c_float)
        _sig(R, "ref_swiglu", None, _f32p, _f32p, _f32p, _sz)
        _sig(R, "ref_argmax", _sz, _f32p, _sz)
        _sig(R, "ref_dot_f32", C.c_float, _f32p, _f32p, _sz)
        _sig(R, "ref_rope_table", None, _f32p, _f32p, _f32p, _sz, _sz, C.c_float)
        _sig(R, "ref_rope_apply", None, _f32p, _sz, _sz, _f32p, _f32p)
        _sig(R, "ref_attention", None, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p)
        _sig(R, "ref_engine_open", _P, C.c_char_p, _sz, C.c_uint, C.c_int)
        _sig(R, "ref_engine_close", None, _P)
        _sig(R, "ref_engine_bytes_per_token", C.c_uint64, _P)
        _sig(R, "ref_engine_forward", C.c_int, _P, C.c_int32, _sz, C.c_int, _f32p)
        _sig(R, "ref_efq_parse", C.c_long, _P, _sz, C.c_char_p, _sz)
        _sig(R, "ref_model_load_efq", C.c_long, C.c_char_p, C.POINTER(C.c_uint64), C.c_char_p, _sz)
        _REF = R
    return _REF


# ---------------------------------------------------------------------------------- helpers

def row_bytes(qtype: int, cols: int) -> int:
    out = C.c_uint64()
    if lib().efo_row_bytes(qtype, cols, C.byref(out)) != 0:
        raise ValueError(f"type {qtype} needs a row length divisible by 32, got {cols}")
    return out.value


def quantize(qtype: int, w: np.ndarray, search: bool = True, threads: int = 8) -> np.ndarray:
    """Row-major [rows, cols] float32 -> packed bytes [rows, row_bytes] (src/quant.cpp:182)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.empty((rows, row_bytes(qtype, cols)), dtype=np.uint8)
    rc = lib().efo_quantize_matrix(qtype, ptr(w, _f32p), rows, cols, ptr(out, _u8p), int(search), threads)
    assert rc == 0
    return out


def dequantize(qtype: int, packed: np.ndarray, cols: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1, row_bytes(qtype, cols))
    out = np.empty((packed.shape[0], cols), dtype=np.float32)
    for r in range(packed.shape[0]):
        assert lib().efo_dequantize_row(qtype, ptr(packed[r], _u8p), cols, ptr(out[r], _f32p)) == 0
    return out


def weight(qtype: int, packed: np.ndarray, rows: int, cols: int) -> efo_weight:
    return efo_weight(qtype, ptr(packed, _u8p), rows, cols)


class Pool:
    """The restated persistent thread pool (src/threadpool.cpp)."""

    def __init__(self, threads: int):
        self.h = lib().efo_pool_create(threads)

    def close(self):
        if self.h:
            lib().efo_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


def matvec(qtype: int, packed: np.ndarray, x: np.ndarray, backend: int = AVX2, pool: Pool | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[0]
    rows = packed.size // row_bytes(qtype, cols)
    w = weight(qtype, packed, rows, cols)
    y = np.empty(rows, dtype=np.float32)
    lib().efo_matvec(backend, ptr(y, _f32p), C.byref(w), ptr(x, _f32p), pool.h if pool else None)
    return y


def matvec_jobs(jobs, backend: int = AVX2, pool: Pool | None = None):
    """jobs: list of (qtype, packed, x); returns the list of y."""
    ws, ys, keep = [], [], []
    for qtype, packed, x in jobs:
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows = packed.size // row_bytes(qtype, x.shape[0])
        ws.append(weight(qtype, packed, rows, x.shape[0]))
        ys.append(np.empty(rows, dtype=np.float32))
        keep.append(x)
    arr = (efo_job * len(jobs))()
    for i in range(len(jobs)):
        arr[i] = efo_job(ptr(ys[i], _f32p), C.pointer(ws[i]), ptr(keep[i], _f32p))
    lib().efo_matvec_jobs(backend, arr, len(jobs), pool.h if pool else None)
    return ys


def exp_array(x: np.ndarray) -> np.ndarray:
    """exp of every element through the host libm (the softmax-term call, src/sampler.cpp:46)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x)
    lib().efo_exp_array(ptr(x, _f64p), ptr(y, _f64p), x.size)
    return y


class Sampler:
    """The restated ef::Sampler (include/ef/sampler.h:21-35)."""

    def __init__(self, temperature=0.0, top_k=0, top_p=1.0, repetition_penalty=1.0, seed=0):
        cfg = efo_sampler_config(temperature, top_k, top_p, repetition_penalty, seed)
        self.h = lib().efo_sampler_create(C.byref(cfg))

    def sample(self, logits: np.ndarray, history=()) -> int:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        hist = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
        tok = lib().efo_sampler_sample(self.h, ptr(logits, _f32p), logits.size, ptr(hist, _i32p), hist.size)
        if tok < 0:
            raise ValueError("sampler: empty vocabulary")
        return tok

    def last_keep(self):
        n = lib().efo_sampler_last_keep(self.h, None, None, 0)
        ids = np.empty(n, dtype=np.int32)
        probs = np.empty(n, dtype=np.float64)
        lib().efo_sampler_last_keep(self.h, ptr(ids, _i32p), ptr(probs, _f64p), n)
        return ids, probs

    def last_r(self) -> float:
        return lib().efo_sampler_last_r(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            lib().efo_sampler_destroy(self.h)
            self.h = None


class RefSampler:
    """The reference's own ef::Sampler, from oracle/_ref."""

    def __init__(self, temperature=0.0, top_k=0, top_p=1.0, repetition_penalty=1.0, seed=0):
        self.h = ref().ref_sampler_create(temperature, top_k, top_p, repetition_penalty, seed)

    def sample(self, logits: np.ndarray, history=()) -> int:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        hist = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
        out = C.c_int32()
        if ref().ref_sampler_sample(self.h, ptr(logits, _f32p), logits.size, ptr(hist, _i32p), hist.size,
                                    C.byref(out)) != 0:
            raise ValueError("sampler: empty vocabulary")
        return out.value

    def __del__(self):
        if getattr(self, "h", None):
            ref().ref_sampler_destroy(self.h)
            self.h = None


def ref_matvec_jobs(jobs, backend: int = AVX2, threads: int = 1):
    """The reference's kern::matvec_jobs over (qtype, packed, x) jobs."""
    n = len(jobs)
    ys, xs, keep = [], [], []
    types = np.array([j[0] for j in jobs], dtype=np.int32)
    rows = (_sz * n)()
    cols = (_sz * n)()
    data = (_u8p * n)()
    yp = (_f32p * n)()
    xp = (_f32p * n)()
    for i, (qtype, packed, x) in enumerate(jobs):
        x = np.ascontiguousarray(x, dtype=np.float32)
        r = packed.size // row_bytes(qtype, x.shape[0])
        y = np.empty(r, dtype=np.float32)
        ys.append(y)
        keep.append((x, packed))
        rows[i], cols[i] = r, x.shape[0]
        data[i] = ptr(packed, _u8p)
        yp[i] = ptr(y, _f32p)
        xp[i] = ptr(x, _f32p)
    assert ref().ref_matvec_jobs(backend, n, yp, ptr(types, _i32p), data, rows, cols, xp, threads) == 0
    return ys
