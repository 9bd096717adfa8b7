"""ctypes binding of libedgeforge_hip.so (include/ef_hip.h).

The product path: loading fails loudly (ImportError-like RuntimeError) when the library is absent;
there is no CPU fallback.  Every call checks the returned status and raises HipError with the
library's message.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libedgeforge_hip.so")

F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 3, 4
QTYPE_NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q8_0: "Q8_0", Q4_0: "Q4_0"}

OK, EINVAL, ERUNTIME, ENODEV, ENOMEM, ESTATE = 0, -1, -2, -3, -4, -5

_P = C.c_void_p
_sz = C.c_size_t
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u64p = C.POINTER(C.c_uint64)


class HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ef_hip_job(C.Structure):
    _fields_ = [("y_dev", _P), ("W", _P), ("x_dev", _P)]


class ef_hip_sampler_config(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float), ("seed", C.c_uint64)]


class ef_hip_model_config(C.Structure):
    _fields_ = [(n, _sz) for n in ("D", "F", "H", "KV", "hd", "V", "L", "max_pos")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float)]


class ef_hip_layer(C.Structure):
    _fields_ = [(n, _P) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")] + \
               [("attn_norm_dev", _P), ("ffn_norm_dev", _P)]


class ef_hip_efq_tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("rule", C.c_char_p), ("qtype", C.c_int), ("ndim", C.c_int),
                ("rows", _sz), ("cols", _sz), ("offset", C.c_uint64), ("bytes", C.c_uint64),
                ("rel_rmse", C.c_double), ("max_abs_err", C.c_double), ("host_data", _P)]


class ef_hip_membench_options(C.Structure):
    _fields_ = [("buffer_bytes", C.c_uint64), ("runs", C.c_int), ("passes", C.c_int), ("warmup_runs", C.c_int)]


class ef_hip_membench_result(C.Structure):
    _fields_ = [("buffer_bytes", C.c_uint64), ("passes", C.c_int), ("bytes_per_run", C.c_uint64),
                ("best_gbps", C.c_double), ("median_gbps", C.c_double), ("worst_gbps", C.c_double),
                ("checksum", C.c_uint64), ("expected_checksum", C.c_uint64), ("checksum_ok", C.c_int)]


class ef_hip_reply_options(C.Structure):
    _fields_ = [("max_new", _sz), ("eos_id", C.c_int32), ("eos_min_p", C.c_float), ("steps_per_check", C.c_int)]


class ef_hip_reply_stats(C.Structure):
    _fields_ = [("prompt_tokens", _sz), ("reused_tokens", _sz), ("prefill_tokens", _sz), ("generated", _sz),
                ("steps", _sz), ("reason", C.c_int), ("prefill_s", C.c_double), ("decode_s", C.c_double),
                ("eos_p_max", C.c_double), ("eos_p_max_step", _sz)]


STOP_NONE, STOP_EOS, STOP_EOS_MIN_P, STOP_MAX_NEW, STOP_CONTEXT = 0, 1, 2, 5, 6


class ef_hip_dist_stats(C.Structure):
    _fields_ = [("n", _sz), ("top1", _sz), ("confident", _sz), ("confident_top1", _sz), ("nonfinite", _sz),
                ("kl_sum", C.c_double), ("kl_max", C.c_double), ("kl_mean", C.c_double)]

# name -> (restype, argtypes); every entry point declared in include/ef_hip.h
SIGNATURES = {
    "ef_hip_init": (C.c_int, [C.c_int]),
    "ef_hip_shutdown": (C.c_int, []),
    "ef_hip_last_error": (C.c_char_p, []),
    "ef_hip_device_name": (C.c_int, [C.c_char_p, _sz]),
    "ef_hip_version": (C.c_int, [C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "ef_hip_malloc": (C.c_int, [C.POINTER(_P), _sz]),
    "ef_hip_free": (C.c_int, [_P]),
    "ef_hip_memcpy_h2d": (C.c_int, [_P, _P, _sz, _P]),
    "ef_hip_memcpy_d2h": (C.c_int, [_P, _P, _sz, _P]),
    "ef_hip_memcpy_d2d": (C.c_int, [_P, _P, _sz, _P]),
    "ef_hip_memset": (C.c_int, [_P, C.c_int, _sz, _P]),
    "ef_hip_stream_create": (C.c_int, [C.POINTER(_P)]),
    "ef_hip_stream_destroy": (C.c_int, [_P]),
    "ef_hip_stream_sync": (C.c_int, [_P]),
    "ef_hip_pointer_kind": (C.c_int, [_P, C.POINTER(C.c_int)]),
    "ef_hip_event_create": (C.c_int, [C.POINTER(_P)]),
    "ef_hip_event_destroy": (C.c_int, [_P]),
    "ef_hip_event_record": (C.c_int, [_P, _P]),
    "ef_hip_event_elapsed_ms": (C.c_int, [_P, _P, _f32p]),
    "ef_hip_weight_register_host": (C.c_int, [_P, C.c_int, _sz, _sz, C.POINTER(_P)]),
    "ef_hip_weight_register_device": (C.c_int, [_P, C.c_int, _sz, _sz, C.POINTER(_P)]),
    "ef_hip_weight_release": (C.c_int, [_P]),
    "ef_hip_weight_refresh": (C.c_int, [_P, _P]),
    "ef_hip_weight_info": (C.c_int, [_P, C.POINTER(C.c_int), C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_P)]),
    "ef_hip_row_bytes": (C.c_int, [C.c_int, _sz, C.POINTER(_sz)]),
    "ef_hip_matvec": (C.c_int, [_P, _P, _P, C.c_int, _sz, _sz, _P]),
    "ef_hip_matvec_jobs": (C.c_int, [C.POINTER(ef_hip_job), _sz, C.c_int, _sz, _sz, _P]),
    "ef_hip_matvec_residual": (C.c_int, [_P, _P, _P, C.c_int, _sz, _sz, _P]),
    "ef_hip_matvec_swiglu": (C.c_int, [_P, _P, _P, _P, C.c_float, _P, C.c_int, _sz, _sz, _P]),
    "ef_hip_matvec_jobs_rmsnorm": (C.c_int, [C.POINTER(ef_hip_job), _sz, _P, C.c_float, C.c_int, _sz, _sz, _P]),
    "ef_hip_rows_f32": (C.c_int, [_P, _P, C.c_int, _P, _sz, _P]),
    "ef_hip_quantize": (C.c_int, [C.c_int, _P, _sz, _sz, C.c_int, _P, _P]),
    "ef_hip_fill_normal": (C.c_int, [_P, _sz, C.c_uint64, C.c_uint64, C.c_float, C.c_float, _P]),
    "ef_hip_rng_state_bytes": (_sz, []),
    "ef_hip_rng_seed": (C.c_int, [_P, _u64p, C.c_int, _P]),
    "ef_hip_sample_workspace_bytes": (_sz, [_sz, C.c_int]),
    "ef_hip_sample": (C.c_int, [_P, _sz, C.c_int, _sz, C.POINTER(ef_hip_sampler_config), _P, _P, _sz, _P, _P, _P,
                                _P]),
    "ef_hip_sample_noalloc": (C.c_int, [_P, _sz, C.c_int, _sz, C.POINTER(ef_hip_sampler_config), _P, _P, _sz, _P,
                                        _P, _P]),
    "ef_hip_argmax": (C.c_int, [_P, _sz, C.c_int, _sz, _P, _P]),
    "ef_hip_sampler_exp": (C.c_int, [_P, _P, _sz, _P]),
    "ef_hip_profile_matvec": (C.c_int, [C.c_int, C.POINTER(_P), C.POINTER(_P), _sz, _P, _P, C.c_float, _P, C.c_int,
                                        C.c_int, _P, _f32p]),
    "ef_hip_engine_create": (C.c_int, [C.POINTER(ef_hip_model_config), C.POINTER(ef_hip_layer), _P, _P, _P, _sz,
                                       C.c_int, C.POINTER(_P)]),
    "ef_hip_engine_destroy": (C.c_int, [_P]),
    "ef_hip_engine_profile": (C.c_int, [_P, C.POINTER(ef_hip_sampler_config), _P, C.c_int,
                                        C.POINTER(C.c_double)]),
    "ef_hip_engine_tables": (C.c_int, [_P, C.POINTER(C.c_int), C.POINTER(C.c_char_p)]),
    "ef_hip_engine_forward": (C.c_int, [_P, _i32p, _sz, C.c_int]),
    "ef_hip_engine_prefill": (C.c_int, [_P, _i32p, _sz, _sz, C.c_int]),
    "ef_hip_engine_logits": (C.c_int, [_P, C.POINTER(_P)]),
    "ef_hip_engine_hidden": (C.c_int, [_P, C.POINTER(_P)]),
    "ef_hip_engine_generate": (C.c_int, [_P, _i32p, _sz, _sz, C.POINTER(ef_hip_sampler_config), _P, _i32p,
                                         C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "ef_hip_membench": (C.c_int, [C.POINTER(ef_hip_membench_options), C.POINTER(ef_hip_membench_result)]),
    "ef_hip_membench_expected_pass_sum": (C.c_uint64, [C.c_uint64]),
    "ef_hip_engine_reply": (C.c_int, [_P, _i32p, _sz, C.POINTER(ef_hip_sampler_config), _P,
                                      C.POINTER(ef_hip_reply_options), _i32p, C.POINTER(C.c_double),
                                      C.POINTER(ef_hip_reply_stats)]),
    "ef_hip_engine_reset": (C.c_int, [_P]),
    "ef_hip_engine_score": (C.c_int, [_P, _i32p, _sz, _sz, C.POINTER(C.c_double), _P]),
    "ef_hip_compare_dist": (C.c_int, [_P, _P, _sz, _sz, _sz, _sz, C.POINTER(C.c_double), C.POINTER(ef_hip_dist_stats),
                                      _P]),
    "ef_hip_neg_log_prob": (C.c_int, [_P, _sz, _sz, _sz, _P, _P, _P]),
    "ef_hip_efq_open": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "ef_hip_efq_parse": (C.c_int, [_P, _sz, C.POINTER(_P)]),
    "ef_hip_efq_close": (C.c_int, [_P]),
    "ef_hip_efq_config": (C.c_int, [_P, C.POINTER(ef_hip_model_config), C.POINTER(C.c_int),
                                    C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "ef_hip_efq_tensor_count": (C.c_int, [_P, C.POINTER(_sz)]),
    "ef_hip_efq_tensor_info": (C.c_int, [_P, _sz, C.POINTER(ef_hip_efq_tensor)]),
    "ef_hip_efq_find": (C.c_int, [_P, C.c_char_p, C.POINTER(_sz)]),
    "ef_hip_efq_bytes_per_token": (C.c_int, [_P, _u64p]),
    "ef_hip_efq_policy": (C.c_int, [_P, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int),
                                    C.POINTER(_sz), C.c_char_p, _sz]),
    "ef_hip_model_load_efq": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "ef_hip_model_upload": (C.c_int, [_P, C.POINTER(_P)]),
    "ef_hip_model_free": (C.c_int, [_P]),
    "ef_hip_model_config_get": (C.c_int, [_P, C.POINTER(ef_hip_model_config), C.POINTER(C.c_int),
                                          C.POINTER(C.c_int64)]),
    "ef_hip_model_description": (C.c_int, [_P, C.c_char_p, _sz]),
    "ef_hip_model_bytes_per_token": (C.c_int, [_P, _u64p]),
    "ef_hip_model_layer": (C.c_int, [_P, _sz, C.POINTER(ef_hip_layer)]),
    "ef_hip_model_tensors": (C.c_int, [_P, C.POINTER(_P), C.POINTER(_P), C.POINTER(_P)]),
    "ef_hip_model_engine_create": (C.c_int, [_P, _sz, C.c_int, C.POINTER(_P)]),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function name include/ef_hip.h declares (parsed from the header text)."""
    import re
    root = os.path.dirname(HERE)
    text = open(os.path.join(root, "include", "ef_hip.h")).read()
    return sorted(set(re.findall(r"\b(ef_hip_[a-z0-9_]+)\s*\(", text)))


def lib() -> C.CDLL:
    """The loaded library; raises when it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m edgeforge_amd.build` "
                               "(the HIP path has no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name, None)
            if f is None:
                continue
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().ef_hip_last_error()
        raise HipError(rc, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


_inited = False


def init(device: int = 0) -> None:
    global _inited
    if not _inited:
        call("ef_hip_init", device)
        _inited = True


def device_name() -> str:
    buf = C.create_string_buffer(256)
    call("ef_hip_device_name", buf, 256)
    return buf.value.decode()
