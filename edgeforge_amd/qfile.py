"""The .efq model file and Model::load_efq over the C-ABI (include/ef_hip.h, .efq section).

    QuantFile.open(path)      ef::QuantFile::open (include/ef/qfile.h:98, src/qfile.cpp:225-243)
    QuantFile.parse(buf)      ef::parse_efq (include/ef/qfile.h:133, src/qfile.cpp:125-223)
    EfqModel.load_efq(path)   ef::Model::load_efq (src/model.cpp:66-111), weights copied to the GPU

Reading and validating a file is host-only (no GPU); a rejected file raises HipError with the
reader's message, where the reference throws ef::Error with the same wording.  There is no CPU
fallback for the model: EfqModel needs the HIP library and a device.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib as EL
from .model import Config, Engine


@dataclass(frozen=True)
class QTensor:
    """ef::QTensor (include/ef/qfile.h:80-92)."""
    name: str
    type: int
    rule: str
    shape: tuple
    offset: int
    bytes: int
    rel_rmse: float
    max_abs_err: float

    def rows(self) -> int:
        return self.shape[0] if len(self.shape) == 2 else 1

    def cols(self) -> int:
        return self.shape[-1] if self.shape else 0


class QuantFile:
    """A validated .efq file: memory-mapped (open) or over a bytes object (parse)."""

    def __init__(self, handle: int, keep=None):
        self.h = handle
        self._keep = keep  # the buffer a parsed handle points into
        n = C.c_size_t()
        EL.call("ef_hip_efq_tensor_count", self.h, C.byref(n))
        self._tensors, self._ptrs = [], []
        for i in range(n.value):
            t = EL.ef_hip_efq_tensor()
            EL.call("ef_hip_efq_tensor_info", self.h, i, C.byref(t))
            shape = (t.rows, t.cols) if t.ndim == 2 else (t.cols,)
            self._tensors.append(QTensor(t.name.decode(), t.qtype, t.rule.decode(), shape, t.offset, t.bytes,
                                         t.rel_rmse, t.max_abs_err))
            self._ptrs.append(t.host_data)
        self._index = {t.name: i for i, t in enumerate(self._tensors)}

    @classmethod
    def open(cls, path: str) -> "QuantFile":
        h = C.c_void_p()
        EL.call("ef_hip_efq_open", str(path).encode(), C.byref(h))
        return cls(h.value)

    @classmethod
    def parse(cls, data: bytes) -> "QuantFile":
        buf = C.create_string_buffer(bytes(data), len(data))
        h = C.c_void_p()
        EL.call("ef_hip_efq_parse", buf, len(data), C.byref(h))
        return cls(h.value, keep=buf)

    def config(self) -> dict:
        """ModelConfig fields (include/ef/model_config.h:14-38) the decode path uses."""
        c, tied, bos, eos = EL.ef_hip_model_config(), C.c_int(), C.c_int64(), C.c_int64()
        EL.call("ef_hip_efq_config", self.h, C.byref(c), C.byref(tied), C.byref(bos), C.byref(eos))
        return {"D": c.D, "F": c.F, "H": c.H, "KV": c.KV, "hd": c.hd, "V": c.V, "L": c.L, "max_pos": c.max_pos,
                "eps": c.eps, "rope_theta": c.rope_theta, "tie_word_embeddings": bool(tied.value),
                "bos_token_id": bos.value, "eos_token_id": eos.value}

    def policy(self) -> dict:
        """QuantPolicy (include/ef/qfile.h:53-59): layer / lm_head / embed types, overrides, name."""
        la, lm, em, no = C.c_int(), C.c_int(), C.c_int(), C.c_size_t()
        name = C.create_string_buffer(256)
        EL.call("ef_hip_efq_policy", self.h, C.byref(la), C.byref(lm), C.byref(em), C.byref(no), name, 256)
        return {"layers": la.value, "lm_head": lm.value, "embed": em.value, "n_overrides": no.value,
                "name": name.value.decode()}

    def tensors(self) -> list[QTensor]:
        return list(self._tensors)

    def find(self, name: str) -> QTensor | None:
        i = self._index.get(name)
        return None if i is None else self._tensors[i]

    def at(self, name: str) -> QTensor:
        idx = C.c_size_t()
        EL.call("ef_hip_efq_find", self.h, name.encode(), C.byref(idx))
        return self._tensors[idx.value]

    def data(self, t: QTensor) -> np.ndarray:
        """A copy of the tensor's bytes as stored in the file."""
        p = self._ptrs[self._index[t.name]]
        return np.ctypeslib.as_array((C.c_uint8 * t.bytes).from_address(p)).copy() if t.bytes else np.empty(0, np.uint8)

    def bytes_per_token(self) -> int:
        out = C.c_uint64()
        EL.call("ef_hip_efq_bytes_per_token", self.h, C.byref(out))
        return out.value

    def close(self) -> None:
        if getattr(self, "h", None):
            EL.call("ef_hip_efq_close", self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class EfqModel:
    """Model::load_efq on the device: every tensor of the file in one HBM arena."""

    def __init__(self, handle: int):
        self.h = handle
        c, tied, eos = EL.ef_hip_model_config(), C.c_int(), C.c_int64()
        EL.call("ef_hip_model_config_get", self.h, C.byref(c), C.byref(tied), C.byref(eos))
        self.cfg = Config(D=c.D, F=c.F, H=c.H, KV=c.KV, hd=c.hd, V=c.V, L=c.L, max_pos=c.max_pos, eps=c.eps,
                          rope_theta=c.rope_theta)
        self.tied, self.eos_token_id = bool(tied.value), eos.value
        buf = C.create_string_buffer(512)
        EL.call("ef_hip_model_description", self.h, buf, 512)
        self.description = buf.value.decode()
        bpt = C.c_uint64()
        EL.call("ef_hip_model_bytes_per_token", self.h, C.byref(bpt))
        self.bytes_per_token = bpt.value

    @classmethod
    def load_efq(cls, path: str) -> "EfqModel":
        EL.init()
        h = C.c_void_p()
        EL.call("ef_hip_model_load_efq", str(path).encode(), C.byref(h))
        return cls(h.value)

    @classmethod
    def upload(cls, f: QuantFile) -> "EfqModel":
        EL.init()
        h = C.c_void_p()
        EL.call("ef_hip_model_upload", f.h, C.byref(h))
        return cls(h.value)

    def layer_handles(self, l: int) -> EL.ef_hip_layer:
        out = EL.ef_hip_layer()
        EL.call("ef_hip_model_layer", self.h, l, C.byref(out))
        return out

    def engine(self, max_seq: int, batch: int = 1) -> Engine:
        return Engine(self, max_seq, batch)

    def free(self) -> None:
        if getattr(self, "h", None):
            EL.call("ef_hip_model_free", self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
