"""GGUF files through the library's reader (kf_gguf_*, include/kf_hip.h): the format the reference's loader reads
(crates/kf-gguf/src/lib.rs), so real model tensors reach the quantized products with their bytes unchanged."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import KfError, KF_E_INVALID, last_error, lib

MAX_DIMS = 16


@dataclass(frozen=True)
class TensorInfo:
    """TensorInfo (crates/kf-gguf/src/lib.rs:145-161): dims innermost first, as ggml stores ne."""

    name: str
    dims: tuple
    ggml_type: int
    shard: int
    offset: int
    nbytes: int  # -1: a type without a known block layout, or dims that do not fit it

    @property
    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


class GGUF:
    """An open GGUF file (and its sibling shards). Tensor data are views into the library's read-only maps, valid until
    close(): copy them (np.array(...)) to keep them longer."""

    def __init__(self, path: str):
        self._L = lib()
        self._h = self._L.kf_gguf_open(str(path).encode())
        if not self._h:
            raise KfError(KF_E_INVALID, last_error())
        self.tensors = [self._info(i) for i in range(self._L.kf_gguf_n_tensors(self._h))]
        self._by_name = {t.name: i for i, t in enumerate(self.tensors)}
        self.meta = {k: v for k, v in self._meta()}

    def close(self) -> None:
        if self._h:
            self._L.kf_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def n_shards(self) -> int:
        return self._L.kf_gguf_n_shards(self._h)

    def tensor(self, name: str) -> TensorInfo | None:
        i = self._by_name.get(name)
        return None if i is None else self.tensors[i]

    def data(self, name: str):
        """The tensor's bytes as a read-only numpy uint8 view of the map (Gguf::bytes)."""
        import numpy as np

        i = self._by_name.get(name)
        if i is None:
            raise KfError(KF_E_INVALID, f"no tensor {name}")
        p = self._L.kf_gguf_tensor_data(self._h, i)
        if not p:
            raise KfError(KF_E_INVALID, last_error())
        n = self.tensors[i].nbytes
        buf = (ctypes.c_uint8 * n).from_address(p)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def _info(self, i: int) -> TensorInfo:
        name = ctypes.c_char_p()
        dims = (ctypes.c_int64 * MAX_DIMS)()
        ty, shard = ctypes.c_uint32(), ctypes.c_int()
        off, nb = ctypes.c_uint64(), ctypes.c_int64()
        nd = self._L.kf_gguf_tensor_info(self._h, i, ctypes.byref(name), dims, MAX_DIMS, ctypes.byref(ty), ctypes.byref(shard),
                                         ctypes.byref(off), ctypes.byref(nb))
        if nd < 0:
            raise KfError(nd, last_error())
        return TensorInfo(name.value.decode("utf-8", "replace"), tuple(dims[:nd]), ty.value, shard.value, off.value, nb.value)

    def _scalar(self, i: int, kind: int, idx: int):
        L, h = self._L, self._h
        if kind in (6, 12):
            v = ctypes.c_double()
            rc = L.kf_gguf_kv_f64(h, i, idx, ctypes.byref(v))
            out = v.value
        elif kind == 8:
            s, n = ctypes.c_void_p(), ctypes.c_uint64()
            rc = L.kf_gguf_kv_str(h, i, idx, ctypes.byref(s), ctypes.byref(n))
            out = ctypes.string_at(s, n.value).decode("utf-8", "replace") if rc == 0 else None
        elif kind == 7:
            v = ctypes.c_uint64()
            rc = L.kf_gguf_kv_u64(h, i, idx, ctypes.byref(v))
            out = bool(v.value)
        elif kind in (1, 3, 5, 11):
            v = ctypes.c_int64()
            rc = L.kf_gguf_kv_i64(h, i, idx, ctypes.byref(v))
            out = v.value
        else:
            v = ctypes.c_uint64()
            rc = L.kf_gguf_kv_u64(h, i, idx, ctypes.byref(v))
            out = v.value
        if rc != 0:
            raise KfError(rc, last_error())
        return out

    def _meta(self):
        L, h = self._L, self._h
        for i in range(L.kf_gguf_n_kv(h)):
            key = ctypes.c_char_p()
            kind, elem, count = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
            rc = L.kf_gguf_kv(h, i, ctypes.byref(key), ctypes.byref(kind), ctypes.byref(elem), ctypes.byref(count))
            if rc != 0:
                raise KfError(rc, last_error())
            if kind.value == 9:
                # arrays of scalars; nested arrays are kept by the reader but not flattened here
                value = [self._scalar(i, elem.value, k) for k in range(count.value)] if elem.value != 9 else None
            else:
                value = self._scalar(i, kind.value, 0)
            yield key.value.decode("utf-8", "replace"), value
