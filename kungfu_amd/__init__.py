"""kungfu_amd — MI355X-native (gfx950) quantized linear-layer hot path of kungfu.

The product is the C-ABI library ``kungfu_amd/lib/libkf_hip.so`` (declared in ``include/kf_hip.h``): hand-written HIP
kernels for the dequant-fused GEMV and the int8 products on GGUF q8_0 / q4_K block bytes, plus a C++ backend object
mirroring kungfu's ``Backend`` trait for ``Op::MatMul``. This module binds it with ctypes for Python callers (tests and
the benchmark), passing torch device tensors as plain device pointers. It never falls back to any CPU path: if the
library is missing, or a call fails, it raises.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "lib", "libkf_hip.so")
HEADER = os.path.join(ROOT, "include", "kf_hip.h")

TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
ACT_Q8_0 = 3
ACT_Q8K = 4
BLOCK = {TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144), TYPE_Q5_K: (256, 176), TYPE_Q6_K: (256, 210)}

KF_OK = 0
KF_E_INVALID = -1
KF_E_UNSUPPORTED = -2
KF_E_HIP = -3
KF_E_NOMEM = -4

_lib = None


class KfError(RuntimeError):
    """A failed kf-hip call: the status code and the library's message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"kf-hip error {code}: {msg}")
        self.code = code


def build(verbose: bool = False) -> str:
    from . import _build

    return _build.build(verbose=verbose)


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (the product path has no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    P, I, U, L64, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_int64, ctypes.c_size_t
    sig = {
        "kf_hip_abi_version": ([], I),
        "kf_hip_last_error": ([], ctypes.c_char_p),
        "kf_hip_act_bytes": ([I, I], S),
        "kf_hip_act_offsets": ([I, I, P], None),
        "kf_hip_act_kind": ([U], I),
        "kf_hip_quant_act": ([P, P, I, I, I, P], I),
        "kf_hip_rms_norm_q8": ([P, P, P, I, I, ctypes.c_float, I, P, P], I),
        "kf_hip_gated_act_q8": ([P, P, I, I, I, I, I, P, P], I),
        "kf_hip_gemv": ([U, P, L64, P, P, P, P, I, I, I, P], I),
        "kf_hip_matmul": ([U, P, I, I, P, I, P, P, P, P, P], I),
        "kf_hip_matmul_noalloc": ([U, P, I, I, P, I, P, P, P, P], I),
        "kf_hip_noalloc_scratch_bytes": ([], S),
        "kf_hip_gemv_group": ([U, P, L64, P, P, I, I, P, I, P], I),
        "kf_hip_matmul_group": ([U, P, I, P, I, P, P, P, I, P], I),
        "kf_hip_block_ints": ([U, P, L64, P, I, I, I, P, P], I),
        "kf_hip_stream_read": ([P, S, I, P, P], I),
        "kf_hip_set_knob": ([ctypes.c_char_p, I], I),
        "kf_hip_release_stream": ([P], I),
        "kf_hip_get_knob": ([ctypes.c_char_p], I),
        "kf_hip_rms_norm_matmul": ([U, P, I, I, P, I, P, P, ctypes.c_float, P, P, P, P, P], I),
        "kf_hip_gemm_i8": ([U, P, L64, P, P, P, P, I, I, I, P], I),
        "kf_hip_moe_group": ([P, I, I, P, P, P], I),
        "kf_hip_moe_gemv": ([U, P, P, L64, L64, P, I, I, I, P, P, I, I, I, P, P], I),
        "kf_hip_moe_combine": ([P, P, P, P, P, I, I, I, ctypes.c_float, P], I),
        "kf_hip_moe_gemm": ([U, P, P, L64, L64, I, P, I, I, I, P, I, P, P, P], I),
        "kf_hip_moe_scratch_bytes": ([I, I, I, I, I], S),
        "kf_hip_moe_ffn": ([U, P, P, P, I, I, I, P, I, P, P, I, ctypes.c_float, P, S, P, P], I),
        "kf_hip_backend_new": ([I], P),
        "kf_hip_backend_free": ([P], None),
        "kf_hip_backend_add_weight": ([P, U, P, I, P, S], I),
        "kf_hip_backend_matmul": ([P, I, P, I, I, P, P], I),
        "kf_hip_backend_matmul_slice": ([P, I, I, P, I, I, P], I),
        "kf_quantize_q8_0": ([P, L64, I, P], I),
        "kf_quantize_q4_k": ([P, L64, I, P], I),
        "kf_quantize_q5_k": ([P, L64, I, P], I),
        "kf_quantize_q6_k": ([P, L64, I, P], I),
        "kf_synth_normal": ([ctypes.c_uint64, ctypes.c_float, P, S], None),
        "kf_gguf_open": ([ctypes.c_char_p], P),
        "kf_gguf_close": ([P], None),
        "kf_gguf_n_shards": ([P], I),
        "kf_gguf_n_tensors": ([P], L64),
        "kf_gguf_find_tensor": ([P, ctypes.c_char_p], L64),
        "kf_gguf_tensor_info": ([P, L64, ctypes.POINTER(ctypes.c_char_p), P, I, P, P, P, P], I),
        "kf_gguf_tensor_data": ([P, L64], P),
        "kf_gguf_n_kv": ([P], L64),
        "kf_gguf_find_kv": ([P, ctypes.c_char_p], L64),
        "kf_gguf_kv": ([P, L64, ctypes.POINTER(ctypes.c_char_p), P, P, P], I),
        "kf_gguf_kv_u64": ([P, L64, ctypes.c_uint64, P], I),
        "kf_gguf_kv_i64": ([P, L64, ctypes.c_uint64, P], I),
        "kf_gguf_kv_f64": ([P, L64, ctypes.c_uint64, P], I),
        "kf_gguf_kv_str": ([P, L64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p), P], I),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res


def declared_symbols() -> list[str]:
    """Every function include/kf_hip.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kf_[a-z0-9_]+)\s*\(", text)))


def check(rc: int) -> int:
    if rc < 0:
        raise KfError(rc, last_error())
    return rc


def release_stream(stream) -> None:
    """Returns the stream's split-K scratch slot (kf_hip_release_stream) after waiting for its work."""
    check(lib().kf_hip_release_stream(stream))


def set_knob(name: str, value) -> None:
    """Sets a launch knob (kf_hip_set_knob): an int, True / False for a flag knob, or None to unset it."""
    v = -1 if value is None or value is False else 1 if value is True else int(value)
    check(lib().kf_hip_set_knob(name.encode(), v))


def get_knob(name: str) -> int:
    v = lib().kf_hip_get_knob(name.encode())
    if v == -2:
        raise KfError(KF_E_INVALID, f"unknown knob {name}")
    return v


def last_error() -> str:
    return lib().kf_hip_last_error().decode()


def row_bytes(ty: int, n: int) -> int:
    block, size = BLOCK[ty]
    return n // block * size


def act_kind(ty: int) -> int:
    return check(lib().kf_hip_act_kind(ty))


def act_bytes(rows: int, n: int) -> int:
    return lib().kf_hip_act_bytes(rows, n)


def act_offsets(rows: int, n: int) -> list[int]:
    out = (ctypes.c_size_t * 6)()
    lib().kf_hip_act_offsets(rows, n, out)
    return list(out)


# ------------------------------------------------------------------ host utilities (numpy in, numpy out)

def _np():
    import numpy as np

    return np


def synth_normal(seed: int, sigma: float, n: int):
    np = _np()
    out = np.empty(n, np.float32)
    lib().kf_synth_normal(seed, sigma, out.ctypes.data_as(ctypes.c_void_p), n)
    return out


def quantize(ty: int, x):
    """Host encoder: q8_0 (quantize_row of the reference) or q4_K / q5_K / q6_K (this library's encoders); x [rows][n] f32."""
    np = _np()
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    rows, n = x.shape
    out = np.empty((rows, row_bytes(ty, n)), np.uint8)
    fn = {TYPE_Q8_0: lib().kf_quantize_q8_0, TYPE_Q4_K: lib().kf_quantize_q4_k, TYPE_Q5_K: lib().kf_quantize_q5_k,
          TYPE_Q6_K: lib().kf_quantize_q6_k}[ty]
    rc = fn(x.ctypes.data_as(ctypes.c_void_p), rows, n, out.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise KfError(rc, f"quantize type {ty} of {rows}x{n}")
    return out


# ------------------------------------------------------------------ device calls on torch tensors

def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return stream
    import torch

    return torch.cuda.current_stream().cuda_stream


def quant_act(x, act, kind: int, stream=None) -> None:
    rows, n = x.shape
    check(lib().kf_hip_quant_act(_ptr(x), _ptr(act), rows, n, kind, _stream(stream)))


GLU_SILU, GLU_RELU, GLU_RELU_SQR = 0, 2, 4


def rms_norm_q8(x, act, kind: int, w=None, b=None, eps: float = 1e-5, stream=None) -> None:
    """rms_norm of each row of x [rows][n] (nullable weight / bias [n]) quantized into `act` (kf_hip_rms_norm_q8)."""
    rows, n = x.shape
    check(lib().kf_hip_rms_norm_q8(_ptr(x), _ptr(w), _ptr(b), rows, n, eps, kind, _ptr(act), _stream(stream)))


def gated_act_q8(gate, up, act, kind: int, rows: int, n: int, stride: int, act_fn: int = GLU_SILU, stream=None) -> None:
    """act_fn(gate) * up of `rows` rows of n columns, rows `stride` floats apart, quantized into `act`
    (kf_hip_gated_act_q8). gate/up may be views into one fused [rows][2n] tensor."""
    check(lib().kf_hip_gated_act_q8(_ptr(gate), _ptr(up), rows, n, stride, act_fn, kind, _ptr(act), _stream(stream)))


def gemv(ty: int, w, act, y, rows: int, n: int, n_out: int, bias=None, res=None, stream=None) -> None:
    check(lib().kf_hip_gemv(ty, _ptr(w), row_bytes(ty, n), _ptr(act), _ptr(bias), _ptr(res), _ptr(y), rows, n, n_out, _stream(stream)))


def gemm_i8(ty: int, w, act, y, rows: int, n: int, n_out: int, bias=None, res=None, stream=None) -> None:
    check(lib().kf_hip_gemm_i8(ty, _ptr(w), row_bytes(ty, n), _ptr(act), _ptr(bias), _ptr(res), _ptr(y), rows, n, n_out, _stream(stream)))


def matmul(ty: int, w, x, act, y, n_out: int, bias=None, res=None, stream=None) -> None:
    rows, n = x.shape
    check(lib().kf_hip_matmul(ty, _ptr(w), n, n_out, _ptr(x), rows, _ptr(act), _ptr(bias), _ptr(res), _ptr(y), _stream(stream)))


def matmul_noalloc(ty: int, w, x, y, n_out: int, bias=None, res=None, stream=None) -> None:
    """kf_hip_matmul_noalloc: kf_hip_matmul with the library's static per-GPU activation scratch (no allocation)."""
    rows, n = x.shape
    check(lib().kf_hip_matmul_noalloc(ty, _ptr(w), n, n_out, _ptr(x), rows, _ptr(bias), _ptr(res), _ptr(y), _stream(stream)))


SEG_NONE = -(1 << 63)
MAX_SEGMENTS = 4


def segment_table(members):
    """The reference's segment words (six int64 per member, offsets from the first member's weights and output) for
    members given as (w, y, bias, res) device tensors, bias/res None or a tensor. Returns (words, lead w, lead y)."""
    import numpy as np

    lead_w, lead_y = _ptr(members[0][0]), _ptr(members[0][1])
    words, start = [], 0
    for w, y, bias, res in members:
        n_out = y.shape[-1]
        off = lambda t: SEG_NONE if t is None else _ptr(t) - lead_y
        words += [_ptr(w) - lead_w, _ptr(y) - lead_y, off(bias), off(res), start, n_out]
        start += n_out
    return np.asarray(words, dtype=np.int64), lead_w, lead_y


def gemv_group(ty: int, members, act, rows: int, n: int, stream=None) -> None:
    """Grouped product of members (w, y, bias, res) sharing the quantized activations act (kf_hip_gemv_group)."""
    words, lw, ly = segment_table(members)
    check(lib().kf_hip_gemv_group(ty, lw, row_bytes(ty, n), _ptr(act), ly, rows, n, words.ctypes.data, len(members), _stream(stream)))


def matmul_group(ty: int, members, x, act, stream=None) -> None:
    """Grouped Op::MatMul of members (w, y, bias, res) on one f32 input x [rows][n] (kf_hip_matmul_group)."""
    rows, n = x.shape
    words, lw, ly = segment_table(members)
    check(lib().kf_hip_matmul_group(ty, lw, n, _ptr(x), rows, _ptr(act), ly, words.ctypes.data, len(members), _stream(stream)))


def block_ints(ty: int, w, act, out, rows: int, n: int, n_out: int, stream=None) -> None:
    check(lib().kf_hip_block_ints(ty, _ptr(w), row_bytes(ty, n), _ptr(act), rows, n, n_out, _ptr(out), _stream(stream)))


def rms_norm_matmul(ty: int, w, x, act, y, n_out: int, norm_w=None, norm_b=None, eps: float = 1e-5, bias=None, res=None, stream=None) -> None:
    """rms_norm of x [rows][n_in], quantization and the product kf_hip_matmul selects, one launch at one row
    (kf_hip_rms_norm_matmul)."""
    rows, n_in = x.shape
    check(lib().kf_hip_rms_norm_matmul(ty, _ptr(w), n_in, n_out, _ptr(x), rows, _ptr(norm_w), _ptr(norm_b), eps, _ptr(act), _ptr(bias), _ptr(res),
                                       _ptr(y), _stream(stream)))


def stream_read(buf, sink, per_thread: int = 8, stream=None) -> None:
    """Streaming read of a device tensor with plain 16-byte loads (kf_hip_stream_read): the HBM read-rate probe."""
    check(lib().kf_hip_stream_read(_ptr(buf), buf.numel() * buf.element_size(), per_thread, _ptr(sink), _stream(stream)))


def moe_group(slots, total: int, n_slots: int, order, offsets, stream=None) -> None:
    check(lib().kf_hip_moe_group(_ptr(slots), total, n_slots, _ptr(order), _ptr(offsets), _stream(stream)))


def moe_gemv(ty: int, w, act, act_rows: int, n: int, n_out: int, order, offsets, n_slots: int, n_used: int, per_slot: bool, y,
             w_up=None, expert_bytes: int | None = None, stream=None) -> None:
    eb = row_bytes(ty, n) * n_out if expert_bytes is None else expert_bytes
    check(lib().kf_hip_moe_gemv(ty, _ptr(w), _ptr(w_up), eb, row_bytes(ty, n), _ptr(act), act_rows, n, n_out, _ptr(order), _ptr(offsets),
                                n_slots, n_used, int(per_slot), _ptr(y), _stream(stream)))


def moe_combine(part, wts, slots, out, rows: int, n_used: int, n_embd: int, scale: float = 1.0, host=None, stream=None) -> None:
    check(lib().kf_hip_moe_combine(_ptr(part), _ptr(wts), _ptr(slots), _ptr(host), _ptr(out), rows, n_used, n_embd, scale, _stream(stream)))


def moe_gemm(ty: int, w, act, pairs: int, n: int, n_out: int, offsets, n_slots: int, y, expert_bytes: int, w2=None, n_split: int = 0,
             out_rows=None, stream=None) -> None:
    """The grouped tile GEMM (kf_hip_moe_gemm): act holds `pairs` activation rows in group order."""
    check(lib().kf_hip_moe_gemm(ty, _ptr(w), _ptr(w2), expert_bytes, row_bytes(ty, n), n_split, _ptr(act), pairs, n, n_out, _ptr(offsets),
                                n_slots, _ptr(out_rows), _ptr(y), _stream(stream)))


def moe_scratch_bytes(rows: int, n_used: int, n_embd: int, n_ff: int, n_slots: int) -> int:
    return lib().kf_hip_moe_scratch_bytes(rows, n_used, n_embd, n_ff, n_slots)


def moe_ffn(ty: int, gate, up, down, n_slots: int, n_embd: int, n_ff: int, x, sel, wts, out, scratch, scale: float = 1.0, stream=None) -> None:
    """The routed expert layer (kf_hip_moe_ffn): x [rows][n_embd] f32, sel/wts [rows][n_used] int32/f32, out [rows][n_embd]."""
    rows, n_used = sel.shape
    check(lib().kf_hip_moe_ffn(ty, _ptr(gate), _ptr(up), _ptr(down), n_slots, n_embd, n_ff, _ptr(x), rows, _ptr(sel), _ptr(wts), n_used, scale,
                               _ptr(scratch), scratch.numel() * scratch.element_size(), _ptr(out), _stream(stream)))


def alloc_act(rows: int, n: int, device="cuda"):
    """A device scratch for quantized activations (uint8 tensor, 256-byte aligned by the caching allocator)."""
    import torch

    t = torch.empty(act_bytes(rows, n), dtype=torch.uint8, device=device)
    assert t.data_ptr() % 256 == 0
    return t


def act_views(act, rows: int, n: int):
    """(q, d16, s16, d32, s32) torch views of a scratch filled by quant_act."""
    import torch

    o = act_offsets(rows, n)
    q = act[o[0] : o[0] + rows * n].view(torch.int8).view(rows, n)
    d16 = act[o[1] : o[1] + rows * (n // 16) * 4].view(torch.float32).view(rows, n // 16)
    s16 = act[o[2] : o[2] + rows * (n // 16) * 4].view(torch.int32).view(rows, n // 16)
    d32 = act[o[3] : o[3] + rows * (n // 32) * 4].view(torch.float32).view(rows, n // 32)
    s32 = act[o[4] : o[4] + rows * (n // 32) * 4].view(torch.int32).view(rows, n // 32)
    return q, d16, s16, d32, s32


def act_xa(act, rows: int, n: int):
    """The xa section (Q8K kind): f16 [rows][ceil(n / 256)][16], per 256 columns the eight per-32 sums as hi then lo."""
    import torch

    o = act_offsets(rows, n)
    nsb = (n + 255) // 256
    return act[o[5] : o[5] + rows * nsb * 32].view(torch.float16).view(rows, nsb, 16)


class Backend:
    """The Backend-trait mirror of the library (kf_hip_backend_*): owns device weights, host rows in and out."""

    def __init__(self, device: int = 0):
        self._h = lib().kf_hip_backend_new(device)
        if not self._h:
            raise KfError(KF_E_INVALID, last_error())

    def close(self) -> None:
        if self._h:
            lib().kf_hip_backend_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add_weight(self, ty: int, dims, data) -> int:
        np = _np()
        data = np.ascontiguousarray(data, np.uint8)
        d = (ctypes.c_int64 * len(dims))(*dims)
        return check(lib().kf_hip_backend_add_weight(self._h, ty, d, len(dims), data.ctypes.data_as(ctypes.c_void_p), data.nbytes))

    def matmul(self, wid: int, x, n_out: int, bias=None):
        np = _np()
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        rows, cols = x.shape
        y = np.empty((rows, n_out), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        check(lib().kf_hip_backend_matmul(self._h, wid, x.ctypes.data_as(ctypes.c_void_p), rows, cols,
                                          None if b is None else b.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p)))
        return y

    def matmul_slice(self, wid: int, index: int, x, n_out: int):
        np = _np()
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        rows, cols = x.shape
        y = np.empty((rows, n_out), np.float32)
        check(lib().kf_hip_backend_matmul_slice(self._h, wid, index, x.ctypes.data_as(ctypes.c_void_p), rows, cols,
                                                y.ctypes.data_as(ctypes.c_void_p)))
        return y
