"""CPU oracle for kungfu's quantized linear-layer arithmetic — TEST INFRASTRUCTURE ONLY.

This package wraps ``oracle/build/libkf_oracle.so`` (built from ``oracle/kf_oracle.c`` by ``oracle/Makefile``) with
numpy-friendly functions. Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may
import it, and only as the checker: the product library ``kungfu_amd`` never routes through it.

Each C function restates a piece of the Rust reference and cites the file:line it follows (see kf_oracle.c).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libkf_oracle.so")

TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_Q8_K = 15
ACT_Q8_0 = 3
ACT_Q8K = 4

LAYOUT = {TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144), TYPE_Q5_K: (256, 176), TYPE_Q6_K: (256, 210), TYPE_Q8_K: (256, 292)}

_lib = None


def build() -> None:
    """Compile the oracle library with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    P = ctypes.c_void_p
    I = ctypes.c_int
    U = ctypes.c_uint32
    L.kfo_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.kfo_f16_to_f32.restype = ctypes.c_float
    L.kfo_f32_to_f16.argtypes = [ctypes.c_float]
    L.kfo_f32_to_f16.restype = ctypes.c_uint16
    L.kfo_type_info.argtypes = [U, P, P]
    L.kfo_act_kind.argtypes = [U]
    L.kfo_q8_0_quantize_row.argtypes = [P, I, P]
    L.kfo_q8_0_quantize_row.restype = None
    L.kfo_dequant_row.argtypes = [U, P, I, P]
    L.kfo_dot_row.argtypes = [U, P, P, I]
    L.kfo_dot_row.restype = ctypes.c_float
    L.kfo_quantize_activations.argtypes = [I, P, I, I, P, P, P]
    L.kfo_round_activations.argtypes = [I, P, I, P]
    L.kfo_round_activations.restype = None
    L.kfo_dot_i8.argtypes = [U, P, I, P, P, P, I, P]
    L.kfo_block_ints.argtypes = [U, P, I, P, P, P]
    L.kfo_matmul_slice.argtypes = [U, P, I, I, P, I, P, P, I]
    L.kfo_matmul_i8.argtypes = [U, P, I, I, P, I, P, P, I]
    L.kfo_moe_ffn.argtypes = [U, P, P, P, I, I, I, P, I, P, P, I, P, I]
    L.kfo_moe_ffn_i8.argtypes = [U, P, P, P, I, I, I, P, I, P, P, I, P, I]
    L.kfo_silu.argtypes = [ctypes.c_float]
    L.kfo_rms_norm.argtypes = [P, P, P, I, I, ctypes.c_float, P]
    L.kfo_gated.argtypes = [I, P, P, I, I, I, P]
    L.kfo_silu.restype = ctypes.c_float


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def row_bytes(ty: int, n: int) -> int:
    block, size = LAYOUT[ty]
    return n // block * size


def act_kind(ty: int) -> int:
    return lib().kfo_act_kind(ty)


def f16_to_f32(h: int) -> float:
    return lib().kfo_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().kfo_f32_to_f16(f)


def f32_to_f16_array(x: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.kfo_f32_to_f16(float(v)) for v in np.asarray(x, np.float32).ravel()], dtype=np.uint16)


def q8_0_quantize(x: np.ndarray) -> np.ndarray:
    """q8_0::quantize_row over every row of x [rows][n] -> bytes [rows][row_bytes]"""
    x = _c(np.atleast_2d(x), np.float32)
    rows, n = x.shape
    out = np.zeros((rows, row_bytes(TYPE_Q8_0, n)), np.uint8)
    for r in range(rows):
        lib().kfo_q8_0_quantize_row(_p(x[r]), n, _p(out[r]))
    return out


def dequant(ty: int, w: np.ndarray, n: int) -> np.ndarray:
    w = _c(np.atleast_2d(w), np.uint8)
    out = np.zeros((w.shape[0], n), np.float32)
    for r in range(w.shape[0]):
        rc = lib().kfo_dequant_row(ty, _p(w[r]), n, _p(out[r]))
        assert rc == 0, f"type {ty} not restated"
    return out


def dot_row(ty: int, w_row: np.ndarray, x: np.ndarray) -> float:
    w_row = _c(w_row, np.uint8)
    x = _c(x, np.float32)
    return float(lib().kfo_dot_row(ty, _p(w_row), _p(x), x.size))


def quantize_activations(kind: int, x: np.ndarray):
    """-> (q int8 [rows][n], d16 f32 [rows][n/16], sum16 i32 [rows][n/16]) or None"""
    x = _c(np.atleast_2d(x), np.float32)
    rows, n = x.shape
    q = np.zeros((rows, n), np.int8)
    d = np.zeros((rows, max(n // 16, 1)), np.float32)
    s = np.zeros((rows, max(n // 16, 1)), np.int32)
    rc = lib().kfo_quantize_activations(kind, _p(x), rows, n, _p(q), _p(d), _p(s))
    if rc != 0:
        return None
    return q, d[:, : n // 16], s[:, : n // 16]


def round_activations(kind: int, x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    out = np.zeros_like(x)
    lib().kfo_round_activations(kind, _p(x), x.size, _p(out))
    return out


def dot_i8(ty: int, w_row: np.ndarray, q: np.ndarray, d16: np.ndarray, sum16: np.ndarray) -> np.ndarray:
    w_row = _c(w_row, np.uint8)
    q = _c(np.atleast_2d(q), np.int8)
    d16 = _c(np.atleast_2d(d16), np.float32)
    sum16 = _c(np.atleast_2d(sum16), np.int32)
    rows, n = q.shape
    y = np.zeros(rows, np.float32)
    rc = lib().kfo_dot_i8(ty, _p(w_row), n, _p(q), _p(d16), _p(sum16), rows, _p(y))
    assert rc == 0
    return y


def block_ints(ty: int, w_row: np.ndarray, q_row: np.ndarray, sum16_row: np.ndarray) -> np.ndarray:
    w_row = _c(w_row, np.uint8)
    q_row = _c(q_row, np.int8).ravel()
    sum16_row = _c(sum16_row, np.int32).ravel()
    n = q_row.size
    cnt = {TYPE_Q8_0: n // 32, TYPE_Q6_K: n // 256}.get(ty, 2 * (n // 256))
    out = np.zeros(cnt, np.int32)
    rc = lib().kfo_block_ints(ty, _p(w_row), n, _p(q_row), _p(sum16_row), _p(out))
    assert rc == 0
    return out


def matmul_slice(ty: int, w: np.ndarray, n_in: int, n_out: int, x: np.ndarray, bias=None, threads: int = 0) -> np.ndarray:
    """ops::matmul_slice, the CPU backend's float product; y [rows][n_out]"""
    w = _c(w, np.uint8)
    x = _c(np.atleast_2d(x), np.float32)
    rows = x.shape[0]
    y = np.zeros((rows, n_out), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    rc = lib().kfo_matmul_slice(ty, _p(w), n_in, n_out, _p(x), rows, _p(b), _p(y), threads)
    assert rc == 0, rc
    return y


def matmul_i8(ty: int, w: np.ndarray, n_in: int, n_out: int, x: np.ndarray, bias=None, threads: int = 0) -> np.ndarray:
    w = _c(w, np.uint8)
    x = _c(np.atleast_2d(x), np.float32)
    rows = x.shape[0]
    y = np.zeros((rows, n_out), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    rc = lib().kfo_matmul_i8(ty, _p(w), n_in, n_out, _p(x), rows, _p(b), _p(y), threads)
    assert rc == 0, rc
    return y


def moe_ffn(ty, gate, up, down, n_exp, n_embd, n_ff, x, sel, wts, threads: int = 0) -> np.ndarray:
    x = _c(np.atleast_2d(x), np.float32)
    rows = x.shape[0]
    sel = _c(sel, np.int32)
    wts = _c(wts, np.float32)
    n_used = sel.shape[1]
    out = np.zeros((rows, n_embd), np.float32)
    rc = lib().kfo_moe_ffn(ty, _p(_c(gate, np.uint8)), _p(_c(up, np.uint8)), _p(_c(down, np.uint8)), n_exp, n_embd, n_ff,
                           _p(x), rows, _p(sel), _p(wts), n_used, _p(out), threads)
    assert rc == 0, rc
    return out


def moe_ffn_i8(ty, gate, up, down, n_exp, n_embd, n_ff, x, sel, wts, threads: int = 0) -> np.ndarray:
    """experts::hidden_rows + down_cols: the int8 expert path (the GPU's arithmetic)."""
    x = _c(np.atleast_2d(x), np.float32)
    rows = x.shape[0]
    sel = _c(sel, np.int32)
    wts = _c(wts, np.float32)
    n_used = sel.shape[1]
    out = np.zeros((rows, n_embd), np.float32)
    rc = lib().kfo_moe_ffn_i8(ty, _p(_c(gate, np.uint8)), _p(_c(up, np.uint8)), _p(_c(down, np.uint8)), n_exp, n_embd, n_ff,
                              _p(x), rows, _p(sel), _p(wts), n_used, _p(out), threads)
    assert rc == 0, rc
    return out


def silu(v: float) -> float:
    return float(lib().kfo_silu(v))


def rms_norm(x: np.ndarray, w=None, b=None, eps: float = 1e-5) -> np.ndarray:
    """ops::rms_norm (crates/kf-backend-cpu/src/ops.rs:222-239) of rows x [rows][n]."""
    x = _c(x, np.float32)
    rows, n = x.shape
    out = np.empty_like(x)
    rc = lib().kfo_rms_norm(_p(x), _p(None if w is None else _c(w, np.float32)), _p(None if b is None else _c(b, np.float32)),
                            rows, n, eps, _p(out))
    assert rc == 0, rc
    return out


def gated(act: int, gate: np.ndarray, up: np.ndarray, rows: int, n: int, stride: int) -> np.ndarray:
    """ops::gated without a limit (crates/kf-backend-cpu/src/ops.rs:44-57): act(gate) * up, act 0 silu / 2 relu /
    4 relu squared; gate and up are flat arrays whose rows are `stride` floats apart."""
    gate, up = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty((rows, n), np.float32)
    rc = lib().kfo_gated(act, _p(gate), _p(up), rows, n, stride, _p(out))
    assert rc == 0, rc
    return out


def load_fixture(path: str):
    """The reference fixture format (crates/kf-quant/tests/parity.rs:58-69): u32 n, u32 rows, raw block bytes,
    then n*rows f32 LE of ggml's dequant output."""
    raw = open(path, "rb").read()
    n, rows = np.frombuffer(raw[:8], "<u4")
    n, rows = int(n), int(rows)
    floats = n * rows
    raw_len = len(raw) - 8 - 4 * floats
    blocks = np.frombuffer(raw[8 : 8 + raw_len], np.uint8).copy()
    want = np.frombuffer(raw[8 + raw_len :], "<f4").copy().reshape(rows, n)
    return n, rows, blocks.reshape(rows, -1), want
