"""ctypes front end for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` for the expected values and by
bench.py's ``cpu_baseline`` leg. The product package ``satori_amd`` never imports this module.

Every wrapper takes and returns numpy arrays and raises the exception class the reference raises
(ArgumentException, ArgumentOutOfRangeException, InvalidDataException, OverflowException), using
the classes the product defines so host-logic tests can compare both sides.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0, Q4_0, Q4_K, Q6_K = 0, 1, 2, 3
GEOMETRY = {Q8_0: (32, 34), Q4_0: (32, 18), Q4_K: (256, 144), Q6_K: (256, 210)}


class OracleError(Exception):
    """Status code returned by the oracle; ``code`` mirrors the reference exception."""

    NAMES = {1: "ArgumentException", 2: "ArgumentOutOfRangeException", 3: "InvalidDataException",
             9: "OverflowException"}

    def __init__(self, code: int):
        super().__init__(self.NAMES.get(code, f"status {code}"))
        self.code = code
        self.name = self.NAMES.get(code, f"status {code}")


def build(force: bool = False) -> str:
    """Compile liboracle.so with its Makefile (gcc)."""
    cmd = ["make", "-s", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I = ctypes.c_int
SZ = ctypes.c_size_t


def _declare(l):
    sig = {
        "or_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
        "or_t2_byte_length": (ctypes.c_int64, [I, I, I]),
        "or_t2_quantize": (I, [P, I, I, I, P, SZ]),
        "or_t2_validate": (I, [P, SZ, I, I, I]),
        "or_t2_dequantize": (None, [P, I, I, I, P]),
        "or_t2_matvec_scalar": (None, [P, I, I, I, P, P]),
        "or_t2_matvec_avx2": (None, [P, I, I, I, P, P]),
        "or_stq2_write_header": (None, [P, I, I, I]),
        "or_stq2_read_header": (I, [P, P, P, P]),
        "or_tb_validate": (I, [P, SZ, I, I, I]),
        "or_rms_norm": (None, [P, P, ctypes.c_float, I, P]),
        "or_rms_norm_heads": (None, [P, P, ctypes.c_float, I, I]),
        "or_rope": (None, [P, I, I, I]),
        "or_rope_half": (None, [P, I, I, I, ctypes.c_double, I]),
        "or_swiglu": (None, [P, P, I, P]),
        "or_add": (None, [P, P, I, P]),
        "or_grouped_attention": (None, [P, P, P, I, I, I, I, P, P]),
        "or_q_decode_row": (None, [P, I, I, P]),
        "or_tb_from_t2": (None, [P, I, I, I, P]),
        "or_tb_to_t2": (None, [P, I, I, I, P]),
        "or_tb_matvec_scalar": (None, [P, I, I, I, P, P]),
        "or_q_byte_length": (ctypes.c_int64, [I, I, I]),
        "or_q_validate": (I, [P, SZ, I, I, I]),
        "or_q_matvec_scalar": (None, [P, I, I, I, P, P]),
        "or_q_matvec_avx2": (None, [P, I, I, I, P, P]),
        "or_q_decode_block": (None, [P, I, P]),
        "or_q4k_dot_block": (ctypes.c_float, [P, P]),
        "or_q4k_decode_block": (None, [P, P]),
        "or_q4k_dot_product": (ctypes.c_int32, [P, P]),
        "or_q4k_min_product": (ctypes.c_int32, [P, P]),
        "or_q4k_dot_block_quantized": (ctypes.c_float, [P, P]),
        "or_q6k_dot_block": (ctypes.c_float, [P, P]),
        "or_q6k_decode_block": (None, [P, P]),
        "or_q6k_dot_product": (ctypes.c_int32, [P, P]),
        "or_q6k_dot_block_quantized": (ctypes.c_float, [P, P]),
        "or_q8k_quantize_block": (None, [P, P]),
        "or_q8k_quantize_row": (I, [P, I, P, SZ]),
        "or_q_matvec_batch": (I, [P, I, I, I, P, I, P]),
        "or_qk_matvec_quantized_avx2": (None, [P, I, I, I, P, P]),
        "or_qk_matvec_quantized_tiled_avx2": (None, [P, I, I, I, P, I, P]),
        "or_corpus_random_matrix": (None, [I, I, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), dtype=np.uint8) if isinstance(a, (bytes, bytearray)) else a,
                                dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(code: int):
    if code:
        raise OracleError(code)


def half_to_float(bits: int) -> float:
    return lib().or_half_to_float(bits)


# ---- Ternary2 ----

def t2_byte_length(rows: int, columns: int, block: int) -> int:
    n = lib().or_t2_byte_length(rows, columns, block)
    if n < 0:
        raise OracleError(-n)
    return n


def t2_quantize(weights, rows: int, columns: int, block: int = 64) -> np.ndarray:
    w = _f32(weights).reshape(-1)
    if w.size != rows * columns:
        raise OracleError(1)
    out = np.zeros(t2_byte_length(rows, columns, block), dtype=np.uint8)
    _check(lib().or_t2_quantize(_ptr(w), rows, columns, block, _ptr(out), out.size))
    return out


def t2_validate(data, rows: int, columns: int, block: int) -> None:
    d = _u8(data)
    _check(lib().or_t2_validate(_ptr(d), d.size, rows, columns, block))


def tb_validate(data, rows: int, columns: int, block: int) -> None:
    d = _u8(data)
    _check(lib().or_tb_validate(_ptr(d), d.size, rows, columns, block))


def tb_from_t2(t2, rows: int, columns: int, block: int) -> np.ndarray:
    d = _u8(t2)
    out = np.zeros(d.size, dtype=np.uint8)
    lib().or_tb_from_t2(_ptr(d), rows, columns, block, _ptr(out))
    return out


def tb_to_t2(tb, rows: int, columns: int, block: int) -> np.ndarray:
    d = _u8(tb)
    out = np.zeros(d.size, dtype=np.uint8)
    lib().or_tb_to_t2(_ptr(d), rows, columns, block, _ptr(out))
    return out


def tb_matvec_scalar(data, rows: int, columns: int, block: int, x) -> np.ndarray:
    d, xv = _u8(data), _f32(x)
    y = np.zeros(rows, dtype=np.float32)
    lib().or_tb_matvec_scalar(_ptr(d), rows, columns, block, _ptr(xv), _ptr(y))
    return y


def t2_dequantize(data, rows: int, columns: int, block: int) -> np.ndarray:
    d = _u8(data)
    out = np.zeros(rows * columns, dtype=np.float32)
    lib().or_t2_dequantize(_ptr(d), rows, columns, block, _ptr(out))
    return out.reshape(rows, columns)


def t2_matvec_scalar(data, rows: int, columns: int, block: int, x) -> np.ndarray:
    d, xv = _u8(data), _f32(x)
    y = np.zeros(rows, dtype=np.float32)
    lib().or_t2_matvec_scalar(_ptr(d), rows, columns, block, _ptr(xv), _ptr(y))
    return y


def t2_matvec_avx2(data, rows: int, columns: int, block: int, x, y: np.ndarray | None = None) -> np.ndarray:
    d, xv = _u8(data), _f32(x)
    if y is None:
        y = np.zeros(rows, dtype=np.float32)
    lib().or_t2_matvec_avx2(_ptr(d), rows, columns, block, _ptr(xv), _ptr(y))
    return y


def stq2_header(rows: int, columns: int, block: int) -> bytes:
    h = np.zeros(32, dtype=np.uint8)
    lib().or_stq2_write_header(_ptr(h), rows, columns, block)
    return h.tobytes()


def stq2_read_header(header: bytes):
    h = _u8(header)
    r, c, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(lib().or_stq2_read_header(_ptr(h), ctypes.byref(r), ctypes.byref(c), ctypes.byref(b)))
    return r.value, c.value, b.value


# ---- GGUF block formats ----

def q_byte_length(rows: int, columns: int, fmt: int) -> int:
    n = lib().or_q_byte_length(rows, columns, fmt)
    if n < 0:
        raise OracleError(-n)
    return n


def q_validate(data, rows: int, columns: int, fmt: int) -> None:
    d = _u8(data)
    _check(lib().or_q_validate(_ptr(d), d.size, rows, columns, fmt))


def q_matvec_scalar(data, rows: int, columns: int, fmt: int, x) -> np.ndarray:
    d, xv = _u8(data), _f32(x)
    y = np.zeros(rows, dtype=np.float32)
    lib().or_q_matvec_scalar(_ptr(d), rows, columns, fmt, _ptr(xv), _ptr(y))
    return y


def q_matvec_avx2(data, rows: int, columns: int, fmt: int, x, y: np.ndarray | None = None) -> np.ndarray:
    d, xv = _u8(data), _f32(x)
    if y is None:
        y = np.zeros(rows, dtype=np.float32)
    lib().or_q_matvec_avx2(_ptr(d), rows, columns, fmt, _ptr(xv), _ptr(y))
    return y


def q_matvec_batch(data, rows: int, columns: int, fmt: int, x, positions: int) -> np.ndarray:
    d, xv = _u8(data), _f32(x)
    y = np.zeros(rows * positions, dtype=np.float32)
    _check(lib().or_q_matvec_batch(_ptr(d), rows, columns, fmt, _ptr(xv), positions, _ptr(y)))
    return y


def qk_matvec_quantized_avx2(data, rows: int, columns: int, fmt: int, activations, y: np.ndarray | None = None):
    d, a = _u8(data), _u8(activations)
    if y is None:
        y = np.zeros(rows, dtype=np.float32)
    lib().or_qk_matvec_quantized_avx2(_ptr(d), rows, columns, fmt, _ptr(a), _ptr(y))
    return y


def qk_matvec_quantized_tiled_avx2(data, rows: int, columns: int, fmt: int, activations, positions: int,
                                   y: np.ndarray | None = None):
    """ExecuteQuantizedTiled over `positions` (1..256) Q8_K rows at once: output [positions][rows]."""
    d, a = _u8(data), _u8(activations)
    if not 1 <= positions <= 256 or a.size != positions * (columns // 256) * 292:
        raise ValueError("positions must be 1..256 with one Q8_K row each")
    if y is None:
        y = np.zeros(positions * rows, dtype=np.float32)
    lib().or_qk_matvec_quantized_tiled_avx2(_ptr(d), rows, columns, fmt, _ptr(a), positions, _ptr(y))
    return y


def decode_block(block, fmt: int) -> np.ndarray:
    b = _u8(block)
    out = np.zeros(GEOMETRY[fmt][0], dtype=np.float32)
    lib().or_q_decode_block(_ptr(b), fmt, _ptr(out))
    return out


def decode_matrix(data, rows: int, columns: int, fmt: int) -> np.ndarray:
    e, nb = GEOMETRY[fmt]
    d = _u8(data).reshape(rows, columns // e, nb)
    out = np.zeros((rows, columns), dtype=np.float32)
    for r in range(rows):
        for b in range(columns // e):
            out[r, b * e:(b + 1) * e] = decode_block(d[r, b], fmt)
    return out


def q4k_dot_block(block, x) -> float:
    return lib().or_q4k_dot_block(_ptr(_u8(block)), _ptr(_f32(x)))


def q4k_decode_block(block) -> np.ndarray:
    out = np.zeros(256, dtype=np.float32)
    lib().or_q4k_decode_block(_ptr(_u8(block)), _ptr(out))
    return out


def q4k_dot_product(block, activation) -> int:
    return lib().or_q4k_dot_product(_ptr(_u8(block)), _ptr(_u8(activation)))


def q4k_min_product(block, activation) -> int:
    return lib().or_q4k_min_product(_ptr(_u8(block)), _ptr(_u8(activation)))


def q4k_dot_block_quantized(block, activation) -> float:
    return lib().or_q4k_dot_block_quantized(_ptr(_u8(block)), _ptr(_u8(activation)))


def q6k_dot_block(block, x) -> float:
    return lib().or_q6k_dot_block(_ptr(_u8(block)), _ptr(_f32(x)))


def q6k_decode_block(block) -> np.ndarray:
    out = np.zeros(256, dtype=np.float32)
    lib().or_q6k_decode_block(_ptr(_u8(block)), _ptr(out))
    return out


def q6k_dot_product(block, activation) -> int:
    return lib().or_q6k_dot_product(_ptr(_u8(block)), _ptr(_u8(activation)))


def q6k_dot_block_quantized(block, activation) -> float:
    return lib().or_q6k_dot_block_quantized(_ptr(_u8(block)), _ptr(_u8(activation)))


def q8k_quantize_block(x) -> np.ndarray:
    xv = _f32(x)
    out = np.zeros(292, dtype=np.uint8)
    lib().or_q8k_quantize_block(_ptr(xv), _ptr(out))
    return out


def q8k_quantize_row(x) -> np.ndarray:
    xv = _f32(x).reshape(-1)
    if xv.size % 256:
        raise OracleError(1)
    out = np.zeros(xv.size // 256 * 292, dtype=np.uint8)
    _check(lib().or_q8k_quantize_row(_ptr(xv), xv.size, _ptr(out), out.size))
    return out


def corpus_random_matrix(rows: int, columns: int):
    """NumericalCorpus.RandomMatrix: (weights [rows][columns], input [columns])."""
    w = np.zeros(rows * columns, dtype=np.float32)
    x = np.zeros(columns, dtype=np.float32)
    lib().or_corpus_random_matrix(rows, columns, _ptr(w), _ptr(x))
    return w.reshape(rows, columns), x


# ---- TransformerOps (FP64 restatements) ----

def rms_norm(x, weights, epsilon: float) -> np.ndarray:
    xv, wv = _f32(x), _f32(weights)
    out = np.zeros(xv.size, dtype=np.float32)
    lib().or_rms_norm(_ptr(xv), _ptr(wv), epsilon, xv.size, _ptr(out))
    return out


def rms_norm_heads(vector, weights, epsilon: float, head_dim: int) -> np.ndarray:
    v = _f32(vector).copy()
    wv = _f32(weights)
    lib().or_rms_norm_heads(_ptr(v), _ptr(wv), epsilon, head_dim, v.size)
    return v


def rope(vector, head_dim: int, position: int) -> np.ndarray:
    v = _f32(vector).copy()
    lib().or_rope(_ptr(v), v.size, head_dim, position)
    return v


def rope_half(vector, head_dim: int, position: int, base: float, rotary: int) -> np.ndarray:
    v = _f32(vector).copy()
    lib().or_rope_half(_ptr(v), v.size, head_dim, position, base, rotary)
    return v


def swiglu(gate, up) -> np.ndarray:
    g, u = _f32(gate), _f32(up)
    out = np.zeros(g.size, dtype=np.float32)
    lib().or_swiglu(_ptr(g), _ptr(u), g.size, _ptr(out))
    return out


def add(left, right) -> np.ndarray:
    a, b = _f32(left), _f32(right)
    out = np.zeros(a.size, dtype=np.float32)
    lib().or_add(_ptr(a), _ptr(b), a.size, _ptr(out))
    return out


def grouped_attention(query, keys, values, query_heads: int, kv_heads: int, head_dim: int, tokens: int) -> np.ndarray:
    q, k, v = _f32(query), _f32(keys), _f32(values)
    scores = np.zeros(max(tokens, 1), dtype=np.float64)
    out = np.zeros(q.size, dtype=np.float32)
    lib().or_grouped_attention(_ptr(q), _ptr(k), _ptr(v), query_heads, kv_heads, head_dim, tokens, _ptr(scores), _ptr(out))
    return out


def q_decode_row(row, columns: int, fmt: int) -> np.ndarray:
    r = _u8(row)
    out = np.zeros(columns, dtype=np.float32)
    lib().or_q_decode_row(_ptr(r), columns, fmt, _ptr(out))
    return out
