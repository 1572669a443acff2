"""Shared test helpers: fixture loading, seeded synthetic data and the reference's error bounds.

The oracle (oracle/oracle.py) supplies the expected values; these helpers only load data and compute
bounds in FP64.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_json(name: str) -> dict:
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def hexbytes(s: str) -> np.ndarray:
    return np.frombuffer(bytes.fromhex(s), dtype=np.uint8)


def gguf_tensor(name: str) -> tuple[np.ndarray, dict]:
    """Payload bytes of the single tensor of a golden GGUF file, at the offsets its manifest records."""
    manifest = load_json("gguf-manifest.json")
    entry = next(f for f in manifest["fixtures"] if f["file"] == name)
    with open(os.path.join(GOLDEN, name), "rb") as f:
        data = f.read()
    assert data[:4] == b"GGUF" and struct.unpack_from("<I", data, 4)[0] == 3
    start = entry["data_start"] + entry["relative_offset"]
    return np.frombuffer(data[start:start + entry["payload_bytes"]], dtype=np.uint8), entry


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def gamma(n: float) -> float:
    u = 2.0 ** -24
    return n * u / (1 - n * u)


def ternary2_bound(dequantized: np.ndarray, x: np.ndarray, block: int) -> np.ndarray:
    """NumericalValidation kernel bound (validation/Satori.Validation/NumericalValidation.cs:71-88):
    gamma(B + blocks + 2) * sum|wq * x| + (C + blocks) * float.Epsilon, per row, in FP64."""
    columns = dequantized.shape[1]
    blocks = (columns + block - 1) // block
    absolute = np.abs(dequantized.astype(np.float64)) @ np.abs(x.astype(np.float64))
    return gamma(block + blocks + 2) * absolute + (columns + blocks) * float(np.finfo(np.float32).smallest_subnormal)


def relative_bound(weights: np.ndarray, x: np.ndarray, tolerance: float = 1e-5) -> np.ndarray:
    """The path's parity gate: tolerance * sum_i |w_i * x_i| per row, FP64."""
    return tolerance * (np.abs(weights.astype(np.float64)) @ np.abs(x.astype(np.float64)))


def fp64_matvec(weights: np.ndarray, x: np.ndarray) -> np.ndarray:
    return weights.astype(np.float64) @ x.astype(np.float64)


def critical_cases(block: int):
    """NumericalCorpus.CriticalCases (validation/Satori.Validation/NumericalCorpus.cs:18-38)."""
    def pattern(name, rows, columns, weight, activation):
        w = np.array([weight(i) for i in range(rows * columns)], dtype=np.float32).reshape(rows, columns)
        x = np.array([activation(i) for i in range(columns)], dtype=np.float32)
        return name, w, x

    from oracle import oracle as O

    TINY = float(np.finfo(np.float32).smallest_subnormal)
    fmax = np.finfo(np.float32).max
    w, x = O.corpus_random_matrix(7, block * 2 + 3)
    yield "random", w, x
    yield pattern("zeros", 3, block + 1, lambda i: 0, lambda i: 1)
    yield pattern("alternating", 5, block * 2 + 1, lambda i: 1 if i % 2 == 0 else -1, lambda i: 1)
    yield pattern("sparse", 3, block - 1, lambda i: 4 if i % 17 == 0 else 0, lambda i: i % 3 - 1)
    yield pattern("small-scale", 3, block + 3, lambda i: 1e-30 if i % 2 == 0 else -1e-30, lambda i: 1)
    yield pattern("large-scale", 3, block + 3, lambda i: 1e30 if i % 2 == 0 else -1e30, lambda i: 1e-10)
    yield pattern("subnormal", 2, block + 1, lambda i: TINY if i % 2 == 0 else -TINY, lambda i: 1)
    yield pattern("max-scale", 2, block + 1, lambda i: fmax if i % 2 == 0 else -fmax, lambda i: 1e-38)
    yield pattern("single-weight", 1, 1, lambda i: -2, lambda i: 3)


def special_scale_payload(fmt, rows, columns, scales):
    # QuantizedTests.cs:186-214 (Q8_0) and Q4Tests.cs:239-268 (Q4_0): signed, zero, -0, subnormal, 65504.
    from oracle import oracle as O

    e, nb = O.GEOMETRY[int(fmt)]
    blocks = columns // 32
    data = np.zeros(rows * blocks * nb, np.uint8)
    for row in range(rows):
        for b in range(blocks):
            off = (row * blocks + b) * nb
            data[off:off + 2] = np.frombuffer(np.float16(scales[row % len(scales)]).tobytes(), np.uint8)
            if int(fmt) == 0:
                for j in range(32):
                    data[off + 2 + j] = ((row * 32 + b * 17 + j * 7) % 256 - 128) & 0xFF
            else:
                for j in range(16):
                    lo, hi = (j + b) % 16, (15 - j + b) % 16
                    data[off + 2 + j] = lo | (hi << 4)
    return data


def attention_boundary_case():
    """The closed-form inputs of VulkanAttentionTests.cs:17-22 (6 heads of 48 lanes, 128 tokens) and the
    FP64 expected outputs of fixtures/operators/attention-boundaries-v1.json, keyed by token count."""
    width = 288
    i = np.arange(width)
    q = ((i % 17 - 8) * 0.125).astype(np.float32)
    token = np.arange(128)[:, None]
    keys = (((token * 13 + i * 7) % 31 - 15) * 0.0625).astype(np.float32)
    values = (((token * 5 + i * 11) % 37 - 18) * 0.125).astype(np.float32)
    cases = {c["count"]: np.array(c["expected"], np.float64) for c in load_json("attention-boundaries-v1.json")["cases"]}
    return q, keys, values, cases
