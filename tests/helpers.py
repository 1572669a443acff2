"""Shared test helpers: fixture loading, seeded synthetic data and the reference's error bounds.

The oracle (oracle/oracle.py) is the checker; these helpers only load data and compute bounds in FP64.
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
