"""Host-side logic of the product, on the CPU: the C-ABI library loads and exports every symbol the header
declares, and its host-only entry points (shape lengths, payload validation, Ternary2 quantizer, synthetic
GGUF quantizers) agree with the oracle and raise the reference's exception for each failure. No kernel
runs here."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import satori_amd as S
from helpers import critical_cases, hexbytes, load_json, rng
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BQ = S.BlockQuantization


def declared_functions() -> list[str]:
    with open(os.path.join(ROOT, "include", "satori_hip.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(satori_hip_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_entry_point():
    lib = ctypes.CDLL(S._ffi.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 32
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/satori_hip.h but not exported"
    assert set(names) == set(S._ffi.SIGNATURES), "ctypes binding and header disagree"
    assert S._ffi.lib().satori_hip_abi_version() == 4


def test_context_without_gfx950_device_is_platform_not_supported():
    if S.device_count() > 0:
        pytest.skip("a gfx950 device is present")
    with pytest.raises(S.PlatformNotSupportedException):
        S.HipContext(0)


@pytest.mark.parametrize("rows,columns,block", [(1, 1, 64), (4096, 4096, 128), (4096, 4096, 64), (7, 259, 256),
                                                (1024, 1024, 256)])
def test_ternary2_payload_length_matches_oracle(rows, columns, block):
    assert S.payload_length(S.TERNARY2, rows, columns, block) == O.t2_byte_length(rows, columns, block)


@pytest.mark.parametrize("fmt,rows,columns", [(BQ.Q8_0, 4096, 4096), (BQ.Q4_0, 11008, 4096), (BQ.Q4_K, 8960, 1536),
                                              (BQ.Q6_K, 1536, 8960), (BQ.Q6_K, 151936, 1536)])
def test_quantized_payload_length_matches_oracle(fmt, rows, columns):
    assert S.QuantizedMatrixShape(rows, columns, fmt).byte_length == O.q_byte_length(rows, columns, int(fmt))


def test_shape_failures_map_to_reference_exceptions():
    for args in ((S.TERNARY2, 0, 1, 64), (S.TERNARY2, 1, 0, 64), (S.TERNARY2, 1, 1, 32), (BQ.Q4_K, 1, 128, 0),
                 (BQ.Q8_0, 1, 33, 0), (BQ.Q8_0, -1, 32, 0), (99, 1, 32, 0)):
        with pytest.raises(S.ArgumentOutOfRangeException):
            S.payload_length(*args)
    with pytest.raises(S.OverflowException):
        S.payload_length(S.TERNARY2, 2_000_000, 100_000, 64)
    with pytest.raises(S.OverflowException):
        S.QuantizedMatrixShape(2_000_000, 1 << 20, BQ.Q8_0)
    assert issubclass(S.ArgumentOutOfRangeException, S.ArgumentException)


def test_ternary2_from_packed_validation_agrees_with_oracle():
    g = rng(4)
    base = O.t2_quantize(g.standard_normal((3, 70)).astype(np.float32), 3, 70, 64)
    S.Ternary2Matrix.from_packed(3, 70, 64, base)
    corruptions = []
    for index in range(0, base.size, 7):
        c = base.copy()
        c[index] ^= 0xFF
        corruptions.append(c)
    zero_scale = base.copy()
    zero_scale[:4] = 0
    corruptions.append(zero_scale)
    for c in corruptions:
        try:
            O.t2_validate(c, 3, 70, 64)
            expected = None
        except O.OracleError as e:
            expected = e.code
        if expected is None:
            S.Ternary2Matrix.from_packed(3, 70, 64, c)
        else:
            with pytest.raises(S.ArgumentException) as info:
                S.Ternary2Matrix.from_packed(3, 70, 64, c)
            assert info.value.status == expected
    with pytest.raises(S.ArgumentException):
        S.Ternary2Matrix.from_packed(3, 70, 64, base[:-1])


def test_quantized_validation_agrees_with_oracle():
    g = rng(5)
    for fmt in BQ:
        e, nb = O.GEOMETRY[int(fmt)]
        rows, columns = 3, 2 * e
        data = S.quantize_weights(g.standard_normal((rows, columns)).astype(np.float32), rows, columns, fmt)
        S.QuantizedMatVec.validate_payload(data, S.QuantizedMatrixShape(rows, columns, fmt))
        offsets = {BQ.Q4_K: (1, 3), BQ.Q6_K: (209,)}.get(fmt, (1,))
        for block in range(rows * 2):
            for off in offsets:
                bad = data.copy()
                bad[block * nb + off] = 0x7C  # exponent all ones: infinity or NaN
                with pytest.raises(S.InvalidDataException):
                    S.QuantizedMatVec.validate_payload(bad, S.QuantizedMatrixShape(rows, columns, fmt))
                with pytest.raises(O.OracleError):
                    O.q_validate(bad, rows, columns, int(fmt))
        with pytest.raises(S.ArgumentException):
            S.QuantizedMatVec.validate_payload(data[:-1], S.QuantizedMatrixShape(rows, columns, fmt))


@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_quantizer_bytes_equal_oracle(block):
    for name, w, x in critical_cases(block):
        rows, columns = w.shape
        assert np.array_equal(S.Ternary2Matrix.quantize(w, rows, columns, block).data,
                              O.t2_quantize(w, rows, columns, block)), name
    g = rng(block)
    w = g.standard_normal((64, 1000)).astype(np.float32)
    assert np.array_equal(S.Ternary2Matrix.quantize(w, 64, 1000, block).data, O.t2_quantize(w, 64, 1000, block))
    with pytest.raises(S.ArgumentException):
        S.Ternary2Matrix.quantize(np.array([np.nan], np.float32), 1, 1, block)


def test_ternary2_save_writes_stq2(tmp_path):
    m = S.Ternary2Matrix.quantize(np.array([1.0], np.float32), 1, 1)
    path = tmp_path / "one.stq2"
    m.save(str(path))
    data = path.read_bytes()
    assert data[:32] == O.stq2_header(1, 1, 64)  # MappedTernary2Tests.cs:40-46 bytes
    assert data[32:] == m.data.tobytes()
    with pytest.raises(FileExistsError):  # FileMode.CreateNew
        m.save(str(path))


@pytest.mark.parametrize("fmt", list(BQ))
def test_synthetic_quantizers_are_valid_and_close(fmt):
    g = rng(20261014)
    rows, columns = 16, 512
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    O.q_validate(data, rows, columns, int(fmt))
    decoded = O.decode_matrix(data, rows, columns, int(fmt))
    rel = np.sqrt(np.mean((decoded - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    limit = {BQ.Q8_0: 0.01, BQ.Q4_0: 0.2, BQ.Q4_K: 0.2, BQ.Q6_K: 0.06}[fmt]
    assert rel < limit, rel
    zeros = S.quantize_weights(np.zeros((2, 512), np.float32), 2, 512, fmt)
    assert np.all(O.decode_matrix(zeros, 2, 512, int(fmt)) == 0)


def test_q4k_scale_packing_round_trips_through_reference_decoder():
    # Every 6-bit scale/min value survives pack -> Q4KCodec.GetScaleMin: quantize weights whose sub-block
    # ranges force distinct scales, then check the decoder reproduces the weights to within a step.
    g = rng(8)
    w = np.zeros((1, 256), np.float32)
    for j in range(8):
        w[0, 32 * j:32 * j + 32] = g.uniform(-0.1 * (j + 1), 0.05 * (8 - j), 32)
    data = S.quantize_weights(w, 1, 256, BQ.Q4_K)
    decoded = O.q4k_decode_block(data)
    step = float(data[0:2].view(np.float16)[0]) * 63 + float(data[2:4].view(np.float16)[0]) * 63
    assert np.max(np.abs(decoded - w[0])) < step


def test_fixture_blocks_pass_product_validation():
    for fixture, fmt in (("q4k-v1.json", BQ.Q4_K), ("q6k-v1.json", BQ.Q6_K)):
        for case in load_json(fixture)["cases"]:
            S.QuantizedMatVec.validate_payload(hexbytes(case["block_hex"]), S.QuantizedMatrixShape(1, 256, fmt))


@pytest.mark.parametrize("tokens,head_dim,launches", [
    (1, 128, 2), (32, 128, 2),        # one workgroup per head: inputs + attention
    (33, 128, 2), (512, 128, 2),      # split with the inputs inside it: split + combine
    (2048, 128, 2), (2049, 128, 2),   # 32 splits of 64 / 65 tokens
    (2560, 128, 2),                   # 32 splits of 80 tokens, the last fused length
    (2561, 128, 3), (4096, 128, 3),   # 32 splits of 81 / 128 tokens: inputs + split + combine
    (4097, 128, 3), (8192, 128, 3),   # 33 / 64 splits of 125 / 128 tokens
    (131072, 128, 3), (131073, 128, 3),  # 64 splits of 2,048 tokens, then as many as keep a split at 2,048
    (65537, 128, 3),
    (512, 320, 3),                    # a head wider than the split workgroup's 256 lanes
])
def test_decode_attention_launch_count_follows_split_rule(tokens, head_dim, launches):
    from satori_amd.decode import decode_attention_launches
    assert decode_attention_launches(tokens, head_dim) == launches
