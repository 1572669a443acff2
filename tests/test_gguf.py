"""GGUF v3 container parse through the library (satori_hip_gguf_*), against the reference's own GGUF tests:
tests/Satori.Numerics.Tests/GgufTests.cs and GgufStructureTests.cs (same cases, same expected failure kinds),
on the reference's golden files (tests/golden/*.gguf, copied as data) and on containers built here the way
the reference's GgufContainerFixture builds them. No GPU: the catalogue and windows are host-side.
"""
from __future__ import annotations

import math
import os
import struct

import numpy as np
import pytest

import satori_amd as S
from helpers import GOLDEN


def golden(name: str) -> str:
    return os.path.join(GOLDEN, name)


def gguf_string(value) -> bytes:
    raw = value.encode("utf-8") if isinstance(value, str) else bytes(value)
    return struct.pack("<Q", len(raw)) + raw


def container(alignment: int, metadata: bytes = b"", extras: int = 0, tensors=None) -> bytes:
    """Header + metadata + tensor infos, zero-padded to the alignment (the layout GgufContainerFixture.Prefix
    writes: architecture "llama" and general.alignment first, then `extras` more entries)."""
    if tensors is None:
        tensors = [("first", [2], 0, 0), ("second", [2], 1, alignment)]
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 2 + extras))
    out += gguf_string("general.architecture") + struct.pack("<I", 8) + gguf_string("llama")
    out += gguf_string("general.alignment") + struct.pack("<II", 4, alignment)
    out += metadata
    for name, shape, type_, offset in tensors:
        out += gguf_string(name) + struct.pack("<I", len(shape))
        for d in shape:
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", type_, offset)
    while len(out) % alignment:
        out += b"\0"
    return bytes(out)


def write_file(tmp_path, data: bytes, length: int | None = None, name: str = "weights.bin") -> str:
    path = str(tmp_path / name)
    with open(path, "wb") as f:
        f.write(data)
        if length is not None and length > len(data):
            f.truncate(length)
    return path


# ---------------------------------------------------------------------------------------------
# GgufTests.cs
# ---------------------------------------------------------------------------------------------

def test_repeated_opens_keep_names_and_scalar_types_stable():
    # GgufTests.cs:8-19 (1000 opens there; 200 here).
    for _ in range(200):
        with S.GgufFile(golden("q8_0.gguf")) as f:
            assert f.read_scalar("general.architecture") == "llama"
            assert f.read_scalar("general.quantization_version") == 2
            assert f.tensors["weights"].type == 8


@pytest.mark.parametrize("name,type_,length,offset", [("q4_0", 2, 18, 160), ("q8_0", 8, 34, 160),
                                                      ("f32", 0, 12, 128), ("f16", 1, 6, 128)])
def test_golden_catalogue_and_scoped_bounds(name, type_, length, offset):
    # GgufTests.cs:31-47.
    f = S.GgufFile(golden(name + ".gguf"))
    assert len(f.tensors) == 1
    tensor = next(iter(f.tensors.values()))
    assert (tensor.type, tensor.byte_length, tensor.offset) == (type_, length, offset)
    assert f.read_scalar("general.architecture") == "llama"
    with pytest.raises(S.ArgumentOutOfRangeException):
        f.read_tensor("weights", length, 1)
    assert f.read_tensor("weights", length, 0) == b""
    with open(golden(name + ".gguf"), "rb") as raw:
        assert f.read_tensor("weights", 0, length) == raw.read()[offset:offset + length]
    f.dispose()
    with pytest.raises(S.ObjectDisposedException):
        f.read_tensor("weights", 0, 1)
    f.dispose()  # idempotent


def test_every_truncation_rejects_without_publishing_catalogue(tmp_path):
    # GgufTests.cs:49-58: every proper prefix of the golden file is corrupt.
    with open(golden("q8_0.gguf"), "rb") as f:
        data = f.read()
    for n in range(len(data)):
        path = write_file(tmp_path, data[:n], name=f"t{n}.gguf")
        with pytest.raises(S.InvalidDataException):
            S.GgufFile(path)


def test_mutated_structure_and_unsupported_version_reject(tmp_path):
    # GgufTests.cs:60-75.
    with open(golden("q8_0.gguf"), "rb") as f:
        data = bytearray(f.read())
    for index in (0, 32, 45, 137):
        mutated = bytearray(data)
        mutated[index] = 0xFF
        with pytest.raises(S.InvalidDataException):
            S.GgufFile(write_file(tmp_path, bytes(mutated), name=f"m{index}.gguf"))
    struct.pack_into("<I", data, 4, 2)
    with pytest.raises(S.NotSupportedException):
        S.GgufFile(write_file(tmp_path, bytes(data), name="v2.gguf"))


def test_window_copies_survive_disposal():
    # GgufTests.cs:77-87 (the callback's span outlives Dispose): a window read before disposal stays valid,
    # and reads after disposal fail.
    f = S.GgufFile(golden("q8_0.gguf"))
    block = f.read_tensor("weights", 0, 34)
    f.dispose()
    assert block[1] == 0x38
    with pytest.raises(S.ObjectDisposedException):
        f.read_metadata("general.architecture")


def test_missing_names_raise_key_not_found():
    with S.GgufFile(golden("q8_0.gguf")) as f:
        with pytest.raises(S.KeyNotFoundException):
            f.read_tensor("absent", 0, 0)
        with pytest.raises(S.KeyNotFoundException):
            f.read_metadata("general.absent")


# ---------------------------------------------------------------------------------------------
# GgufStructureTests.cs
# ---------------------------------------------------------------------------------------------

def _value(type_: int) -> bytes:
    return {
        0: struct.pack("<B", 17), 1: struct.pack("<b", -17), 2: struct.pack("<H", 17), 3: struct.pack("<h", -17),
        4: struct.pack("<I", 17), 5: struct.pack("<i", -17), 6: struct.pack("<f", math.inf),
        7: struct.pack("<B", 1), 8: gguf_string("è\0漢"),
        9: struct.pack("<IQ", 7, 2) + bytes([0, 1]), 10: struct.pack("<Q", 17), 11: struct.pack("<q", -17),
        12: struct.pack("<d", math.nan),
    }[type_]


@pytest.mark.parametrize("alignment", [8, 64, 4096])
def test_mixed_tensors_all_scalar_types_and_flat_arrays(tmp_path, alignment):
    # GgufStructureTests.cs:7-31.
    meta = b"".join(gguf_string(f"custom.value_{t}") + struct.pack("<I", t) + _value(t) for t in range(13))
    meta += gguf_string("custom.empty") + struct.pack("<IIQ", 9, 8, 0)
    meta += gguf_string("custom.strings") + struct.pack("<IIQ", 9, 8, 2) + gguf_string("è\0漢") + gguf_string("")
    prefix = container(alignment, meta, 15)
    with S.GgufFile(write_file(tmp_path, prefix, len(prefix) + alignment * 2 + 3)) as f:
        assert len(f.tensors) == 2 and len(f.metadata) == 17
        assert f.read_scalar("custom.value_8") == "è\0漢"
        assert f.read_scalar("custom.value_4") == 17
        assert f.read_scalar("custom.value_11") == -17
        assert math.isnan(f.read_scalar("custom.value_12"))
        assert f.read_scalar("custom.value_6") == math.inf
        assert f.read_scalar("custom.value_7") is True
        assert f.metadata["custom.empty"].element_count == 0
        assert f.metadata["custom.strings"].element_count == 2
        assert f.metadata["custom.value_4"].element_count is None
        assert f.tensors["second"].offset == len(prefix) + alignment
        assert f.data_offset == len(prefix)
        with pytest.raises(S.InvalidOperationException):
            f.read_scalar("custom.value_9")


def test_oversized_sparse_file_rejects_before_mapping(tmp_path):
    # GgufStructureTests.cs:51-57.
    try:
        path = write_file(tmp_path, b"", (1 << 40) + 1)
    except OSError:
        pytest.skip("the temporary file system does not take a 1 TiB sparse file")
    with pytest.raises(S.NotSupportedException, match="File limit"):
        S.GgufFile(path)


@pytest.mark.parametrize("split_count,split_no,rejected", [(0, 0, False), (1, 0, False), (2, 0, True), (1, 1, True)])
def test_split_count_zero_is_treated_as_unsharded(tmp_path, split_count, split_no, rejected):
    # GgufStructureTests.cs:59-76.
    meta = (gguf_string("split.count") + struct.pack("<IH", 2, split_count)
            + gguf_string("split.no") + struct.pack("<IH", 2, split_no))
    prefix = container(32, meta, 2)
    path = write_file(tmp_path, prefix, len(prefix) + 64)
    if rejected:
        with pytest.raises(S.NotSupportedException):
            S.GgufFile(path)
    else:
        with S.GgufFile(path) as f:
            assert len(f.tensors) == 2


def test_sparse_tensor_beyond_two_gib_uses_int64_windows(tmp_path):
    # GgufStructureTests.cs:78-94.
    first = 1 << 31
    prefix = container(32, tensors=[("large", [first // 4], 0, 0), ("tail", [1], 0, first)])
    path = str(tmp_path / "sparse.gguf")
    try:
        with open(path, "wb") as f:
            f.write(prefix)
            f.truncate(len(prefix) + first + 32)
            f.seek(len(prefix) + first)
            f.write(bytes([1, 2, 3, 4]))
    except OSError:
        pytest.skip("the temporary file system does not take a 2 GiB sparse file")
    with S.GgufFile(path) as f:
        assert f.read_tensor("tail", 0, 4) == bytes([1, 2, 3, 4])
        with pytest.raises(S.ArgumentOutOfRangeException):
            f.read_tensor("large", first - 1, 2)


@pytest.mark.parametrize("defect", ["bool", "key", "duplicate", "utf8", "typed"])
def test_invalid_metadata_rejects(tmp_path, defect):
    # GgufStructureTests.cs:96-114.
    key = {"key": "BAD.key", "duplicate": "general.architecture", "typed": "general.file_type"}.get(defect, "custom.test")
    meta = gguf_string(key)
    if defect == "utf8":
        meta += struct.pack("<IQ", 8, 1) + b"\xff"
    else:
        meta += struct.pack("<IB", 7, 2 if defect == "bool" else 1)
    prefix = container(32, meta, 1)
    with pytest.raises(S.InvalidDataException):
        S.GgufFile(write_file(tmp_path, prefix, len(prefix) + 64))


@pytest.mark.parametrize("defect", ["overlap", "overflow", "zero", "unaligned", "duplicate"])
def test_invalid_tensor_structure_rejects(tmp_path, defect):
    # GgufStructureTests.cs:116-136.
    tensors = {
        "overlap": [("a", [32], 0, 0), ("b", [1], 0, 32)],
        "overflow": [("a", [2**63 - 1, 2], 0, 0)],
        "zero": [("a", [0], 0, 0)],
        "unaligned": [("a", [1], 0, 1)],
        "duplicate": [("a", [1], 0, 0), ("a", [1], 0, 32)],
    }[defect]
    prefix = container(32, tensors=tensors)
    with pytest.raises(S.InvalidDataException):
        S.GgufFile(write_file(tmp_path, prefix, len(prefix) + 256))


def test_gap_and_reverse_physical_order_are_unsupported_rather_than_corrupt(tmp_path):
    # GgufStructureTests.cs:138-149.
    for offsets in ((32, 64), (32, 0)):
        prefix = container(32, tensors=[("a", [1], 0, offsets[0]), ("b", [1], 0, offsets[1])])
        with pytest.raises(S.NotSupportedException):
            S.GgufFile(write_file(tmp_path, prefix, len(prefix) + 128, name=f"g{offsets[1]}.gguf"))


def test_k_quantized_types_are_accepted(tmp_path):
    # GgufStructureTests.cs:151-170: Q4_K (2 blocks) then Q6_K (1 block).
    meta = gguf_string("general.quantization_version") + struct.pack("<II", 4, 2)
    prefix = container(32, meta, 1, [("q4k", [256, 2], 12, 0), ("q6k", [256, 1], 14, 288)])
    with S.GgufFile(write_file(tmp_path, prefix, len(prefix) + 512)) as f:
        assert len(f.tensors) == 2
        assert f.tensors["q4k"].type == 12 and f.tensors["q6k"].type == 14
        assert f.tensors["q4k"].byte_length == 288 and f.tensors["q6k"].byte_length == 210


def test_quantized_tensors_require_quantization_version(tmp_path):
    # GgufFile.cs:156: a quantized tensor without general.quantization_version is corrupt; version 3 is
    # outside the profile.
    prefix = container(32, tensors=[("q8", [32, 1], 8, 0)])
    with pytest.raises(S.InvalidDataException, match="quantization version"):
        S.GgufFile(write_file(tmp_path, prefix, len(prefix) + 64))
    meta = gguf_string("general.quantization_version") + struct.pack("<II", 4, 3)
    prefix = container(32, meta, 1, [("q8", [32, 1], 8, 0)])
    with pytest.raises(S.NotSupportedException):
        S.GgufFile(write_file(tmp_path, prefix, len(prefix) + 64, name="v3.gguf"))


@pytest.mark.parametrize("case,kind", [
    ("alignment 24", S.InvalidDataException), ("alignment 4", S.NotSupportedException),
    ("architecture", S.InvalidDataException), ("type", S.NotSupportedException),
    ("rank 5", S.NotSupportedException), ("type 3", S.NotSupportedException),
    ("row 31", S.InvalidDataException), ("array type", S.NotSupportedException),
    ("empty name", S.InvalidDataException),
])
def test_profile_limits(tmp_path, case, kind):
    # GgufFile.cs:106-147: alignment, architecture, general.type, rank, tensor type, block multiple, array
    # element type, tensor name.
    if case.startswith("alignment"):
        a = int(case.split()[1])
        out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 1, 2))
        out += gguf_string("general.architecture") + struct.pack("<I", 8) + gguf_string("llama")
        out += gguf_string("general.alignment") + struct.pack("<II", 4, a)
        out += gguf_string("a") + struct.pack("<IQIQ", 1, 1, 0, 0)
        data = bytes(out) + bytes(64)
    elif case == "architecture":
        out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 1, 1))
        out += gguf_string("general.architecture") + struct.pack("<I", 8) + gguf_string("Llama")
        out += gguf_string("a") + struct.pack("<IQIQ", 1, 1, 0, 0)
        data = bytes(out) + bytes(64)
    elif case == "type":
        data = container(32, gguf_string("general.type") + struct.pack("<I", 8) + gguf_string("adapter"), 1) + bytes(64)
    elif case == "rank 5":
        data = container(32, tensors=[("a", [1, 1, 1, 1, 1], 0, 0)]) + bytes(64)
    elif case == "type 3":
        data = container(32, tensors=[("a", [32], 3, 0)]) + bytes(64)
    elif case == "row 31":
        meta = gguf_string("general.quantization_version") + struct.pack("<II", 4, 2)
        data = container(32, meta, 1, [("a", [31, 1], 8, 0)]) + bytes(64)
    elif case == "array type":
        data = container(32, gguf_string("custom.a") + struct.pack("<IIQ", 9, 9, 1), 1) + bytes(64)
    else:
        data = container(32, tensors=[("", [1], 0, 0)]) + bytes(64)
    with pytest.raises(kind):
        S.GgufFile(write_file(tmp_path, data))


def test_quantized_matrix_binding_checks(tmp_path):
    # GgufQuantizedMatrix.cs:16-19: only rank-2 Q8_0/Q4_0/Q4_K/Q6_K tensors bind; the shape is
    # (rows = dims[1], columns = dims[0]); the payload is validated.
    with S.GgufFile(golden("f32.gguf")) as f:
        with pytest.raises(S.NotSupportedException):
            S.GgufQuantizedMatrix(f, "weights")
    with S.GgufFile(golden("q8_0.gguf")) as f:
        m = S.GgufQuantizedMatrix(f, "weights")
        dims = f.tensors["weights"].dimensions
        assert (m.shape.rows, m.shape.columns, m.shape.format) == (dims[1], dims[0], S.BlockQuantization.Q8_0)
    # A non-finite Q8_0 scale is corrupt payload.
    meta = gguf_string("general.quantization_version") + struct.pack("<II", 4, 2)
    prefix = container(32, meta, 1, [("w", [32, 1], 8, 0)])
    block = struct.pack("<H", 0x7C00) + bytes(32)  # +Inf scale
    path = write_file(tmp_path, prefix + block + bytes(30))
    with S.GgufFile(path) as f:
        with pytest.raises(S.InvalidDataException):
            S.GgufQuantizedMatrix(f, "w")


def test_utf8_acceptance_matches_strict_decoding(tmp_path):
    # Tensor names go through the strict UTF-8 check (GgufCursor.cs:46-53): overlong forms, surrogates and
    # code points above U+10FFFF are corrupt; valid multi-byte names are accepted. Python's strict codec
    # is the independent judge.
    samples = [b"ok", "è".encode(), "漢".encode(), "😀".encode(), b"\xc0\xaf", b"\xe0\x80\xaf", b"\xed\xa0\x80",
               b"\xf4\x90\x80\x80", b"\xf0\x8f\xbf\xbf", b"\xc2", b"\xe2\x82", b"\x80", b"\xff"]
    for i, raw in enumerate(samples):
        try:
            raw.decode("utf-8", "strict")
            valid = True
        except UnicodeDecodeError:
            valid = False
        tensors = [(raw, [1], 0, 0)]
        out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 1, 1))
        out += gguf_string("general.architecture") + struct.pack("<I", 8) + gguf_string("llama")
        out += gguf_string(raw) + struct.pack("<IQIQ", 1, 1, 0, 0)
        while len(out) % 32:
            out += b"\0"
        path = write_file(tmp_path, bytes(out) + bytes(32), name=f"u{i}.gguf")
        if valid:
            with S.GgufFile(path) as f:
                assert raw.decode("utf-8") in f.tensors
        else:
            with pytest.raises(S.InvalidDataException):
                S.GgufFile(path)
