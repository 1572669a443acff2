"""Ternary bitplane layout (src/Satori.Core/TernaryBitplaneMatrix.cs, TernaryBitplaneMatVec.cs): validation,
the lossless Ternary2 conversions and the STB1 file, through the library (satori_hip_bitplane_*) and the
oracle, against the reference's tests (tests/Satori.Numerics.Tests/TernaryBitplaneTests.cs). No GPU."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import satori_amd as S
from helpers import critical_cases, rng
from oracle import oracle as O


def golden_payload() -> np.ndarray:
    # TernaryBitplaneTests.cs:11-15: one row of 8 columns, B = 64, scale 0.5, positive plane 0x89 (weights 0,
    # 3, 7), negative plane 0x14 (weights 2, 4).
    p = np.zeros(20, np.uint8)
    p[:4] = np.frombuffer(struct.pack("<f", 0.5), np.uint8)
    p[4], p[12] = 0x89, 0x14
    return p


def test_independent_golden_and_codec_reject_invalid_planes():
    # TernaryBitplaneTests.cs:9-37.
    p = golden_payload()
    m = S.TernaryBitplaneMatrix.from_packed(1, 8, 64, p)
    ones = np.ones(8, np.float32)
    assert O.tb_matvec_scalar(p, 1, 8, 64, ones).tolist() == [0.5]
    t2 = m.to_ternary2().data
    assert (t2[4], t2[5]) == (0x61, 0x42)
    assert np.array_equal(t2, O.tb_to_t2(p, 1, 8, 64))
    for defect in range(5):
        bad = p.copy()
        if defect == 0:
            bad[12] |= 1              # weight 0 in both planes
        elif defect == 1:
            bad[5] = 1                # a bit past the last column
        else:
            bad[:4] = np.frombuffer(struct.pack("<f", [-0.0, float("nan"), 0.0][defect - 2]), np.uint8)
        with pytest.raises(S.ArgumentException):
            S.TernaryBitplaneMatrix.from_packed(1, 8, 64, bad)
        with pytest.raises(O.OracleError):
            O.tb_validate(bad, 1, 8, 64)


@pytest.mark.parametrize("block", [64, 128, 256])
def test_corpus_round_trip_preserves_every_byte_and_scalar_result(block):
    # TernaryBitplaneTests.cs:39-58: FromTernary2 then ToTernary2 gives the same bytes, and the bitplane
    # scalar product equals the Ternary2 scalar product exactly.
    for name, w, x in critical_cases(block):
        rows, columns = w.shape
        t2 = S.Ternary2Matrix.quantize(w, rows, columns, block)
        tb = S.TernaryBitplaneMatrix.from_ternary2(t2)
        assert np.array_equal(tb.data, O.tb_from_t2(t2.data, rows, columns, block)), name
        assert np.array_equal(tb.to_ternary2().data, t2.data), name
        expected = O.t2_matvec_scalar(t2.data, rows, columns, block, x)
        actual = O.tb_matvec_scalar(tb.data, rows, columns, block, x)
        assert np.array_equal(expected.view(np.uint32), actual.view(np.uint32)), name


@pytest.mark.parametrize("block", [64, 128, 256])
def test_random_payloads_convert_and_validate_like_the_oracle(block):
    # Random valid payloads (ragged columns, zero-scale blocks) convert identically in the library and the
    # oracle; single-bit corruptions are accepted or rejected by both alike.
    g = rng(31 + block)
    for columns in (1, 7, 8, 9, 63, 64, 65, block - 1, block + 1, 3 * block + 5):
        rows = 3
        w = g.standard_normal((rows, columns)).astype(np.float32)
        w[1, : min(columns, block)] = 0.0  # a zero-scale block
        t2 = S.Ternary2Matrix.quantize(w, rows, columns, block)
        tb = O.tb_from_t2(t2.data, rows, columns, block)
        O.tb_validate(tb, rows, columns, block)
        mine = S.TernaryBitplaneMatrix.from_ternary2(t2)
        assert np.array_equal(mine.data, tb)
        for _ in range(40):
            bad = tb.copy()
            bad[g.integers(0, bad.size)] ^= np.uint8(1 << int(g.integers(0, 8)))
            try:
                O.tb_validate(bad, rows, columns, block)
                oracle_ok = True
            except O.OracleError:
                oracle_ok = False
            try:
                S.TernaryBitplaneMatrix.from_packed(rows, columns, block, bad)
                library_ok = True
            except S.ArgumentException:
                library_ok = False
            assert oracle_ok == library_ok


def test_file_header_is_independent_and_truncations_reject(tmp_path):
    # TernaryBitplaneTests.cs:60-80.
    p = golden_payload()
    m = S.TernaryBitplaneMatrix.from_packed(1, 8, 64, p)
    path = str(tmp_path / "m.stb1")
    m.save(path)
    with open(path, "rb") as f:
        data = f.read()
    assert data[:4] == b"STB1"
    assert struct.unpack_from("<H", data, 4)[0] == 1
    assert struct.unpack_from("<q", data, 24)[0] == 20
    loaded = S.TernaryBitplaneMatrix.load(path)
    assert np.array_equal(loaded.data, p) and (loaded.rows, loaded.columns, loaded.block_size) == (1, 8, 64)
    for length in range(len(data)):
        cut = str(tmp_path / f"cut{length}.stb1")
        with open(cut, "wb") as f:
            f.write(data[:length])
        with pytest.raises(S.InvalidDataException):
            S.TernaryBitplaneMatrix.load(cut)
    # An STQ2 header, an invalid payload and a wrong declared length are invalid files too.
    for mutate in (lambda b: b"STQ2" + b[4:], lambda b: b[:44] + bytes([b[44] | 1]) + b[45:],
                   lambda b: b[:24] + struct.pack("<q", 21) + b[32:]):
        bad = str(tmp_path / "bad.stb1")
        with open(bad, "wb") as f:
            f.write(mutate(data))
        with pytest.raises(S.InvalidDataException):
            S.TernaryBitplaneMatrix.load(bad)
