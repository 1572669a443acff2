"""Pins the CPU oracle (oracle/) before the GPU tests compare against it.

Every oracle function is checked against at least one of: the reference's golden fixtures
(tests/golden, copied data), the reference tests' known-answer values, FP64 brute force, or an exact
algebraic identity chosen so that a plausible mistake (swapped nibble, dropped centring, wrong sub-block
index) fails. Planted-mistake tests mutate an independent numpy decoder (never the product) and show the
same fixtures reject it.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import (critical_cases, fp64_matvec, gguf_tensor, hexbytes, load_json, rng, special_scale_payload,
                     ternary2_bound)
from oracle import oracle as O

TINY = float(np.finfo(np.float32).smallest_subnormal)
FMAX = float(np.finfo(np.float32).max)


def check_error(code):
    return pytest.raises(O.OracleError, match=O.OracleError.NAMES[code])


# --------------------------------------------------------------------------------------------
# Independent numpy decoders, written from the layout in docs/gguf-subset-v1.md:93-98 and
# Q4KCodec.cs:5-18 / Q6KCodec.cs:6-19. `mistake` plants a plausible error.
# --------------------------------------------------------------------------------------------

def np_q4k_decode(block: np.ndarray, mistake: str = "") -> np.ndarray:
    d = float(block[0:2].view(np.float16)[0])
    dmin = float(block[2:4].view(np.float16)[0])
    s = block[4:16].astype(np.int64)
    qs = block[16:144].astype(np.int64)
    scale, mins = np.zeros(8, np.int64), np.zeros(8, np.int64)
    for j in range(8):
        if j < 4 and mistake != "scale-min-branch":
            scale[j], mins[j] = s[j] & 63, s[j + 4] & 63
        else:
            jj = j if j >= 4 else j + 4
            scale[j] = (s[jj + 4] & 0xF) | ((s[jj - 4] >> 6) << 4)
            mins[j] = (s[jj + 4] >> 4) | ((s[jj] >> 6) << 4)
    w = np.zeros(256)
    for g in range(4):
        lo, hi = qs[32 * g:32 * g + 32] & 15, qs[32 * g:32 * g + 32] >> 4
        if mistake == "nibble-swap":
            lo, hi = hi, lo
        w[64 * g:64 * g + 32] = d * scale[2 * g] * lo - dmin * mins[2 * g]
        w[64 * g + 32:64 * g + 64] = d * scale[2 * g + 1] * hi - dmin * mins[2 * g + 1]
    return w


def np_q6k_decode(block: np.ndarray, mistake: str = "") -> np.ndarray:
    ql, qh = block[:128].astype(np.int64), block[128:192].astype(np.int64)
    sc = block[192:208].view(np.int8).astype(np.int64)
    d = float(block[208:210].view(np.float16)[0])
    w = np.zeros(256)
    offset = 0 if mistake == "no-centring" else 32
    for h in range(2):
        for l in range(32):
            a, b, hb = ql[64 * h + l], ql[64 * h + 32 + l], qh[32 * h + l]
            q = [(a & 15) | ((hb & 3) << 4), (b & 15) | (((hb >> 2) & 3) << 4),
                 (a >> 4) | (((hb >> 4) & 3) << 4), (b >> 4) | (((hb >> 6) & 3) << 4)]
            for k in range(4):
                sub = 8 * h + 2 * k + l // 16 if mistake != "scale-index" else 8 * h + k + l // 16
                w[128 * h + 32 * k + l] = d * sc[sub] * (q[k] - offset)
    return w


# --------------------------------------------------------------------------------------------
# Ternary2
# --------------------------------------------------------------------------------------------

def test_ternary2_encoding_matches_binary_fixture():
    # Ternary2Tests.cs:9-22 and docs/ternary2-v1.md example.
    src = np.zeros(64, np.float32)
    src[0], src[1] = 2, -2
    expected = np.zeros(20, np.uint8)
    expected[2], expected[3], expected[4] = 0x80, 0x3D, 0x09
    assert np.array_equal(O.t2_quantize(src, 1, 64), expected)
    assert np.array_equal(O.t2_quantize(np.zeros(64, np.float32), 1, 64), np.zeros(20, np.uint8))


def test_ternary2_validation_rejects_corrupt_blocks():
    # Ternary2Tests.cs:24-42.
    payload = np.zeros(20, np.uint8)
    payload[:4] = np.frombuffer(np.float32(1).tobytes(), np.uint8)
    payload[4] = 3
    with check_error(1):
        O.t2_validate(payload, 1, 1, 64)
    payload[4] = 4  # non-zero padding after the single valid weight
    with check_error(1):
        O.t2_validate(payload, 1, 1, 64)
    payload[4] = 1
    payload[:4] = 0
    with check_error(1):
        O.t2_validate(payload, 1, 1, 64)
    payload[4] = 0
    for scale in (np.nan, np.inf, -1.0, -0.0):
        payload[:4] = np.frombuffer(np.float32(scale).tobytes(), np.uint8)
        with check_error(1):
            O.t2_validate(payload, 1, 1, 64)
    payload[:4] = np.frombuffer(np.float32(0.5).tobytes(), np.uint8)
    O.t2_validate(payload, 1, 1, 64)
    with check_error(1):
        O.t2_validate(payload[:19], 1, 1, 64)


def test_ternary2_shape_rules():
    # Ternary2Shape.cs:5-15.
    assert O.t2_byte_length(1, 1, 64) == 20
    assert O.t2_byte_length(4096, 4096, 128) == 4718592
    assert O.t2_byte_length(4096, 4096, 64) == 5242880 and O.t2_byte_length(4096, 4096, 256) == 4456448
    for bad in ((0, 1, 64), (1, 0, 64), (1, 1, 32), (1, 1, 100)):
        with check_error(2):
            O.t2_byte_length(*bad)
    with check_error(9):
        O.t2_byte_length(2_000_000, 100_000, 64)


def test_ternary2_quantization_extremes():
    # Ternary2Tests.cs:90-102.
    for value in (FMAX, TINY, 0.0):
        data = O.t2_quantize(np.array([value, -value], np.float32), 1, 2)
        assert O.t2_dequantize(data, 1, 2, 64).tolist() == [[value, -value]]
    for value in (np.nan, np.inf, -np.inf):
        with check_error(1):
            O.t2_quantize(np.array([value], np.float32), 1, 1)


def test_ternary2_readme_demo():
    # src/Satori.Console/Program.cs:169-175, README.md:27.
    data = O.t2_quantize(np.array([2, -2, 0, 0, 1, -1], np.float32), 2, 3)
    assert data.size == 40
    assert O.t2_matvec_scalar(data, 2, 3, 64, [2, -1, 3]).tolist() == [4.0, np.float32(-8 / 3)]
    assert O.t2_matvec_avx2(data, 2, 3, 64, [2, -1, 3]).tolist() == [4.0, np.float32(-8 / 3)]


def test_ternary2_corpus_matches_xorshift_definition():
    # NumericalCorpus.cs:41-47, restated in Python for the first values.
    state, values = 1729, []
    for _ in range(8):
        state ^= (state << 13) & 0xFFFFFFFF
        state ^= state >> 17
        state ^= (state << 5) & 0xFFFFFFFF
        values.append(np.float32((state >> 8) * (1.0 / 8388608.0) - 1))
    w, x = O.corpus_random_matrix(1, 4)
    assert w.reshape(-1).tolist() == [np.float32(v * 2) for v in values[:4]]
    assert x.tolist() == values[4:8]


@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_kernels_within_reference_bound_on_critical_corpus(block):
    # NumericalCorpusTests.cs:149-158 and Ternary2Avx2Tests.cs:115-125, scalar and AVX2 restatements.
    for name, w, x in critical_cases(block):
        rows, columns = w.shape
        data = O.t2_quantize(w, rows, columns, block)
        wq = O.t2_dequantize(data, rows, columns, block)
        bound = ternary2_bound(wq, x, block)
        exact = fp64_matvec(wq, x)
        for kernel in (O.t2_matvec_scalar, O.t2_matvec_avx2):
            y = kernel(data, rows, columns, block, x)
            assert np.all(np.isfinite(y)), name
            assert np.all(np.abs(y - exact) <= bound), (name, kernel.__name__)
        if name == "random":  # quantization error dominates kernel error (NumericalCorpusTests.cs:155-156)
            original = fp64_matvec(w, x)
            assert np.sqrt(np.mean((exact - original) ** 2)) > 100 * np.sqrt(
                np.mean((O.t2_matvec_scalar(data, rows, columns, block, x) - exact) ** 2))


@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_kernels_on_column_tails(block):
    for columns in list(range(1, 18)) + [63, 64, 65, 127, 128, 129, 255, 256, 257]:
        w, x = O.corpus_random_matrix(3, columns)
        data = O.t2_quantize(w, 3, columns, block)
        wq = O.t2_dequantize(data, 3, columns, block)
        for kernel in (O.t2_matvec_scalar, O.t2_matvec_avx2):
            y = kernel(data, 3, columns, block, x)
            assert np.all(np.abs(y - fp64_matvec(wq, x)) <= ternary2_bound(wq, x, block)), (columns, kernel)


def test_ternary2_closed_form_block_sums():
    # y = sum_blocks scale * (sum_{code 1} x - sum_{code 2} x): the scalar kernel in FP32 equals the FP64
    # closed form to FP32 rounding, and a wrong code assignment (+/- swapped) is far outside it.
    g = rng(3)
    w = g.standard_normal((9, 700)).astype(np.float32)
    x = g.uniform(-1, 1, 700).astype(np.float32)
    data = O.t2_quantize(w, 9, 700, 128)
    blocks = (700 + 127) // 128
    closed = np.zeros(9)
    for r in range(9):
        for b in range(blocks):
            off = (r * blocks + b) * 36
            scale = float(data[off:off + 4].view(np.float32)[0])
            codes = np.unpackbits(data[off + 4:off + 36], bitorder="little").reshape(-1, 2)
            c = codes[:, 0] + 2 * codes[:, 1]
            xs = x[b * 128:min(700, b * 128 + 128)].astype(np.float64)
            c = c[:xs.size]
            closed[r] += scale * (xs[c == 1].sum() - xs[c == 2].sum())
    y = O.t2_matvec_scalar(data, 9, 700, 128, x)
    assert np.all(np.abs(y - closed) <= 1e-5 * np.abs(O.t2_dequantize(data, 9, 700, 128)) @ np.abs(x))
    swapped = -closed
    assert np.all(np.abs(y - swapped) > 1e-3)


def test_stq2_header_fixture():
    # MappedTernary2Tests.cs:40-46: exact 32 header bytes for a 1x1 block-64 matrix.
    expected = bytes([0x53, 0x54, 0x51, 0x32, 1, 0, 32, 0, 1, 0, 0, 0, 1, 0, 0, 0,
                      64, 0, 0, 0, 0, 0, 0, 0, 20, 0, 0, 0, 0, 0, 0, 0])
    assert O.stq2_header(1, 1, 64) == expected
    assert O.stq2_read_header(expected) == (1, 1, 64)
    for index in (0, 4, 6, 8, 16, 20, 24):
        corrupt = bytearray(expected)
        corrupt[index] ^= 0xFF
        with check_error(3):
            O.stq2_read_header(bytes(corrupt))


# --------------------------------------------------------------------------------------------
# Q8_0 / Q4_0
# --------------------------------------------------------------------------------------------

@pytest.mark.parametrize("name,fmt", [("q8_0.gguf", O.Q8_0), ("q4_0.gguf", O.Q4_0)])
def test_golden_gguf_decode_and_ones_dot(name, fmt):
    # fixtures/gguf/v1/manifest.json decoded weights; QuantizedTests.cs:168-184 ones-dot = -8.
    payload, entry = gguf_tensor(name)
    assert O.decode_block(payload, fmt).tolist() == entry["decoded_weights"]
    ones = np.ones(32, np.float32)
    assert O.q_matvec_scalar(payload, 1, 32, fmt, ones).tolist() == [-8.0] == [entry["ones_dot_product"]]
    assert O.q_matvec_avx2(payload, 1, 32, fmt, ones).tolist() == [-8.0]


@pytest.mark.parametrize("fmt", [O.Q8_0, O.Q4_0])
def test_legacy_special_scales_match_fp64(fmt):
    # QuantizedTests.cs:186-214 / Q4Tests.cs:239-268 (|err| <= 0.001).
    scales = [0.5, -2.0, 0.0, -0.0, float(np.float16(2 ** -24)), 65504.0, 1.0]
    data = special_scale_payload(fmt, 7, 96, scales)
    x = np.array([(i % 13 - 6) / 16 for i in range(96)], np.float32)
    # Independent FP64: codes and scales read straight from the bytes.
    d = data.reshape(7, 3, O.GEOMETRY[fmt][1])
    sc = d[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    if fmt == O.Q8_0:
        q = d[:, :, 2:].view(np.int8).astype(np.float64)
    else:
        q = np.concatenate([(d[:, :, 2:] & 15).astype(np.float64) - 8, (d[:, :, 2:] >> 4).astype(np.float64) - 8], 2)
    exact = np.einsum("rb,rbj,bj->r", sc, q, x.astype(np.float64).reshape(3, 32))
    for kernel in (O.q_matvec_scalar, O.q_matvec_avx2):
        assert np.all(np.abs(kernel(data, 7, 96, fmt, x) - exact) <= 0.001)


def test_legacy_nonfinite_scales_rejected():
    # QuantizedTests.cs:216-230, Q4Tests.cs:270-278.
    for bits in (0x7C00, 0xFC00, 0x7E00):
        data = np.zeros(34, np.uint8)
        data[0], data[1] = bits & 0xFF, bits >> 8
        with check_error(3):
            O.q_validate(data, 1, 32, O.Q8_0)
        with check_error(3):
            O.q_validate(data[:18], 1, 32, O.Q4_0)
    with check_error(1):
        O.q_validate(np.zeros(33, np.uint8), 1, 32, O.Q8_0)
    with check_error(2):
        O.q_byte_length(1, 128, O.Q4_K)
    assert O.q_byte_length(1, 256, O.Q4_K) == 144


# --------------------------------------------------------------------------------------------
# K formats
# --------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fixture,fmt,decoder", [("q4k-v1.json", O.Q4_K, np_q4k_decode),
                                                 ("q6k-v1.json", O.Q6_K, np_q6k_decode)])
def test_k_decode_and_dot_match_fixture(fixture, fmt, decoder):
    # Q4KCodecTests.cs:392-429, Q6KCodecTests.cs:17-54.
    for case in load_json(fixture)["cases"]:
        block = hexbytes(case["block_hex"])
        ref_w = np.array(case["weights"])
        for w in (O.decode_block(block, fmt), decoder(block)):
            assert np.all(np.abs(w - ref_w) <= 1e-3 + 1e-4 * np.abs(ref_w)), case["name"]
        x = np.array(case["input"], np.float32)
        for y in (O.q_matvec_scalar(block, 1, 256, fmt, x)[0], O.q_matvec_avx2(block, 1, 256, fmt, x)[0]):
            assert abs(y - case["dot"]) <= 1e-2 + 1e-4 * abs(case["dot"]), case["name"]
        if case["name"] == "zero":
            assert np.all(O.decode_block(block, fmt) == 0)


@pytest.mark.parametrize("fixture,fmt,mistakes", [("q4k-v1.json", O.Q4_K, ("nibble-swap", "scale-min-branch")),
                                                  ("q6k-v1.json", O.Q6_K, ("no-centring", "scale-index"))])
def test_k_fixture_rejects_planted_decoder_mistakes(fixture, fmt, mistakes):
    decoder = np_q4k_decode if fmt == O.Q4_K else np_q6k_decode
    cases = load_json(fixture)["cases"]
    for mistake in mistakes:
        caught = False
        for case in cases:
            ref_w = np.array(case["weights"])
            w = decoder(hexbytes(case["block_hex"]), mistake)
            caught |= bool(np.any(np.abs(w - ref_w) > 1e-3 + 1e-4 * np.abs(ref_w)))
        assert caught, f"fixture does not detect planted mistake {mistake}"


def test_k_real_tensor_blocks():
    # KParityTests.cs:177-212.
    for case in load_json("k-real-v1.json")["cases"]:
        fmt = O.Q4_K if case["name"].startswith("q4k:") else O.Q6_K
        raw = hexbytes(case["block_hex"])
        nb = O.GEOMETRY[fmt][1]
        ref_w = np.array(case["weights"])
        x = np.array(case["input"], np.float32)
        for b in range(case["blocks"]):
            block = raw[b * nb:(b + 1) * nb]
            w = O.decode_block(block, fmt)
            assert np.all(np.abs(w - ref_w[b * 256:(b + 1) * 256]) <= 1e-3 + 1e-4 * np.abs(ref_w[b * 256:(b + 1) * 256]))
            dot = O.q4k_dot_block(block, x) if fmt == O.Q4_K else O.q6k_dot_block(block, x)
            assert abs(dot - case["dots"][b]) <= 1e-2 + 1e-4 * abs(case["dots"][b])


def test_k_nonfinite_scales_rejected():
    block = np.zeros(144, np.uint8)
    block[1] = 0x7C  # d = +inf (Q4KCodecTests.cs:441-450)
    with check_error(3):
        O.q_validate(block, 1, 256, O.Q4_K)
    block[1], block[3] = 0, 0x7E  # dmin = NaN
    with check_error(3):
        O.q_validate(block, 1, 256, O.Q4_K)
    q6 = np.zeros(210, np.uint8)
    q6[209] = 0x7C
    with check_error(3):
        O.q_validate(q6, 1, 256, O.Q6_K)


def test_q8k_quantizer_matches_fixture():
    # Q8KCodecTests.cs:22-56: bytes, scale and group sums.
    for case in load_json("q8k-v1.json")["cases"]:
        block = O.q8k_quantize_block(np.array(case["input"], np.float32))
        assert np.array_equal(block, hexbytes(case["block_hex"])), case["name"]
        assert abs(float(block[:4].view(np.float32)[0]) - case["scale"]) <= 1e-6
        assert block[260:292].view(np.int16).tolist() == case["bsums"]
        assert block[4:260].view(np.int8).tolist() == case["codes"]


def test_q8k_row_is_blockwise_and_error_within_one_step():
    # Q8KCodecTests.cs:86-122.
    x = np.sin(np.arange(768) * 0.01).astype(np.float32)
    row = O.q8k_quantize_row(x)
    for b in range(3):
        assert np.array_equal(row[b * 292:(b + 1) * 292], O.q8k_quantize_block(x[b * 256:(b + 1) * 256]))
    u = rng(20261014).uniform(-1, 1, 256).astype(np.float32)
    block = O.q8k_quantize_block(u)
    scale = float(block[:4].view(np.float32)[0])
    codes = block[4:260].view(np.int8).astype(np.float64)
    assert np.all(np.abs(scale * codes - u) <= abs(scale))
    # bsums are the sums of their 16 codes, as int16
    assert np.array_equal(block[260:292].view(np.int16), codes.reshape(16, 16).sum(1).astype(np.int16))
    # first-largest magnitude wins ties: -1 before +1 gives a positive scale...
    tie = np.zeros(256, np.float32)
    tie[3], tie[7] = -1, 1
    assert float(O.q8k_quantize_block(tie)[:4].view(np.float32)[0]) > 0
    tie[3], tie[7] = 1, -1
    assert float(O.q8k_quantize_block(tie)[:4].view(np.float32)[0]) < 0
    assert np.all(O.q8k_quantize_block(np.zeros(256, np.float32)) == 0)


def test_q4k_q8k_dot_matches_fixture_and_zero_activation():
    # Q8KCodecTests.cs:58-84.
    for case in load_json("q8k-v1.json")["cases"]:
        w, a = hexbytes(case["weights_hex"]), hexbytes(case["block_hex"])
        dot = O.q4k_dot_block_quantized(w, a)
        assert abs(dot - case["dot"]) <= 1e-3 + 1e-4 * abs(case["dot"]), case["name"]
    w = hexbytes(load_json("q8k-v1.json")["cases"][0]["weights_hex"])
    a = np.zeros(292, np.uint8)
    a[4:260] = 0x7F
    assert O.q4k_dot_block_quantized(w, a) == 0.0
    zero = O.q8k_quantize_block(np.zeros(256, np.float32))
    assert O.q4k_dot_product(w, zero) == 0 and O.q4k_min_product(w, zero) == 0


def test_q6k_q8k_dot_matches_fixture_composition_and_centring():
    # Q6KQuantizedProductTests.cs:149-259.
    nontrivial = 0
    for case in load_json("q6k-q8k-v1.json")["cases"]:
        w, a = hexbytes(case["weights_hex"]), hexbytes(case["activation_hex"])
        dot = O.q6k_dot_block_quantized(w, a)
        assert abs(dot - case["dot"]) <= 1e-3 + 1e-4 * abs(case["dot"])
        codes = a[4:260].view(np.int8).astype(np.float64)
        scale = float(a[:4].view(np.float32)[0])
        composed = scale * float(O.q6k_decode_block(w).astype(np.float64) @ codes)
        assert abs(dot - composed) <= 1e-3 + 1e-4 * abs(composed)
        d = float(w[208:210].view(np.float16)[0])
        sc = w[192:208].view(np.int8).astype(np.float64)
        offset = 32 * scale * d * float(np.sum(sc * codes.reshape(16, 16).sum(1)))
        nontrivial += abs(offset) > 1e-3
    assert nontrivial > 0
    w = hexbytes(load_json("q6k-q8k-v1.json")["cases"][0]["weights_hex"])
    a = np.zeros(292, np.uint8)
    a[4:260] = 0x7F
    assert O.q6k_dot_block_quantized(w, a) == 0.0


def _k_random_block(fmt, g, d_bits, dmin_bits=0):
    block = g.integers(0, 256, O.GEOMETRY[fmt][1], dtype=np.uint8)
    if fmt == O.Q4_K:
        block[0:2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
        block[2:4] = np.frombuffer(np.uint16(dmin_bits).tobytes(), np.uint8)
    else:
        block[208:210] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
    return block


def test_integer_products_equal_brute_force_through_the_pinned_decoder():
    # With d = 1, dmin = 0 the decoded weights are the integers s_j * q_i (Q4_K) or sc * (q - 32)
    # (Q6_K) exactly, so sum_i w_i * code_i computed from the fixture-pinned decoder must equal
    # DotProduct; with d = 0, dmin = 1 the weights are -m_j and the sum is -MinProduct. Exact.
    g = rng(1)
    one, zero = 0x3C00, 0x0000
    for _ in range(40):
        x = g.standard_normal(256).astype(np.float32) * np.float32(g.uniform(0.01, 100))
        a = O.q8k_quantize_block(x)
        codes = a[4:260].view(np.int8).astype(np.int64)
        b = _k_random_block(O.Q4_K, g, one, zero)
        assert int(round(O.q4k_decode_block(b).astype(np.float64) @ codes)) == O.q4k_dot_product(b, a)
        b = _k_random_block(O.Q4_K, g, zero, one)
        assert int(round(O.q4k_decode_block(b).astype(np.float64) @ codes)) == -O.q4k_min_product(b, a)
        b = _k_random_block(O.Q6_K, g, one)
        assert int(round(O.q6k_decode_block(b).astype(np.float64) @ codes)) == O.q6k_dot_product(b, a)


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q6_K])
def test_batch_restatements_agree_and_equal_compose_row(fmt):
    # The scalar ExecuteBatch restatement, the AVX2 ExecuteQuantizedTiled restatement and ComposeRow
    # (Q6KQuantizedProductTests.cs:351-365) agree bit for bit.
    g = rng(20261014)
    rows, columns = 48, 1024
    payload = g.integers(0, 256, rows * 4 * O.GEOMETRY[fmt][1], dtype=np.uint8)
    nb = O.GEOMETRY[fmt][1]
    for i in range(rows * 4):  # finite scales (Q6KQuantizedProductTests.cs:369-371)
        if fmt == O.Q4_K:
            payload[i * nb:i * nb + 4] = np.frombuffer(np.array([0.01, 0.002], np.float16).tobytes(), np.uint8)
        else:
            payload[i * nb + 208:i * nb + 210] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    x = (np.sin(np.arange(columns) * 0.017) * 0.5).astype(np.float32)
    batch = O.q_matvec_batch(payload, rows, columns, fmt, x, 1)
    avx2 = O.qk_matvec_quantized_avx2(payload, rows, columns, fmt, O.q8k_quantize_row(x))
    assert np.array_equal(batch.view(np.uint32), avx2.view(np.uint32))
    dot = O.q4k_dot_block_quantized if fmt == O.Q4_K else O.q6k_dot_block_quantized
    for r in range(rows):
        total = np.float32(0)
        for b in range(4):
            total = np.float32(total + np.float32(dot(payload[(r * 4 + b) * nb:(r * 4 + b + 1) * nb],
                                                      O.q8k_quantize_block(x[b * 256:(b + 1) * 256]))))
        assert total.view(np.uint32) == batch[r].view(np.uint32)


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q6_K])
def test_tiled_restatement_equals_per_position(fmt):
    # ExecuteQuantizedTiled over several positions (the tiled form the CPU baseline of the prefill times)
    # gives, position by position, the bits of the one-position restatement and of the scalar ExecuteBatch
    # (QuantizedMatVec.cs:136-219), including a zero position and positions with zero blocks.
    g = rng(7 + fmt)
    rows, columns, positions = 40, 1024, 7
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    import satori_amd as S
    payload = S.quantize_weights(w, rows, columns, S.BlockQuantization(fmt))
    x = g.standard_normal((positions, columns)).astype(np.float32)
    x[2] = 0.0
    x[4, 256:512] = 0.0
    x[5] *= np.float32(1e-30)
    acts = np.concatenate([O.q8k_quantize_row(x[p]) for p in range(positions)])
    tiled = O.qk_matvec_quantized_tiled_avx2(payload, rows, columns, fmt, acts, positions)
    batch = O.q_matvec_batch(payload, rows, columns, fmt, x.reshape(-1), positions)
    assert np.array_equal(tiled.view(np.uint32), batch.view(np.uint32))
    for p in range(positions):
        single = O.qk_matvec_quantized_avx2(payload, rows, columns, fmt, O.q8k_quantize_row(x[p]))
        assert np.array_equal(tiled[p * rows:(p + 1) * rows].view(np.uint32), single.view(np.uint32)), p
    with pytest.raises(ValueError):
        O.qk_matvec_quantized_tiled_avx2(payload, rows, columns, fmt, np.zeros(257 * 4 * 292, np.uint8), 257)


@pytest.mark.parametrize("fmt,fixture,rows,columns,positions", [
    (O.Q4_K, "q4k-v1.json", 2, 512, 4), (O.Q4_K, "q4k-v1.json", 3, 512, 1), (O.Q6_K, "q6k-v1.json", 2, 256, 8)])
def test_batch_within_activation_quantization_bound(fmt, fixture, rows, columns, positions):
    # BatchedMatVecTests.cs:61-113: |batch - per-position scalar| <= sum_blocks sum|w| * max|x| / 254.
    blocks = [hexbytes(c["block_hex"]) for c in load_json(fixture)["cases"]]
    nbr = columns // 256
    data = np.concatenate([blocks[i % len(blocks)] for i in range(rows * nbr)])
    x = np.array([[np.sin(p * 0.37 + c * 0.011) * 1.5 for c in range(columns)] for p in range(positions)], np.float32)
    batch = O.q_matvec_batch(data, rows, columns, fmt, x.reshape(-1), positions)
    wq = O.decode_matrix(data, rows, columns, fmt)
    for p in range(positions):
        single = O.q_matvec_scalar(data, rows, columns, fmt, x[p])
        largest = np.abs(x[p]).reshape(nbr, 256).max(1)
        bound = (np.abs(wq).reshape(rows, nbr, 256).sum(2) * (largest / 254.0)).sum(1)
        assert np.all(np.abs(batch[p * rows:(p + 1) * rows] - single) <= bound)


def test_k_avx2_float_matches_scalar():
    # KParityTests.cs:246-270.
    for fixture, fmt in (("q4k-v1.json", O.Q4_K), ("q6k-v1.json", O.Q6_K)):
        cases = load_json(fixture)["cases"]
        for first, second in ((cases[0], cases[1]), (cases[4], cases[7])):
            payload = np.concatenate([hexbytes(first["block_hex"]), hexbytes(second["block_hex"])])
            x = np.array([((i % 17) - 8) * 0.5 for i in range(512)], np.float32)
            s = O.q_matvec_scalar(payload, 1, 512, fmt, x)[0]
            v = O.q_matvec_avx2(payload, 1, 512, fmt, x)[0]
            assert abs(s - v) <= 1e-3 + 1e-4 * abs(s)
