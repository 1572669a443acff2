"""Decode-step operators (src/Satori.Core/TransformerOps.cs): the oracle's FP64 restatements pinned against the
reference's independent float64 fixtures (fixtures/operators/transformer-v1.json and -v2.json, copied to
tests/golden/) with the reference's own tolerance, plus the closed forms of TransformerOpsTests.cs and
QwenOperatorTests.cs. No GPU (the device kernels are checked in test_gpu_parity.py)."""
from __future__ import annotations

import numpy as np

from helpers import load_json, rng
from oracle import oracle as O

FMAX = np.finfo(np.float32).max


def within_fixture(actual, expected, name):
    # TransformerOpsTests.cs:13-16 / QwenOperatorTests.cs:19-26: |a - e| <= 2e-6 + 2e-6 |e|, finite.
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, name
    assert np.all(np.isfinite(actual)), name
    err = np.abs(actual - expected)
    assert np.all(err <= 2e-6 + 2e-6 * np.abs(expected)), f"{name}: max err {err.max()}"


def f32(values):
    return np.asarray(values, np.float32)


def test_oracle_matches_transformer_v1_fixture():
    # TransformerOpsTests.cs:8-25.
    d = load_json("transformer-v1.json")
    within_fixture(O.rms_norm(f32(d["x"]), f32(d["weights"]), np.float32(1e-5)), d["rms"], "rms")
    within_fixture(O.rope(f32(d["x"]), 48, 37), d["rope"], "rope")
    within_fixture(O.swiglu(f32(d["gate"]), f32(d["up"])), d["swiglu"], "swiglu")
    within_fixture(O.grouped_attention(f32(d["query"]), f32(d["keys"]), f32(d["values"]), 2, 2, 48, 7),
                   d["attention"], "attention")


def test_oracle_matches_transformer_v2_fixture():
    # QwenOperatorTests.cs:28-112.
    d = load_json("transformer-v2.json")
    g = d["gqa"]
    within_fixture(O.grouped_attention(f32(g["query"]), f32(g["keys"]), f32(g["values"]), g["query_heads"],
                                       g["kv_heads"], g["head_dim"], g["tokens"]), g["output"], "gqa")
    for key in ("rope_full", "rope_partial"):
        r = d[key]
        within_fixture(O.rope_half(f32(r["input"]), r["head_dim"], r["position"], r["base"], r["rotary"]),
                       r["output"], key)
    n = d["qk_norm"]
    within_fixture(O.rms_norm_heads(f32(n["input"]), f32(n["weights"]), np.float32(n["epsilon"]), len(n["weights"])),
                   n["output"], "qk_norm")
    b = d["bias"]
    within_fixture(O.add(f32(b["base"]), f32(b["bias"])), b["output"], "bias")


def test_oracle_closed_forms():
    # TransformerOpsTests.cs:27-43 (extreme finite values), QwenOperatorTests.cs:45-61 (grouped attention with
    # equal heads is plain attention), TransformerOpsTests.cs:55-63 (Q8_0 row decode).
    assert O.rms_norm(f32([FMAX, -FMAX]), f32([1, 1]), np.float32(1e-5)).tolist() == [1.0, -1.0]
    q = f32([FMAX, FMAX])
    k = f32([FMAX, FMAX, -FMAX, -FMAX])
    assert O.grouped_attention(q, k, f32([3, 4, 100, 200]), 1, 1, 2, 2).tolist() == [3.0, 4.0]
    g = rng(11)
    q, k, v = (g.random(n).astype(np.float32) for n in (8, 24, 24))
    grouped = O.grouped_attention(q, k, v, 2, 2, 4, 3)
    # An independent FP64 computation of plain attention per head.
    expected = np.zeros(8)
    for h in range(2):
        s = np.array([np.dot(q[4 * h:4 * h + 4].astype(np.float64), k[8 * t + 4 * h:8 * t + 4 * h + 4]) for t in range(3)])
        s = np.exp(s / 2.0 - (s / 2.0).max())
        expected[4 * h:4 * h + 4] = (s / s.sum()) @ v.reshape(3, 8)[:, 4 * h:4 * h + 4].astype(np.float64)
    assert np.allclose(grouped, expected, rtol=1e-6, atol=1e-7)
    row = np.zeros(34, np.uint8)
    row[1] = 0xB8  # FP16 -0.5
    row[2:] = (np.arange(32) * 8 - 128).astype(np.int8).view(np.uint8)
    assert O.q_decode_row(row, 32, 0).tolist() == [float((i * 8 - 128) * -0.5) for i in range(32)]
    # A swapped sigmoid branch or a dropped weight factor would fail these.
    assert abs(O.swiglu(f32([-30.0]), f32([1.0]))[0] - (-30.0 / (1 + np.exp(30.0)))) < 1e-16
    assert O.rms_norm(f32([3.0, 4.0]), f32([2.0, 0.5]), np.float32(1e-30)).tolist() == \
        [np.float32(3 / np.sqrt(12.5) * 2), np.float32(4 / np.sqrt(12.5) * 0.5)]


def test_oracle_matches_attention_boundary_fixture():
    # VulkanAttentionTests.cs:17-29 against fixtures/operators/attention-boundaries-v1.json: 6 heads of 48
    # lanes (query and key/value heads alike), 1, 2, 32, 64 and 128 tokens, |a - e| <= 2e-6 + 2e-6 |e|, and
    # the negated values give the negated output. The fixture's reading (score = q.k / sqrt(48), max-subtracted
    # softmax, weighted value sum, one key/value head per query head) is pinned by an FP64 brute force that
    # reproduces it to 1e-12.
    from helpers import attention_boundary_case

    q, keys, values, cases = attention_boundary_case()
    assert sorted(cases) == [1, 2, 32, 64, 128]
    for count, expected in cases.items():
        brute = np.zeros(288)
        for h in range(6):
            lanes = slice(48 * h, 48 * h + 48)
            scores = keys[:count, lanes].astype(np.float64) @ q[lanes].astype(np.float64) / np.sqrt(48.0)
            e = np.exp(scores - scores.max())
            brute[lanes] = (e / e.sum()) @ values[:count, lanes].astype(np.float64)
        assert np.all(np.abs(brute - expected) <= 1e-12 * (1 + np.abs(expected))), f"{count}: brute force"
        k, v = keys[:count].reshape(-1), values[:count].reshape(-1)
        within_fixture(O.grouped_attention(q, k, v, 6, 6, 48, count), expected, f"attention {count}")
        within_fixture(-O.grouped_attention(q, k, -v, 6, 6, 48, count), expected, f"negated {count}")
