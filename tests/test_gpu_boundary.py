"""GPU tests of the drop-in boundary's edges against the oracle, through the C ABI: non-finite activations
where the reference takes them, integer K products of any width, grouped attention over long prefixes and
odd head widths, split-attention workspaces per stream, and the operators' argument rules inside group
input transforms.

Bars: FP32 products |y_gpu - y_ref| <= 1e-5 * sum_i |w_i x_i| per finite row, and NaN / +Inf / -Inf exactly
where the oracle has them; integer K products identical to the oracle (NaN where the oracle has NaN, every
other output the same 32 bits); attention within one unit in the last place of the oracle.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import satori_amd as S
from helpers import relative_bound, rng
from oracle import oracle as O

pytestmark = pytest.mark.gpu

BQ = S.BlockQuantization


def assert_same_specials_within(actual, expected, bound, what=""):
    """NaN, +Inf and -Inf exactly where the oracle has them; finite outputs within the bound."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert np.array_equal(np.isnan(a), np.isnan(e)), f"{what}: NaN positions differ"
    assert np.array_equal(np.isposinf(a), np.isposinf(e)), f"{what}: +Inf positions differ"
    assert np.array_equal(np.isneginf(a), np.isneginf(e)), f"{what}: -Inf positions differ"
    finite = np.isfinite(e)
    err = np.abs(a[finite] - e[finite])
    assert np.all(err <= np.asarray(bound)[finite]), f"{what}: max err {err.max() if err.size else 0}"


def assert_bits_or_nan(actual, expected, what=""):
    """Integer K products: NaN where the oracle has NaN, otherwise the same 32-bit pattern."""
    a, e = np.asarray(actual, np.float32), np.asarray(expected, np.float32)
    assert np.array_equal(np.isnan(a), np.isnan(e)), f"{what}: NaN positions differ"
    keep = ~np.isnan(e)
    bad = np.nonzero(a[keep].view(np.uint32) != e[keep].view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size} outputs differ, first {bad[:5]}"


def _t2_payload(g, rows, columns, block):
    blocks = -(-columns // block)
    codes = g.integers(0, 3, size=(rows, blocks * block), dtype=np.uint8)
    codes[:, columns:] = 0
    return codes, blocks


def _t2_pack(codes, scales, rows, blocks, block):
    packed = codes[:, 0::4] | (codes[:, 1::4] << 2) | (codes[:, 2::4] << 4) | (codes[:, 3::4] << 6)
    out = np.concatenate([scales.view(np.uint8).reshape(rows, blocks, 4), packed.reshape(rows, blocks, block // 4)],
                         axis=2)
    return np.ascontiguousarray(out.reshape(-1))


# ---------------------------------------------------------------------------------------------
# Non-finite activations
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("columns", [1000, 5000])
@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_nonfinite_inputs_propagate_like_the_reference(context, block, columns):
    # Ternary2MatVec.Execute takes any activations (Ternary2MatVec.cs:30-36) and skips code-0 weights
    # (:64-70), so a row is finite when its codes at the non-finite columns are all zero, +-Inf when it
    # adds one infinity, NaN when it adds both or a NaN. Rows are built for each case. At 5000 columns the
    # single-matrix plan cuts each row into five column slices joined by atomic exchanges, and the
    # non-finite columns lie in different slices, so the specials travel through the exchanges.
    g = rng(9090 + block + columns)
    rows = 257
    codes, blocks = _t2_payload(g, rows, columns, block)
    x = g.uniform(-1, 1, columns).astype(np.float32)
    pos_inf, neg_inf, nan = 3, columns // 2 + 17, columns - 100
    x[pos_inf], x[neg_inf], x[nan] = np.inf, -np.inf, np.nan
    special = [pos_inf, neg_inf, nan]
    for r in range(rows):
        kind = r % 5
        codes[r, special] = 0
        if kind == 1:
            codes[r, pos_inf] = 1       # +Inf
        elif kind == 2:
            codes[r, pos_inf] = 2       # -Inf
        elif kind == 3:
            codes[r, [pos_inf, neg_inf]] = 1  # +Inf + -Inf: NaN
        elif kind == 4:
            codes[r, nan] = 1 + r % 2   # NaN
    scales = g.uniform(0.01, 2.0, size=(rows, blocks)).astype(np.float32)
    payload = _t2_pack(codes, scales, rows, blocks, block)
    m = context.create_ternary2(rows, columns, block, payload)
    y = np.zeros(rows, np.float32)
    m.execute(x, y)  # accepted: no ArgumentException for the Ternary2 surface
    m.dispose()
    expected = O.t2_matvec_scalar(payload, rows, columns, block, x)
    wq = O.t2_dequantize(payload, rows, columns, block)
    xf = np.where(np.isfinite(x), x, 0).astype(np.float32)
    assert_same_specials_within(y, expected, relative_bound(wq, xf), f"Ternary2 B{block}")
    assert np.isfinite(y[0::5]).all() and np.isposinf(y[1::5]).all() and np.isnan(y[3::5]).all()


def test_gguf_plugin_seam_still_rejects_nonfinite_inputs(context):
    # IQuantizedMatrix.Execute of a GPU backend rejects them (VulkanQ8Matrix.cs:82-83); the batched surface
    # (QuantizedMatVec.ExecuteBatch) takes them.
    g = rng(31)
    data = S.quantize_weights((g.standard_normal((8, 64)) * 0.1).astype(np.float32), 8, 64, BQ.Q8_0)
    m = context.create(data, S.QuantizedMatrixShape(8, 64, BQ.Q8_0))
    x = np.ones(64, np.float32)
    x[5] = np.nan
    sentinel = np.full(8, 7.0, np.float32)
    with pytest.raises(S.ArgumentException):
        m.execute(x, sentinel)
    assert np.all(sentinel == 7.0)
    m.execute_batch(x, 1, sentinel)
    assert np.isnan(sentinel).any()
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
def test_legacy_batch_nonfinite_inputs_propagate(context, fmt):
    # QuantizedMatVec.ExecuteBatch float path with non-finite activations: a zero weight times an infinity
    # is NaN in the reference's products too (QuantizedMatVec.cs:221-281), so the specials land where the
    # oracle's do; finite rows within the bound.
    g = rng(404 + int(fmt))
    rows, columns, positions = 96, 512, 3
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    w[:, 40:48] = 0  # rows whose codes are zero at the non-finite columns
    data = S.quantize_weights(w, rows, columns, fmt)
    x = g.standard_normal((positions, columns)).astype(np.float32)
    x[0, 44] = np.inf       # only zero weights: NaN in every row (0 * Inf)
    x[1, 100] = -np.inf
    x[2, 300] = np.nan
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.zeros(positions * rows, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    m.dispose()
    wq = O.decode_matrix(data, rows, columns, int(fmt))
    for p in range(positions):
        expected = O.q_matvec_scalar(data, rows, columns, int(fmt), x[p])
        xf = np.where(np.isfinite(x[p]), x[p], 0).astype(np.float32)
        assert_same_specials_within(y[p * rows:(p + 1) * rows], expected, relative_bound(wq, xf), f"{fmt.name} p{p}")


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("positions", [1, 3, 20])
def test_k_batch_nonfinite_inputs_match_the_reference_bits(context, fmt, positions):
    # Q8KCodec.QuantizeBlock with infinities and NaNs (Q8KCodec.cs:44-76): NaN never wins the maximum, an
    # all-NaN-or-zero block quantizes to zero and is skipped, an infinite maximum gives inverse -0, codes 0
    # and scale -Inf, whose block term is NaN. The integer kernel (1-15 positions) and the matrix-core
    # kernel (16+) both follow it.
    g = rng(77 + 10 * int(fmt) + positions)
    rows, columns = 200, 2048
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    x = g.standard_normal((positions, columns)).astype(np.float32)
    for p in range(positions):
        kind = p % 4
        if kind == 0:
            x[p, 256 + 7] = np.nan                       # NaN inside a finite block
        elif kind == 1:
            x[p, 512:768] = 0
            x[p, 512 + 3] = np.nan                       # NaN in an otherwise zero block: a zero block
        elif kind == 2:
            x[p, 1024 + 9] = np.inf                      # infinite block maximum
        else:
            x[p, 1536 + 1], x[p, 1536 + 2] = -np.inf, np.inf
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.zeros(positions * rows, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    m.dispose()
    for p in range(positions):
        expected = O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x[p]))
        assert_bits_or_nan(y[p * rows:(p + 1) * rows], expected, f"{fmt.name} position {p}")
    for p in range(min(positions, 4)):
        q = S.Q8KCodec.quantize_row(x[p], context)
        assert np.array_equal(q, O.q8k_quantize_row(x[p])), f"Q8_K bytes, position {p}"


# ---------------------------------------------------------------------------------------------
# Integer K products of any width (QuantizedKAvx2Kernel.ExecuteQuantizedTiled has no width limit)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("rows,columns,positions", [(300, 29696, 1), (300, 29696, 3), (130, 29696, 16),
                                                    (70, 65536, 1), (33, 57344, 2)])
def test_k_batch_wide_rows_are_bit_exact(context, fmt, rows, columns, positions):
    # Rows wider than one staging of the Q8_K row (112 blocks = 28,672 columns) are summed chunk by chunk in
    # block order; 29,696 (116 blocks), 57,344 (two whole chunks) and 65,536 (256 blocks, a ragged last chunk).
    g = rng(5150 + columns + rows + int(fmt))
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    x = g.standard_normal((positions, columns)).astype(np.float32)
    x[0, 256 * 113:256 * 114] = 0  # a zero block in the second chunk is skipped
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.zeros(positions * rows, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    m.dispose()
    for p in range(positions):
        expected = O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x[p]))
        got = y[p * rows:(p + 1) * rows]
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), f"position {p}"


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
def test_wide_group_with_input_transform_equals_operator_then_group(context, fmt):
    # A decode-step group at 29,696 columns computing RmsNorm(a + b) inside its launch equals the operator
    # followed by the plain group (and the oracle's projection of the operator's output) bit for bit.
    g = rng(8181 + int(fmt))
    columns, rows = 29696, [64, 40]
    datas = [S.quantize_weights((g.standard_normal((r, columns)) * 0.02).astype(np.float32), r, columns, fmt)
             for r in rows]
    mats = [context.create(d, S.QuantizedMatrixShape(r, columns, fmt)) for d, r in zip(datas, rows)]
    a, b = (g.standard_normal(columns).astype(np.float32) for _ in range(2))
    w = g.uniform(0.5, 1.5, columns).astype(np.float32)
    buffers = []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    da, db, dw = dev(a), dev(b), dev(w)
    dsum, dx = dev(a.copy()), dev(np.zeros(columns, np.float32))
    plain_out = [dev(np.zeros(r, np.float32)) for r in rows]
    fused_out = [dev(np.zeros(r, np.float32)) for r in rows]
    plain = S.HipGroup(context, mats, [dx, dx], plain_out, True)
    fused = S.HipGroup(context, mats, [dx, dx], fused_out, True)
    try:
        ops = S.DeviceOps(context)
        ops.add_rms_norm(dsum, db, dw, 1e-6, columns, dx)
        plain.execute()
        fused.set_input_add_rms_norm(da, db, dw, 1e-6)
        fused.execute()
        normed = context.download(np.zeros(columns, np.float32), dx)
        for k, r in enumerate(rows):
            want = context.download(np.zeros(r, np.float32), plain_out[k])
            got = context.download(np.zeros(r, np.float32), fused_out[k])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"member {k}"
            expected = O.qk_matvec_quantized_avx2(datas[k], r, columns, int(fmt), O.q8k_quantize_row(normed))
            assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), f"member {k} vs oracle"
    finally:
        plain.dispose()
        fused.dispose()
        for p in buffers:
            context.free(p)
        for m in mats:
            m.dispose()


def test_group_input_transform_rejects_nonpositive_epsilon(context):
    # RmsNorm's rule (TransformerOps.cs:17) holds inside a group's input transform: epsilon must be positive.
    data = S.quantize_weights(np.zeros((4, 256), np.float32), 4, 256, BQ.Q4_K)
    m = context.create(data, S.QuantizedMatrixShape(4, 256, BQ.Q4_K))
    bufs = [context.alloc(4 * 256) for _ in range(4)]
    group = S.HipGroup(context, [m], [bufs[0]], [bufs[1]], True)
    try:
        for eps in (0.0, -1e-6, float("nan"), float("inf")):
            with pytest.raises(S.ArgumentOutOfRangeException):
                group.set_input_add_rms_norm(bufs[2], bufs[3], bufs[3], eps)
        group.set_input_add_rms_norm(bufs[2], bufs[3], bufs[3], 1e-6)
    finally:
        group.dispose()
        for p in bufs:
            context.free(p)
        m.dispose()


# ---------------------------------------------------------------------------------------------
# Grouped attention: any prefix length and head width (TransformerOps.cs:135-179 has no cap)
# ---------------------------------------------------------------------------------------------

def _within_ulp(actual, expected, name, ulps=1):
    a, e = np.asarray(actual, np.float32), np.asarray(expected, np.float32)
    spacing = np.spacing(np.maximum(np.abs(a), np.abs(e)).astype(np.float32)).astype(np.float64)
    err = np.abs(a.astype(np.float64) - e.astype(np.float64))
    assert np.all(err <= ulps * spacing), f"{name}: max err {err.max()} at {np.argmax(err - ulps * spacing)}"


@pytest.mark.parametrize("tokens", [4097, 6913, 8192, 16384, 32768, 70001, 131073])
def test_attention_long_prefixes_match_oracle(context, tokens):
    # Qwen-1.5B heads (12 query, 2 key/value, 128 lanes): 32 splits up to 4,096 tokens, then splits of 128
    # tokens up to 64 (6,913 tokens: 55 splits), then 64 splits of up to 2,048 tokens.
    g = rng(tokens)
    q = g.standard_normal(12 * 128).astype(np.float32)
    keys = (g.standard_normal(tokens * 256) * 0.3).astype(np.float32)
    values = g.standard_normal(tokens * 256).astype(np.float32)
    out = np.zeros(12 * 128, np.float32)
    S.TransformerOps.grouped_attention(q, keys, values, 12, 2, 128, tokens, out, context)
    _within_ulp(out, O.grouped_attention(q, keys, values, 12, 2, 128, tokens), f"attention {tokens}")


@pytest.mark.parametrize("head_dim,tokens,query_heads,kv_heads", [(80, 300, 14, 2), (80, 7000, 4, 1),
                                                                  (24, 100, 3, 3), (1024, 100, 4, 2),
                                                                  (8320, 40, 2, 1), (130, 33, 6, 3),
                                                                  (1024, 4096, 2, 1), (200, 4096, 2, 1),
                                                                  (8320, 4096, 2, 1)])
def test_attention_odd_head_widths_match_oracle(context, head_dim, tokens, query_heads, kv_heads):
    # Head widths whose eighths are not whole 16-byte quads (80, 24, 130, 200), wider than one workgroup's lanes
    # (1024) and wider than the staged query (8,320 lanes: read from global memory); at 4,096 and 7,000 tokens
    # the splits hold 128 tokens and run on 512-thread workgroups (four token parts per lane).
    g = rng(head_dim * 7 + tokens)
    q = g.standard_normal(query_heads * head_dim).astype(np.float32)
    keys = (g.standard_normal(tokens * kv_heads * head_dim) * 0.2).astype(np.float32)
    values = g.standard_normal(tokens * kv_heads * head_dim).astype(np.float32)
    out = np.zeros(query_heads * head_dim, np.float32)
    S.TransformerOps.grouped_attention(q, keys, values, query_heads, kv_heads, head_dim, tokens, out, context)
    _within_ulp(out, O.grouped_attention(q, keys, values, query_heads, kv_heads, head_dim, tokens),
                f"attention {head_dim} x {tokens}")


@pytest.mark.parametrize("query_heads,kv_heads,head_dim,tokens", [(12, 2, 128, 4096), (12, 2, 128, 2049),
                                                                  (28, 4, 128, 3000), (32, 4, 64, 8192),
                                                                  (4, 1, 80, 7000), (18, 2, 128, 4096)])
def test_grouped_query_split_equals_per_head_split(context, query_heads, kv_heads, head_dim, tokens):
    # Query heads sharing a key/value head: the same attention with every key/value head repeated once per
    # query head (one query head per key/value head) must give the same bits, whichever workgroup layout each
    # takes (one workgroup per key/value head serving its query heads, or one per query head), and both must
    # match the oracle. Group sizes 6, 7, 8 and 4 (80 lanes: eighths of 10 lanes), and 9 (past the grouped
    # form's 8).
    g = rng(query_heads * 1000 + tokens)
    group = query_heads // kv_heads
    q = g.standard_normal(query_heads * head_dim).astype(np.float32)
    keys = (g.standard_normal((tokens, kv_heads, head_dim)) * 0.3).astype(np.float32)
    values = g.standard_normal((tokens, kv_heads, head_dim)).astype(np.float32)
    out = np.zeros(query_heads * head_dim, np.float32)
    S.TransformerOps.grouped_attention(q, keys.reshape(-1), values.reshape(-1), query_heads, kv_heads, head_dim,
                                       tokens, out, context)
    wide_k = np.repeat(keys, group, axis=1).reshape(-1)
    wide_v = np.repeat(values, group, axis=1).reshape(-1)
    per_head = np.zeros(query_heads * head_dim, np.float32)
    S.TransformerOps.grouped_attention(q, wide_k, wide_v, query_heads, query_heads, head_dim, tokens, per_head,
                                       context)
    assert np.array_equal(out.view(np.uint32), per_head.view(np.uint32))
    _within_ulp(out, O.grouped_attention(q, keys.reshape(-1), values.reshape(-1), query_heads, kv_heads, head_dim,
                                         tokens), f"attention {query_heads}/{kv_heads} x {tokens}")


def _hip():
    rt = ctypes.CDLL("libamdhip64.so.7")
    rt.hipStreamCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    rt.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    rt.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    return rt


def test_split_attentions_on_two_streams_do_not_share_a_workspace(context):
    # Two split attentions enqueued back to back on two streams (default priority) run concurrently; each
    # stream has its own partials, so both results equal the oracle's.
    S._ffi.lib()
    rt = _hip()
    streams = [ctypes.c_void_p(), ctypes.c_void_p()]
    for s in streams:
        assert rt.hipStreamCreateWithFlags(ctypes.byref(s), 1) == 0  # non-blocking, default priority
    g = rng(2468)
    tokens = [3000, 5000]
    cases, buffers = [], []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    try:
        for t in tokens:
            q = g.standard_normal(12 * 128).astype(np.float32)
            k = (g.standard_normal(t * 256) * 0.3).astype(np.float32)
            v = g.standard_normal(t * 256).astype(np.float32)
            cases.append((q, k, v, t, dev(q), dev(k), dev(v), dev(np.zeros(12 * 128, np.float32))))
        ops = S.DeviceOps(context)
        for repeat in range(3):
            for (q, k, v, t, dq, dk, dv, do), s in zip(cases, streams):
                ops.grouped_attention(dq, dk, dv, 12, 2, 128, t, do, stream=s.value)
            for s in streams:
                assert rt.hipStreamSynchronize(s) == 0
            for q, k, v, t, dq, dk, dv, do in cases:
                out = context.download(np.zeros(12 * 128, np.float32), do)
                _within_ulp(out, O.grouped_attention(q, k, v, 12, 2, 128, t), f"stream attention {t} #{repeat}")
    finally:
        for s in streams:
            rt.hipStreamDestroy(s)
        for p in buffers:
            context.free(p)


def test_attention_boundary_fixture(context):
    # VulkanAttentionTests.cs:17-29 with fixtures/operators/attention-boundaries-v1.json: 6 heads of 48 lanes at
    # 1, 2, 32, 64 and 128 tokens (across the one-workgroup form's 32-token limit), within 2e-6 + 2e-6 |e| of the
    # reference's FP64 outputs, and the negated values within the same bound of the negated outputs. Three
    # entry points: the grouped attention (host buffers), its no-allocation form, and the decode form (the
    # attention inputs of position count - 1 applied in the launch). The decode form rotates the query and the
    # new key by RopeHalf at that position; rotations keep dot products, so with the cached keys rotated by the
    # same angle (the oracle's RopeHalf, rounded to FP32) it computes the fixture's attention up to those
    # roundings (1.8% of the bound in the oracle).
    from helpers import attention_boundary_case

    q, keys, values, cases = attention_boundary_case()
    ops = S.DeviceOps(context)
    buffers = []

    def dev(arr):
        p = context.alloc(max(arr.nbytes, 4))
        context.upload(p, np.ascontiguousarray(arr))
        buffers.append(p)
        return p

    def check(actual, expected, name):
        err = np.abs(np.asarray(actual, np.float64) - expected)
        assert np.all(np.isfinite(actual)), name
        assert np.all(err <= 2e-6 + 2e-6 * np.abs(expected)), f"{name}: max err {err.max()}"

    try:
        for count, expected in cases.items():
            for sign in (1, -1):
                v = (sign * values[:count]).astype(np.float32)
                out = np.zeros(288, np.float32)
                S.TransformerOps.grouped_attention(q, keys[:count].reshape(-1), v.reshape(-1), 6, 6, 48, count, out,
                                                   context)
                check(sign * out, expected, f"grouped attention {count} sign {sign}")
                dout = dev(np.zeros(288, np.float32))
                ops.grouped_attention_static(dev(q), dev(keys[:count]), dev(v), 6, 6, 48, count, dout)
                check(sign * context.download(np.zeros(288, np.float32), dout), expected,
                      f"static attention {count} sign {sign}")
                position = count - 1
                cache_k = np.stack([O.rope_half(keys[j], 48, position, 10000.0, 48) for j in range(count)])
                cache_k[position] = 0.0  # written by the launch
                cache_v = v.copy()
                cache_v[position] = 0.0
                dq, dck, dcv = dev(q), dev(cache_k), dev(cache_v)
                dout = dev(np.zeros(288, np.float32))
                ops.attention_decode(dq, 0, dev(keys[position]), 0, dev(v[position]), 0, dck, dcv, 6, 6, 48, position,
                                     10000.0, 48, dout)
                check(sign * context.download(np.zeros(288, np.float32), dout), expected,
                      f"decode attention {count} sign {sign}")
    finally:
        for p in buffers:
            context.free(p)


@pytest.mark.parametrize("position,heads,kv_heads,head_dim,rotary,biases", [
    (0, 12, 2, 128, 128, True), (31, 12, 2, 128, 128, True), (32, 12, 2, 128, 128, True),
    (511, 12, 2, 128, 128, True), (2047, 12, 2, 128, 128, True), (2048, 12, 2, 128, 128, True),
    (2559, 12, 2, 128, 128, True), (2560, 12, 2, 128, 128, True),
    (4095, 12, 2, 128, 128, False), (70000, 4, 2, 128, 64, True),
    (300, 14, 2, 80, 80, True), (100, 3, 3, 24, 16, False), (65, 4, 1, 1024, 512, True)])
def test_attention_decode_equals_inputs_then_attention(context, position, heads, kv_heads, head_dim, rotary, biases):
    # satori_hip_attention_decode (the attention inputs applied inside the split attention) against
    # satori_hip_attention_inputs + satori_hip_grouped_attention: the output, the rotated query and the cache
    # rows written at `position` are the same bits; the rest of the cache is untouched.
    g = rng(position * 31 + head_dim)
    qw, kw = heads * head_dim, kv_heads * head_dim
    tokens = position + 1
    q = g.standard_normal(qw).astype(np.float32)
    k = g.standard_normal(kw).astype(np.float32)
    v = g.standard_normal(kw).astype(np.float32)
    qb, kb, vb = ((g.standard_normal(n) * 0.1).astype(np.float32) for n in (qw, kw, kw))
    cache_k = (g.standard_normal(tokens * kw) * 0.3).astype(np.float32)
    cache_v = g.standard_normal(tokens * kw).astype(np.float32)
    buffers = []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    ops = S.DeviceOps(context)
    try:
        results = []
        for fused in (False, True):
            dq, dk, dv = dev(q), dev(k), dev(v)
            dqb, dkb, dvb = (dev(a) if biases else 0 for a in (qb, kb, vb))
            dck, dcv = dev(cache_k), dev(cache_v)
            out = dev(np.zeros(qw, np.float32))
            if fused:
                table = context.alloc(8 * (position + 1) * rotary)
                buffers.append(table)
                ops.rope_table(position + 1, rotary, 1e6, table)
                ops.attention_decode(dq, dqb, dk, dkb, dv, dvb, dck, dcv, heads, kv_heads, head_dim, position, 1e6,
                                     rotary, out, table if position % 2 else 0)
            else:
                ops.attention_inputs(dq, dqb, dk, dkb, dck + 4 * position * kw, dv, dvb, dcv + 4 * position * kw,
                                     heads, kv_heads, head_dim, position, 1e6, rotary)
                ops.grouped_attention(dq, dck, dcv, heads, kv_heads, head_dim, tokens, out)
            results.append([context.download(np.zeros(n, np.float32), p) for p, n in
                            ((out, qw), (dq, qw), (dck, tokens * kw), (dcv, tokens * kw))])
        for name, a, b in zip(("output", "query", "keys", "values"), *results):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
        assert np.array_equal(results[1][2][:position * kw], cache_k[:position * kw])
        expected = O.grouped_attention(results[0][1], results[0][2], results[0][3], heads, kv_heads, head_dim, tokens)
        _within_ulp(results[1][0], expected, "fused attention vs oracle")
    finally:
        for p in buffers:
            context.free(p)
