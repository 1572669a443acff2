"""GPU parity at the benchmark's own workloads, through the C ABI: the exact grouped launches bench.py times
(every resident copy's output of the first launch against the oracle), the Qwen-1.5B-shaped output
projection (151,936 x 1,536 Q6_K) at batch 1, the prefill projections at 256 positions on the matrix cores,
and the whole 28-layer decode token at positions 511 and 4095 checked launch by launch against the oracle.

Bars: FP32 products within 1e-5 * sum_i |w_i x_i| per row of the oracle's scalar restatement; integer K
products and the Q8_K path identical (32-bit patterns); the decode-step operators within one unit in the
last place of the oracle applied to the device's own inputs (Add and the row decode exactly).
"""
from __future__ import annotations

import numpy as np
import pytest

import bench
import satori_amd as S
from helpers import rng
from oracle import oracle as O

pytestmark = pytest.mark.gpu

BQ = S.BlockQuantization


def fp32_bound(data, rows, columns, fmt, x, block=None):
    """1e-5 * sum_i |w_i x_i| per row (FP64) on the decoded weights, decoded row by row by the oracle."""
    ax = np.abs(x.astype(np.float64))
    if fmt is None:
        w = O.t2_dequantize(data, rows, columns, block)
        return 1e-5 * (np.abs(w.astype(np.float64)) @ ax)
    row_bytes = data.size // rows
    out = np.empty(rows)
    for r in range(rows):
        out[r] = np.abs(O.q_decode_row(data[r * row_bytes:(r + 1) * row_bytes], columns, int(fmt))) @ ax
    return 1e-5 * out


def case_expected(data, rows, columns, fmt, x, quantized):
    """(expected outputs, bound or None for bit-exact) of one benchmark case."""
    if fmt is None:  # Ternary2, block size in `quantized`
        return O.t2_matvec_scalar(data, rows, columns, quantized, x), fp32_bound(data, rows, columns, None, x,
                                                                                  quantized)
    if quantized:
        return O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x)), None
    return O.q_matvec_scalar(data, rows, columns, int(fmt), x), fp32_bound(data, rows, columns, fmt, x)


def check_all_copies(context, case, expected, bound, label):
    case.run_group()
    context.synchronize()
    for i, dy in enumerate(case.dy):
        y = context.download(np.zeros(case.rows, np.float32), dy)
        if bound is None:
            assert np.array_equal(y.view(np.uint32), expected.view(np.uint32)), f"{label} copy {i}"
        else:
            err = np.abs(y.astype(np.float64) - expected)
            assert np.all(np.isfinite(y)) and np.all(err <= bound), f"{label} copy {i}: max err {err.max()}"


def test_headline_grouped_launch_every_copy_matches_oracle(context):
    # The timed headline: one grouped launch over 228 resident copies of the seeded 4096 x 4096 B128 matrix
    # (1.076 GB of payload, 1,024 persistent workgroups with cut items finished by the fix-up kernel).
    payload, x = bench.make_ternary2(4096, 4096, 128)
    case = bench.Case(context, "ternary2-4096-b128", lambda: context.create_ternary2(4096, 4096, 128, payload),
                      payload.size, 4096, 4096, x, False)
    try:
        assert case.copies == 228
        expected, bound = case_expected(payload, 4096, 4096, None, x, 128)
        check_all_copies(context, case, expected, bound, "headline")
        check_all_copies(context, case, expected, bound, "headline, second launch")
    finally:
        case.close()


@pytest.mark.parametrize("index", range(9))
def test_benchmark_format_cases_every_copy_matches_oracle(context, index):
    # Every other `formats` case of the benchmark, built exactly as it builds them.
    label, make = bench.other_formats(context)[index]
    case, (data, rows, columns, fmt, x, quantized) = make()
    try:
        expected, bound = case_expected(data, rows, columns, fmt, x, quantized)
        check_all_copies(context, case, expected, bound, label)
    finally:
        case.close()


def test_output_projection_151936x1536_q6k_batch_one(context):
    # The decode token's output projection (DenseForward.cs:298-306) at its Qwen-1.5B shape, as the benchmark
    # builds it (a 4,096-row seeded Q6_K matrix repeated to 151,936 rows), on the Q8_K integer path at one
    # position: host ExecuteBatch and the resident group launch, both bit-exact.
    vocab, d = 151936, 1536
    base, _ = bench.make_gguf(BQ.Q6_K, 4096, d)
    row_bytes = base.size // 4096
    tiled = np.tile(base.reshape(4096, row_bytes), (-(-vocab // 4096), 1))[:vocab].reshape(-1)
    m = context.create(tiled, S.QuantizedMatrixShape(vocab, d, BQ.Q6_K))
    x = rng(151936).standard_normal(d).astype(np.float32)
    expected_base = O.qk_matvec_quantized_avx2(base, 4096, d, O.Q6_K, O.q8k_quantize_row(x))
    expected = expected_base[np.arange(vocab) % 4096]
    y = np.zeros(vocab, np.float32)
    m.execute_batch(x, 1, y)
    assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))
    dx, dy = context.alloc(x.nbytes), context.alloc(4 * vocab)
    context.upload(dx, x)
    group = S.HipGroup(context, [m], [dx], [dy], True)
    group.execute()
    got = context.download(np.zeros(vocab, np.float32), dy)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    group.dispose()
    context.free(dx)
    context.free(dy)
    m.dispose()


@pytest.mark.parametrize("names", [("down",), ("o",), ("q", "k", "v"), ("gate", "up")])
def test_prefill_projections_256_positions_on_matrix_cores(context, names):
    # The prefill's 256-position chunk at the Qwen-1.5B shapes (1536 x 8960 Q6_K down, 1536 x 1536 Q4_K o
    # through ExecuteBatch; the q/k/v and gate/up groups sharing one packed input) against the oracle's
    # per-position ExecuteQuantizedTiled composition, bit for bit.
    roles = {"q": (1536, 1536, BQ.Q4_K), "k": (256, 1536, BQ.Q4_K), "v": (256, 1536, BQ.Q4_K),
             "o": (1536, 1536, BQ.Q4_K), "gate": (8960, 1536, BQ.Q4_K), "up": (8960, 1536, BQ.Q4_K),
             "down": (1536, 8960, BQ.Q6_K)}
    positions = 256
    columns = roles[names[0]][1]
    x = rng(256 + columns).standard_normal((positions, columns)).astype(np.float32)
    x[17] = 0  # an all-zero position
    datas = {n: bench.make_gguf(roles[n][2], roles[n][0], roles[n][1])[0] for n in names}
    mats = {n: context.create(datas[n], S.QuantizedMatrixShape(*roles[n])) for n in names}
    dx = context.alloc(x.nbytes)
    context.upload(dx, x)
    outs = {n: context.alloc(4 * positions * roles[n][0]) for n in names}
    try:
        if len(names) == 1:
            mats[names[0]].execute_batch_device(dx, positions, outs[names[0]])
        else:
            group = S.HipGroup(context, [mats[n] for n in names], [dx] * len(names), [outs[n] for n in names], True)
            group.execute_batch(positions)
            context.synchronize()
            group.dispose()
        quantized = [O.q8k_quantize_row(x[p]) for p in range(positions)]
        for n in names:
            rows, cols, fmt = roles[n]
            y = context.download(np.zeros(positions * rows, np.float32), outs[n]).reshape(positions, rows)
            for p in range(positions):
                expected = O.qk_matvec_quantized_avx2(datas[n], rows, cols, int(fmt), quantized[p])
                assert np.array_equal(y[p].view(np.uint32), expected.view(np.uint32)), f"{n} position {p}"
    finally:
        for p in list(outs.values()) + [dx]:
            context.free(p)
        for m in mats.values():
            m.dispose()


# ---------------------------------------------------------------------------------------------
# The whole Qwen-1.5B-shaped decode token, launch by launch
# ---------------------------------------------------------------------------------------------

def _ulp_close(actual, expected, name, ulps=1):
    a, e = np.asarray(actual, np.float32), np.asarray(expected, np.float32)
    spacing = np.spacing(np.maximum(np.abs(a), np.abs(e)).astype(np.float32)).astype(np.float64)
    err = np.abs(a.astype(np.float64) - e.astype(np.float64))
    assert np.all(err <= ulps * spacing), f"{name}: max err {err.max()} at {np.argmax(err - ulps * spacing)}"


def _bits(actual, expected, name):
    assert np.array_equal(np.asarray(actual, np.float32).view(np.uint32),
                          np.asarray(expected, np.float32).view(np.uint32)), name


@pytest.fixture(scope="module")
def qwen_model(context):
    """The benchmark's Qwen-1.5B-shaped model (28 layers of distinct resident copies of one seeded layer, the
    151,936-row output projection tied to the embedding) plus host copies of its payloads for the oracle."""
    model = bench.DecodeModel(context)
    host = {n: bench.make_gguf(fmt, r, c)[0] for n, (r, c, fmt) in model.roles.items()}
    base, _ = bench.make_gguf(BQ.Q6_K, 4096, model.D)
    row_bytes = base.size // 4096
    host["output"] = np.tile(base.reshape(4096, row_bytes), (-(-model.VOCAB // 4096), 1))[:model.VOCAB].reshape(-1)
    yield model, host
    model.close()


@pytest.mark.parametrize("position", [511, 4095])
def test_qwen_decode_token_launch_by_launch_matches_oracle(context, qwen_model, position):
    # DenseForward.Step / Final (DenseForward.cs:100-162, 298-306) at full size: hidden 1536, 28 layers,
    # 12 / 2 heads of 128, FFN 8960, vocab 151,936, a random key/value prefix of `position` tokens. The fused
    # operator sequence runs one launch at a time; each projection's output equals the oracle's projection of
    # the device's own input bit for bit, each operator's output is within one unit in the last place of the
    # oracle applied to the device's inputs (Add and the row decode exactly). The captured folded token, the
    # benchmark's timed form, then gives the same logits bit for bit.
    from satori_amd.decode import DecoderConfig, DeviceDecoder
    model, host = qwen_model
    d, kv, ffn, vocab = model.D, model.KV, model.FFN, model.VOCAB
    g = rng(2029 + position)
    cfg = DecoderConfig(hidden=d, heads=12, kv_heads=2, head_dim=128, ffn=ffn, epsilon=1e-6, rope_base=1e6,
                        max_tokens=position + 1)
    buffers, vecs_host, vecs_dev = [], [], []

    def dev(a):
        p = context.alloc(a.nbytes)
        context.upload(p, a)
        buffers.append(p)
        return p

    for _ in model.layers:
        vh = {"attn_norm": g.uniform(0.5, 1.5, d).astype(np.float32), "ffn_norm": g.uniform(0.5, 1.5, d).astype(np.float32),
              "q_bias": (g.standard_normal(d) * 0.1).astype(np.float32),
              "k_bias": (g.standard_normal(kv) * 0.1).astype(np.float32),
              "v_bias": (g.standard_normal(kv) * 0.1).astype(np.float32)}
        vecs_host.append(vh)
        vecs_dev.append({k: dev(v) for k, v in vh.items()})
    out_norm_host = g.uniform(0.5, 1.5, d).astype(np.float32)
    dec = DeviceDecoder(context, cfg, model.layers, vecs_dev, dev(out_norm_host), model.output, model.output)
    try:
        for layer in range(len(model.layers)):
            prefix = (g.standard_normal((cfg.max_tokens, kv)) * 0.5).astype(np.float32)
            context.upload(dec.keys[layer], prefix)
            context.upload(dec.values[layer], prefix[::-1].copy())
        token = int(g.integers(0, vocab))
        ops = dec.ops

        def get(ptr, n):
            context.synchronize()
            return context.download(np.zeros(n, np.float32), ptr)

        def proj(name, x, rows, cols, fmt):
            return O.qk_matvec_quantized_avx2(host[name], rows, cols, int(fmt), O.q8k_quantize_row(x))

        dec.embedding.decode_row_device(token, dec.residual)
        rb = host["output"].size // vocab
        _bits(get(dec.residual, d), O.q_decode_row(host["output"][token * rb:(token + 1) * rb], d, O.Q6_K), "embedding")
        residual = get(dec.residual, d)
        ops.rms_norm(dec.residual, vecs_dev[0]["attn_norm"], cfg.epsilon, d, dec.normed)
        _ulp_close(get(dec.normed, d), O.rms_norm(residual, vecs_host[0]["attn_norm"], np.float32(cfg.epsilon)),
                   "rms_norm 0")
        for layer, (grp, vh, vd) in enumerate(zip(dec.groups, vecs_host, vecs_dev)):
            tag = f"layer {layer}"
            k_slot = dec.keys[layer] + 4 * position * kv
            v_slot = dec.values[layer] + 4 * position * kv
            normed = get(dec.normed, d)
            grp["qkv"].execute()
            q, k, v = get(dec.q, d), get(dec.k, kv), get(dec.v, kv)
            _bits(q, proj("q", normed, d, d, BQ.Q4_K), f"{tag} q")
            _bits(k, proj("k", normed, kv, d, BQ.Q4_K), f"{tag} k")
            _bits(v, proj("v", normed, kv, d, BQ.Q4_K), f"{tag} v")
            ops.attention_inputs(dec.q, vd["q_bias"], dec.k, vd["k_bias"], k_slot, dec.v, vd["v_bias"], v_slot,
                                 12, 2, 128, position, cfg.rope_base, 128)
            q2 = get(dec.q, d)
            _ulp_close(q2, O.rope_half(O.add(q, vh["q_bias"]), 128, position, cfg.rope_base, 128), f"{tag} rope q")
            _ulp_close(get(k_slot, kv), O.rope_half(O.add(k, vh["k_bias"]), 128, position, cfg.rope_base, 128),
                       f"{tag} rope k")
            _bits(get(v_slot, kv), O.add(v, vh["v_bias"]), f"{tag} v slot")
            ops.grouped_attention(dec.q, dec.keys[layer], dec.values[layer], 12, 2, 128, position + 1,
                                  dec.context_vec)
            keys = get(dec.keys[layer], (position + 1) * kv)
            values = get(dec.values[layer], (position + 1) * kv)
            ctx_vec = get(dec.context_vec, d)
            _ulp_close(ctx_vec, O.grouped_attention(q2, keys, values, 12, 2, 128, position + 1), f"{tag} attention")
            grp["o"].execute()
            projected = get(dec.projected, d)
            _bits(projected, proj("o", ctx_vec, d, d, BQ.Q4_K), f"{tag} o")
            residual = get(dec.residual, d)
            ops.add_rms_norm(dec.residual, dec.projected, vd["ffn_norm"], cfg.epsilon, d, dec.normed)
            residual = O.add(residual, projected)
            _bits(get(dec.residual, d), residual, f"{tag} residual after attention")
            _ulp_close(get(dec.normed, d), O.rms_norm(residual, vh["ffn_norm"], np.float32(cfg.epsilon)),
                       f"{tag} ffn norm")
            normed = get(dec.normed, d)
            grp["gateup"].execute()
            gate, up = get(dec.gate, ffn), get(dec.up, ffn)
            _bits(gate, proj("gate", normed, ffn, d, BQ.Q4_K), f"{tag} gate")
            _bits(up, proj("up", normed, ffn, d, BQ.Q4_K), f"{tag} up")
            ops.swiglu(dec.gate, dec.up, ffn, dec.activated)
            act = get(dec.activated, ffn)
            _ulp_close(act, O.swiglu(gate, up), f"{tag} swiglu")
            grp["down"].execute()
            projected = get(dec.projected, d)
            _bits(projected, proj("down", act, d, ffn, BQ.Q6_K), f"{tag} down")
            following = vecs_dev[layer + 1]["attn_norm"] if layer + 1 < len(dec.groups) else dec.output_norm
            following_host = vecs_host[layer + 1]["attn_norm"] if layer + 1 < len(dec.groups) else out_norm_host
            ops.add_rms_norm(dec.residual, dec.projected, following, cfg.epsilon, d, dec.normed)
            residual = O.add(residual, projected)
            _bits(get(dec.residual, d), residual, f"{tag} residual after FFN")
            _ulp_close(get(dec.normed, d), O.rms_norm(residual, following_host, np.float32(cfg.epsilon)),
                       f"{tag} next norm")
        normed = get(dec.normed, d)
        dec.final.execute()
        logits = get(dec.logits, vocab)
        _bits(logits, proj("output", normed, vocab, d, BQ.Q6_K), "logits")
        assert np.all(np.isfinite(logits))
        # The benchmark's timed form: the folded token captured once and replayed, same logits bit for bit.
        # The step rewrites this position's cache slots with the same values.
        step = dec.capture(token, position, folded=True)
        for replay in range(2):
            context.upload(dec.logits, np.zeros(vocab, np.float32))
            step.execute()
            _bits(dec.read_logits(), logits, f"captured folded token, replay {replay}")
        step.dispose()
    finally:
        dec.dispose()
        for p in buffers:
            context.free(p)
