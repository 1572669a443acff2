"""The no-allocation grouped attention (satori_hip_grouped_attention_static) through the C ABI: the same
results as satori_hip_grouped_attention bit for bit (the same kernels), within one unit in the last place of
the oracle, on consecutive calls of decreasing size (the static workspace keeps the last call's partials),
recordable into a graph on a fresh context without any warm-up call, and a clear error past its size."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import satori_amd as S
from helpers import rng
from oracle import oracle as O

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _within_ulp(actual, expected, name):
    a, e = np.asarray(actual, np.float32), np.asarray(expected, np.float32)
    spacing = np.spacing(np.maximum(np.abs(a), np.abs(e)).astype(np.float32)).astype(np.float64)
    err = np.abs(a.astype(np.float64) - e.astype(np.float64))
    assert np.all(err <= spacing), f"{name}: max err {err.max()}"


def _status(code):
    if code != 0:
        raise AssertionError(f"status {code}: {S._ffi.lib().satori_hip_last_error().decode()}")


def test_static_attention_equals_allocating_entry_point():
    lib = S._ffi.lib()
    with S.HipContext(0) as ctx:
        h = ctx.handle
        buffers = []

        def dev(arr):
            p = ctx.alloc(arr.nbytes)
            ctx.upload(p, arr)
            buffers.append(p)
            return p

        try:
            g = rng(4711)
            # Two calls in a row, the second smaller (fewer tokens and heads), then a single-workgroup prefix.
            for tokens, heads, kv_heads, head_dim in ((5000, 12, 2, 128), (300, 6, 3, 96), (20, 4, 2, 64)):
                q = g.standard_normal(heads * head_dim).astype(np.float32)
                k = (g.standard_normal(tokens * kv_heads * head_dim) * 0.3).astype(np.float32)
                v = g.standard_normal(tokens * kv_heads * head_dim).astype(np.float32)
                dq, dk, dv = dev(q), dev(k), dev(v)
                out_static, out_ref = dev(np.zeros(heads * head_dim, np.float32)), dev(np.zeros(heads * head_dim, np.float32))
                _status(lib.satori_hip_grouped_attention_static(h, P(dq), P(dk), P(dv), heads, kv_heads, head_dim,
                                                                tokens, P(out_static), None))
                _status(lib.satori_hip_grouped_attention(h, P(dq), P(dk), P(dv), heads, kv_heads, head_dim, tokens,
                                                         P(out_ref), None))
                got = ctx.download(np.zeros(heads * head_dim, np.float32), out_static)
                want = ctx.download(np.zeros(heads * head_dim, np.float32), out_ref)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), tokens
                _within_ulp(got, O.grouped_attention(q, k, v, heads, kv_heads, head_dim, tokens), f"{tokens} tokens")
            # Past the static workspace: 64 heads of 256 lanes over 32 splits need 4,227,072 bytes of partials.
            q, k = dev(np.zeros(64 * 256, np.float32)), dev(np.zeros(1024 * 256, np.float32))
            out = dev(np.zeros(64 * 256, np.float32))
            code = lib.satori_hip_grouped_attention_static(h, P(q), P(k), P(k), 64, 1, 256, 1024, P(out), None)
            assert code == S.ArgumentOutOfRangeException.status
            assert b"static workspace" in lib.satori_hip_last_error()
        finally:
            for p in buffers:
                ctx.free(p)


def test_static_attention_captures_without_warm_up():
    # A fresh context records the attention into a graph with no earlier call (nothing to allocate); each
    # replay, with eager attentions of another size between them, gives the eager result.
    lib = S._ffi.lib()
    with S.HipContext(0) as ctx:
        h = ctx.handle
        g = rng(99)
        tokens, other = 3000, 700
        q = g.standard_normal(12 * 128).astype(np.float32)
        k = (g.standard_normal(tokens * 256) * 0.3).astype(np.float32)
        v = g.standard_normal(tokens * 256).astype(np.float32)
        arrays = [q, k, v, np.zeros(12 * 128, np.float32), np.zeros(12 * 128, np.float32)]
        dq, dk, dv, dout, dother = (ctx.alloc(a.nbytes) for a in arrays)
        for p, a in zip((dq, dk, dv, dout, dother), arrays):
            ctx.upload(p, a)
        try:
            ctx.capture_begin()
            try:
                _status(lib.satori_hip_grouped_attention_static(h, P(dq), P(dk), P(dv), 12, 2, 128, tokens, P(dout),
                                                                None))
            finally:
                step = ctx.capture_end()
            expected = O.grouped_attention(q, k, v, 12, 2, 128, tokens)
            first = None
            for replay in range(3):
                ctx.upload(dout, np.zeros(12 * 128, np.float32))
                _status(lib.satori_hip_grouped_attention_static(h, P(dq), P(dk), P(dv), 12, 2, 128, other, P(dother),
                                                                None))
                step.execute()
                got = ctx.download(np.zeros(12 * 128, np.float32), dout)
                _within_ulp(got, expected, f"replay {replay}")
                first = got if first is None else first
                assert np.array_equal(got.view(np.uint32), first.view(np.uint32)), replay
            step.dispose()
        finally:
            for p in (dq, dk, dv, dout, dother):
                ctx.free(p)
