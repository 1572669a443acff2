"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI (satori_amd -> libsatori_hip.so).

Bars (the tolerance is written in each test):
  * FP32-activation products (Ternary2, Q8_0, Q4_0, Q4_K, Q6_K): |y_gpu - y_ref| <= 1e-5 * sum_i |w_i x_i|
    per row (+ the reference's subnormal floor), against the FP64 product on the decoded weights and the
    oracle's scalar restatement; plus the reference's own gamma bounds where its tests use them.
  * Q8_K activation bytes: identical.
  * Integer K products (ExecuteBatch): identical FP32 outputs to the oracle's ExecuteQuantizedTiled
    composition.
"""
from __future__ import annotations

import numpy as np
import pytest

import satori_amd as S
from helpers import (critical_cases as _critical_cases, fp64_matvec, gguf_tensor, hexbytes, load_json,
                     relative_bound, rng, special_scale_payload as _special_scale_payload, ternary2_bound)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TINY = float(np.finfo(np.float32).smallest_subnormal)
BQ = S.BlockQuantization


def assert_within(actual, expected, bound, what=""):
    actual = np.asarray(actual, dtype=np.float64)
    err = np.abs(actual - np.asarray(expected, dtype=np.float64))
    assert np.all(np.isfinite(actual)), f"{what}: non-finite output"
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, f"{what}: rows {bad[:8]} err {err[bad[:8]]} bound {np.asarray(bound)[bad[:8]]}"


def run(matrix: S.HipQuantizedMatrix, x: np.ndarray) -> np.ndarray:
    y = np.zeros(matrix.rows, dtype=np.float32)
    matrix.execute(x.astype(np.float32), y)
    return y


# ---------------------------------------------------------------------------------------------
# Ternary2
# ---------------------------------------------------------------------------------------------

def test_ternary2_demo_matches_reference_output(context):
    # src/Satori.Console/Program.cs:169-175 and README.md:27: [4, -2.6666667], 40 bytes.
    m = S.Ternary2Matrix.quantize(np.array([2, -2, 0, 0, 1, -1], np.float32), 2, 3)
    assert m.byte_length == 40
    y = np.zeros(2, np.float32)
    S.Ternary2MatVec.execute(m, np.array([2, -1, 3], np.float32), y, context)
    assert y.tolist() == O.t2_matvec_scalar(m.data, 2, 3, 64, [2, -1, 3]).tolist() == [4.0, np.float32(-8 / 3)]


@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_critical_corpus_within_reference_bound(context, block):
    # Ternary2Avx2Tests.cs:115-125 / NumericalCorpusTests.cs:149-158: error/bound <= 1 for every row.
    for name, w, x in _critical_cases(block):
        rows, columns = w.shape
        payload = O.t2_quantize(w, rows, columns, block)
        m = context.create_ternary2(rows, columns, block, payload)
        y = run(m, x)
        wq = O.t2_dequantize(payload, rows, columns, block)
        expected = fp64_matvec(wq, x)
        assert_within(y, expected, ternary2_bound(wq, x, block), f"{name} B{block}")
        scalar = O.t2_matvec_scalar(payload, rows, columns, block, x)
        assert_within(y, scalar, relative_bound(wq, x) + (columns + 8) * TINY, f"{name} B{block} vs scalar")
        m.dispose()


@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_column_tails(context, block):
    # Ternary2Avx2Tests.cs:120-124: columns 1..17, 63..65, 127..129, 255..257, corpus rows.
    for columns in list(range(1, 18)) + [63, 64, 65, 127, 128, 129, 255, 256, 257, 4099]:
        w, x = O.corpus_random_matrix(3, columns)
        payload = O.t2_quantize(w, 3, columns, block)
        m = context.create_ternary2(3, columns, block, payload)
        y = run(m, x)
        wq = O.t2_dequantize(payload, 3, columns, block)
        assert_within(y, fp64_matvec(wq, x), ternary2_bound(wq, x, block), f"C={columns} B{block}")
        m.dispose()


@pytest.mark.parametrize("size", [1024, 2048, 4096])
@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_benchmark_shapes_match_scalar_reference(context, size, block):
    # The benchmark matrices: N(0,1) weights quantized by Ternary2Matrix.Quantize, x ~ U(-1, 1).
    g = rng(1729 + size + block)
    w = g.standard_normal((size, size), dtype=np.float32)
    x = g.uniform(-1, 1, size).astype(np.float32)
    payload = S.Ternary2Matrix.quantize(w, size, size, block).data
    assert np.array_equal(payload, O.t2_quantize(w, size, size, block)), "quantizer bytes differ from oracle"
    m = context.create_ternary2(size, size, block, payload)
    y = run(m, x)
    again = run(m, x)  # repeated calls agree bitwise
    assert np.array_equal(y.view(np.uint32), again.view(np.uint32))
    wq = O.t2_dequantize(payload, size, size, block)
    bound = relative_bound(wq, x)
    assert_within(y, O.t2_matvec_scalar(payload, size, size, block, x), bound, "vs scalar reference")
    assert_within(y, fp64_matvec(wq, x), bound, "vs FP64")
    m.dispose()


def _t2_random_payload(g, rows: int, columns: int, block: int) -> np.ndarray:
    """Valid Ternary2 payload with uniform codes in {0, +1, -1} and positive scales; padding codes zero."""
    blocks = -(-columns // block)
    codes = g.integers(0, 3, size=(rows, blocks * block), dtype=np.uint8)
    codes[:, columns:] = 0
    packed = codes[:, 0::4] | (codes[:, 1::4] << 2) | (codes[:, 2::4] << 4) | (codes[:, 3::4] << 6)
    scales = g.uniform(0.01, 2.0, size=(rows, blocks)).astype(np.float32)
    out = np.concatenate([scales.view(np.uint8).reshape(rows, blocks, 4),
                          packed.reshape(rows, blocks, block // 4)], axis=2)
    return np.ascontiguousarray(out.reshape(-1))


# Ternary2 launches split the columns over workgroups (a second kernel adds the splits) unless the rows
# alone give about 1024 workgroups of 4, 8 or 16 panels of 64 rows. Small shapes above cover the split plans;
# the tests below cover the unsplit ones (one and two panels per wave) through very tall matrices and
# grouped launches, with ragged columns, an odd block count for B = 64, members whose rows end inside a
# panel, the widest slice one workgroup stages (14,336 columns) and a grouped launch split for width.
@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_tall_matrix_pair_tables(context, block):
    g = rng(4242 + block)
    base_rows, columns = 1031, 1050
    base = _t2_random_payload(g, base_rows, columns, block)
    x = g.uniform(-1, 1, columns).astype(np.float32)
    rows = 1024 * 256 + 77
    row_bytes = base.size // base_rows
    payload = np.tile(base.reshape(base_rows, row_bytes), (-(-rows // base_rows), 1))[:rows].reshape(-1)
    m = context.create_ternary2(rows, columns, block, payload)
    y = run(m, x)
    m.dispose()
    wq = O.t2_dequantize(base, base_rows, columns, block)
    scalar = O.t2_matvec_scalar(base, base_rows, columns, block, x)
    index = np.arange(rows) % base_rows
    assert_within(y, scalar[index], relative_bound(wq, x)[index], f"tall B{block} vs scalar")
    assert_within(y, fp64_matvec(wq, x)[index], relative_bound(wq, x)[index], f"tall B{block} vs FP64")


@pytest.mark.parametrize("columns,members", [(4099, 128), (14336, 64), (14337, 64)])
@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_grouped_pair_tables(context, block, columns, members):
    g = rng(777 + block + columns)
    shapes = [4096, 4001]
    payloads = [_t2_random_payload(g, r, columns, block) for r in shapes]
    mats = [context.create_ternary2(r, columns, block, p) for r, p in zip(shapes, payloads)]
    xs = [g.uniform(-1, 1, columns).astype(np.float32) for _ in range(3)]
    dxs = []
    for x in xs:
        dxs.append(context.alloc(x.nbytes))
        context.upload(dxs[-1], x)
    order = [(i % 2, i % 3) for i in range(members)]
    ys = [context.alloc(4 * shapes[k]) for k, _ in order]
    group = S.HipGroup(context, [mats[k] for k, _ in order], [dxs[j] for _, j in order], ys)
    group.execute()
    context.synchronize()
    first = [context.download(np.zeros(shapes[k], np.float32), ys[i]) for i, (k, _) in enumerate(order)]
    group.execute()  # a second launch must give the same bits
    context.synchronize()
    expected = {}
    for k in range(2):
        wq = O.t2_dequantize(payloads[k], shapes[k], columns, block)
        for j in range(3):
            expected[k, j] = (O.t2_matvec_scalar(payloads[k], shapes[k], columns, block, xs[j]),
                              fp64_matvec(wq, xs[j]), relative_bound(wq, xs[j]))
    for i, (k, j) in enumerate(order):
        got = context.download(np.zeros(shapes[k], np.float32), ys[i])
        assert np.array_equal(got.view(np.uint32), first[i].view(np.uint32)), f"member {i}: launches differ"
        scalar, exact, bound = expected[k, j]
        assert_within(got, scalar, bound, f"member {i} B{block} C={columns} vs scalar")
        assert_within(got, exact, bound, f"member {i} B{block} C={columns} vs FP64")
    group.dispose()
    for p in ys + dxs:
        context.free(p)
    for m in mats:
        m.dispose()


# Groups whose ranges cut items into two pieces (the pieces' row sums are added by the fix-up kernel). 64 members
# of 4096^2 make 16,384 (panel group, tile) units over 1,024 workgroups of eight waves (B = 64, 256): every range
# is exactly half an item, a lone earlier or later piece; 160 members make 40,960 units, 40 a range, so a range
# holds a whole item and an item's earlier tiles, or a later piece and an earlier piece. B = 128 takes
# sixteen-wave workgroups here: items of 16 panels, half the units over half the workgroups, the same cuts. Each group runs eagerly twice and replays three
# times from a captured step, with eager launches between the replays; every launch gives the eager bits, within
# the reference's bound of the scalar restatement and of the FP64 product.
@pytest.mark.parametrize("members", [64, 160])
@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_grouped_cut_items_eager_and_replayed(context, block, members):
    g = rng(4242 + block + members)
    rows = columns = 4096
    payload = _t2_random_payload(g, rows, columns, block)
    m = context.create_ternary2(rows, columns, block, payload)
    xs = [g.uniform(-1, 1, columns).astype(np.float32) for _ in range(3)]
    dxs = [context.alloc(x.nbytes) for x in xs]
    for p, x in zip(dxs, xs):
        context.upload(p, x)
    ys = [context.alloc(4 * rows) for _ in range(members)]
    group = S.HipGroup(context, [m] * members, [dxs[i % 3] for i in range(members)], ys)
    step = None

    def run(launch):
        for p in ys:
            context.upload(p, np.full(rows, np.nan, np.float32))
        launch()
        context.synchronize()
        return [context.download(np.zeros(rows, np.float32), p).view(np.uint32) for p in ys]

    try:
        eager = run(group.execute)
        wq = O.t2_dequantize(payload, rows, columns, block)
        for j, x in enumerate(xs):
            bound = relative_bound(wq, x)
            scalar = O.t2_matvec_scalar(payload, rows, columns, block, x)
            exact = fp64_matvec(wq, x)
            for i in range(j, members, 3):
                assert_within(eager[i].view(np.float32), scalar, bound, f"member {i} B{block} vs scalar")
                assert_within(eager[i].view(np.float32), exact, bound, f"member {i} B{block} vs FP64")
        again = run(group.execute)
        assert all(np.array_equal(a, b) for a, b in zip(again, eager)), "second eager launch differs"
        step = S.HipStep(context, [group])
        for replay in range(3):
            got = run(step.execute)
            for i, (a, b) in enumerate(zip(got, eager)):
                assert np.array_equal(a, b), f"replay {replay}: member {i} differs from the eager launch"
            group.execute()  # eager launch between replays
            context.synchronize()
    finally:
        if step is not None:
            step.dispose()
        group.dispose()
        for p in ys + dxs:
            context.free(p)
        m.dispose()


# A single matrix at one position takes the sliced plan when the chip holds all of its workgroups at once:
# eight waves per workgroup when at most eight slices of eight tiles cover a row and the workgroups fit,
# else sixteen; rows too wide for eight slices of sixteen tiles get sixteen waves taking several tiles each.
# The slices of a panel are joined by a tree of atomic exchanges (1 to 8 slices; an odd count promotes the
# slice without a sibling). The shapes reach each branch (3, 5, 6, 7 and 8 slices among them). Each matrix
# is run three times, with another matrix's launch in between, and must give the same bits every time (the
# exchange slots return to empty after each launch).
@pytest.mark.parametrize("rows,columns", [(1, 1), (64, 128), (65, 1000), (200, 3072), (4000, 4100), (130, 7168),
                                          (4096, 4096), (11008, 4096), (4096, 11008), (300, 129 * 128),
                                          (100, 65536)])
@pytest.mark.parametrize("block", [64, 128, 256])
def test_ternary2_single_matrix_sliced_plans(context, block, rows, columns):
    g = rng(9001 + block + rows + columns)
    payload = _t2_random_payload(g, rows, columns, block)
    x = g.uniform(-1, 1, columns).astype(np.float32)
    m = context.create_ternary2(rows, columns, block, payload)
    other = context.create_ternary2(64, 256, block, _t2_random_payload(g, 64, 256, block))
    first = run(m, x)
    run(other, g.uniform(-1, 1, 256).astype(np.float32))
    for _ in range(2):
        again = run(m, x)
        assert np.array_equal(again.view(np.uint32), first.view(np.uint32)), "repeated launches differ"
    m.dispose()
    other.dispose()
    wq = O.t2_dequantize(payload, rows, columns, block)
    bound = relative_bound(wq, x)
    assert_within(first, O.t2_matvec_scalar(payload, rows, columns, block, x), bound, f"{rows}x{columns} B{block} vs scalar")
    assert_within(first, fp64_matvec(wq, x), bound, f"{rows}x{columns} B{block} vs FP64")


def test_ternary2_zero_rows_are_exactly_zero(context):
    # Ternary2Tests.cs:57-58: an all-zero row next to non-zero rows.
    w, x = O.corpus_random_matrix(7, 2 * 128 + 3)
    w[1] = 0
    payload = O.t2_quantize(w, 7, w.shape[1], 128)
    m = context.create_ternary2(7, w.shape[1], 128, payload)
    y = run(m, x)
    assert y[1] == 0.0 and not np.signbit(y[1])
    m.dispose()


def test_mapped_ternary2_equals_owned(context, tmp_path):
    # MappedTernary2Tests.cs:9-30: mapped == owned bitwise.
    g = rng(7)
    w = g.standard_normal((33, 300), dtype=np.float32)
    x = g.uniform(-1, 1, 300).astype(np.float32)
    matrix = S.Ternary2Matrix.quantize(w, 33, 300, 64)
    path = tmp_path / "m.stq2"
    matrix.save(str(path))
    owned = context.create_ternary2(33, 300, 64, matrix.data)
    with S.MappedTernary2Matrix(str(path), context) as mapped:
        y1 = np.zeros(33, np.float32)
        mapped.execute(x, y1)
    assert np.array_equal(y1, run(owned, x))
    owned.dispose()


def test_mapped_ternary2_rejects_corrupt_files(context, tmp_path):
    # MappedTernary2Tests.cs:47-68: corrupt headers and payloads are InvalidDataException.
    matrix = S.Ternary2Matrix.quantize(np.ones((2, 64), np.float32), 2, 64, 64)
    good = O.stq2_header(2, 64, 64) + matrix.data.tobytes()
    corruptions = {
        "magic": lambda b: b"XTQ2" + b[4:],
        "version": lambda b: b[:4] + b"\x02\x00" + b[6:],
        "header": lambda b: b[:6] + b"\x20\x01" + b[8:],
        "reserved": lambda b: b[:20] + b"\x01" + b[21:],
        "length": lambda b: b[:24] + b"\x00\x00\x00\x00\x00\x00\x00\x00" + b[32:],
        "truncated": lambda b: b[:-1],
        "trailing": lambda b: b + b"\x00",
        "block": lambda b: b[:16] + (100).to_bytes(4, "little") + b[20:],
        "rows": lambda b: b[:8] + (0).to_bytes(4, "little") + b[12:],
        "code3": lambda b: b[:36] + b"\x03" + b[37:],
        "negative-scale": lambda b: b[:32] + np.float32(-1).tobytes() + b[36:],
        "short": lambda b: b[:20],
    }
    for name, corrupt in corruptions.items():
        path = tmp_path / f"{name}.stq2"
        path.write_bytes(corrupt(good))
        with pytest.raises(S.InvalidDataException):
            S.MappedTernary2Matrix(str(path), context)


# ---------------------------------------------------------------------------------------------
# Q8_0 / Q4_0
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("name,fmt", [("q8_0.gguf", BQ.Q8_0), ("q4_0.gguf", BQ.Q4_0)])
def test_golden_gguf_ones_dot(context, name, fmt):
    # QuantizedTests.cs:168-184: the golden tensors dot a ones vector to exactly -8.
    payload, entry = gguf_tensor(name)
    shape = S.QuantizedMatrixShape(entry["dimensions"][1], entry["dimensions"][0], fmt)
    m = context.create(payload, shape)
    assert run(m, np.ones(32, np.float32)).tolist() == [-8.0]
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
def test_legacy_special_scales_match_fp64(context, fmt):
    scales = [0.5, -2.0, 0.0, -0.0, float(np.float16(2 ** -24)), 65504.0, 1.0]
    rows, columns = 7, 96
    data = _special_scale_payload(fmt, rows, columns, scales)
    x = np.array([(i % 13 - 6) / 16 for i in range(columns)], np.float32)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = run(m, x)
    wq = O.decode_matrix(data, rows, columns, int(fmt))
    expected = fp64_matvec(wq, x)
    assert_within(y, expected, np.full(rows, 0.001), "reference tolerance 0.001")
    assert_within(y, expected, relative_bound(wq, x) + 64 * TINY, "1e-5 gate")
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
def test_legacy_critical_cases_within_gamma_bound(context, fmt):
    # Q8Validation.CriticalCases / Compare (validation/Satori.Validation/Q8Validation.cs:9-53) and
    # QuantizedAvx2Tests.cs:280-321: gamma(C + C/32 + 2) * sum|product| + n * float.Epsilon.
    scales = [0.5, -2.0, 0.0, -0.0, float(np.float16(2 ** -24)), 65504.0, 1.0]
    for rows in (1, 7, 63, 64, 65, 129):
        for columns in (32, 64, 96, 288, 768):
            data = _special_scale_payload(fmt, rows, columns, scales)
            x = np.array([(i * 17 % 31 - 15) / 16 for i in range(columns)], np.float32)
            m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
            y = run(m, x)
            wq = O.decode_matrix(data, rows, columns, int(fmt))
            n = columns + columns / 32 + 2
            u = 2.0 ** -24
            g = n * u / (1 - n * u)
            bound = g * (np.abs(wq.astype(np.float64)) @ np.abs(x.astype(np.float64))) + n * TINY
            assert_within(y, fp64_matvec(wq, x), bound, f"{fmt.name} {rows}x{columns}")
            m.dispose()


def test_concurrent_execution_then_disposal_race():
    # VulkanQ8Tests.cs:119-140: four threads execute one matrix concurrently, each result checked; then an
    # execution races the disposal of the matrix and its context: it either completes or raises
    # ObjectDisposedException, and repeated disposal is a no-op. Calls release the GIL in the library,
    # which serialises them per context.
    import threading

    rows, columns = 257, 768
    g = rng(119)
    w = (g.standard_normal((rows, columns), dtype=np.float32) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, BQ.Q8_0)
    wq = O.decode_matrix(data, rows, columns, int(BQ.Q8_0))
    ctx = S.HipContext(0)
    m = ctx.create(data, S.QuantizedMatrixShape(rows, columns, BQ.Q8_0))
    errors = []

    def worker(seed):
        try:
            x = rng(seed).standard_normal(columns, dtype=np.float32)
            for _ in range(10):
                y = np.zeros(rows, np.float32)
                m.execute(x, y)
                assert_within(y, fp64_matvec(wq, x), relative_bound(wq, x) + 64 * TINY, f"thread {seed}")
        except BaseException as e:  # re-raised in the test thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(60)
    assert not errors, errors
    start = threading.Barrier(2)
    outcome = []

    def work():
        start.wait()
        try:
            m.execute(np.ones(columns, np.float32), np.zeros(rows, np.float32))
            outcome.append("completed")
        except S.ObjectDisposedException:
            outcome.append("disposed")
        except BaseException as e:
            outcome.append(e)

    def dispose():
        start.wait()
        m.dispose()
        ctx.dispose()

    pair = [threading.Thread(target=work), threading.Thread(target=dispose)]
    for t in pair:
        t.start()
    for t in pair:
        t.join(60)
    assert outcome in (["completed"], ["disposed"]), outcome
    m.dispose()
    ctx.dispose()
    with pytest.raises(S.ObjectDisposedException):
        m.execute(np.ones(columns, np.float32), np.zeros(rows, np.float32))


@pytest.mark.parametrize("fmt,rows,columns", [(BQ.Q8_0, 4096, 4096), (BQ.Q4_0, 11008, 4096),
                                              (BQ.Q4_0, 4096, 11008), (BQ.Q8_0, 65, 96)])
def test_legacy_benchmark_shapes_match_scalar_reference(context, fmt, rows, columns):
    g = rng(20261014 + rows + columns)
    w = (g.standard_normal((rows, columns), dtype=np.float32) * 0.02).astype(np.float32)
    x = g.standard_normal(columns, dtype=np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    O.q_validate(data, rows, columns, int(fmt))
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = run(m, x)
    scalar = O.q_matvec_scalar(data, rows, columns, int(fmt), x)
    wq = O.decode_matrix(data, rows, columns, int(fmt)) if rows * columns <= 1 << 20 else None
    if wq is not None:
        bound = relative_bound(wq, x)
        assert_within(y, fp64_matvec(wq, x), bound, "vs FP64")
    else:
        # Sum |w x| via the oracle on |payload|-decoded weights is costly at this size; bound by the
        # scalar kernel's own magnitudes: |w_i x_i| summed with the absolute input against |w|.
        absolute = np.zeros(rows, np.float64)
        e = 32
        blocks = columns // e
        nb = O.GEOMETRY[int(fmt)][1]
        d = data.reshape(rows, blocks, nb)
        scales = np.abs(d[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0])
        if fmt == BQ.Q8_0:
            q = np.abs(d[:, :, 2:].view(np.int8).astype(np.float64))
        else:
            lo = (d[:, :, 2:] & 15).astype(np.float64) - 8
            hi = (d[:, :, 2:] >> 4).astype(np.float64) - 8
            q = np.abs(np.concatenate([lo, hi], axis=2))
        absolute = np.einsum("rb,rbj,bj->r", scales, q, np.abs(x.astype(np.float64)).reshape(blocks, e))
        bound = 1e-5 * absolute
    assert_within(y, scalar, bound, f"{fmt.name} {rows}x{columns} vs scalar reference")
    m.dispose()


# ---------------------------------------------------------------------------------------------
# K formats, FP32 activations (Execute)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fixture,fmt", [("q4k-v1.json", BQ.Q4_K), ("q6k-v1.json", BQ.Q6_K)])
def test_k_fixture_blocks_dot(context, fixture, fmt):
    # Q4KCodecTests.cs:413-429 / Q6KCodecTests.cs: one-block matrices against the FP64 fixture dot.
    for case in load_json(fixture)["cases"]:
        block = hexbytes(case["block_hex"])
        x = np.array(case["input"], np.float32)
        m = context.create(block, S.QuantizedMatrixShape(1, 256, fmt))
        y = run(m, x)
        ref = case["dot"]
        assert abs(y[0] - ref) <= 1e-2 + 1e-4 * abs(ref), (case["name"], y[0], ref)
        wq = O.decode_block(block, int(fmt)).reshape(1, 256)
        assert_within(y, O.q_matvec_scalar(block, 1, 256, int(fmt), x), relative_bound(wq, x) + 8 * TINY,
                      case["name"])
        m.dispose()


def test_k_real_tensor_blocks(context):
    # KParityTests.cs:177-212: real Q4_K / Q6_K bytes against the fixture's FP64 dots.
    for case in load_json("k-real-v1.json")["cases"]:
        fmt = BQ.Q4_K if case["name"].startswith("q4k:") else BQ.Q6_K
        raw = hexbytes(case["block_hex"])
        x = np.array(case["input"], np.float32)
        nb = O.GEOMETRY[int(fmt)][1]
        for b in range(case["blocks"]):
            block = raw[b * nb:(b + 1) * nb]
            m = context.create(block, S.QuantizedMatrixShape(1, 256, fmt))
            y = run(m, x)
            ref = case["dots"][b]
            assert abs(y[0] - ref) <= 1e-2 + 1e-4 * abs(ref), (case["name"], b, y[0], ref)
            m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("rows,columns", [(8960, 1536), (1536, 8960), (1536, 1536), (256, 1536), (17, 512),
                                          (4096, 4096)])
def test_k_float_path_matches_scalar_reference(context, fmt, rows, columns):
    g = rng(20261014 + rows * 7 + columns)
    w = (g.standard_normal((rows, columns), dtype=np.float32) * 0.02).astype(np.float32)
    x = g.standard_normal(columns, dtype=np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = run(m, x)
    wq = O.decode_matrix(data, rows, columns, int(fmt)) if rows * columns <= 1 << 21 else None
    scalar = O.q_matvec_scalar(data, rows, columns, int(fmt), x)
    if wq is None:
        sub = slice(0, rows, 37)  # the row bound needs the decoded rows; check a deterministic subset
        wq_rows = np.stack([O.decode_matrix(data.reshape(rows, -1)[r], 1, columns, int(fmt))[0]
                            for r in range(rows)[sub]])
        assert_within(y[sub], scalar[sub], relative_bound(wq_rows, x), "vs scalar (row subset)")
        # every row: a looser size-independent check against the scalar path
        assert np.allclose(y, scalar, rtol=1e-4, atol=1e-4)
    else:
        assert_within(y, scalar, relative_bound(wq, x), "vs scalar")
        assert_within(y, fp64_matvec(wq, x), relative_bound(wq, x), "vs FP64")
    m.dispose()


# ---------------------------------------------------------------------------------------------
# Q8_K and the integer K products (ExecuteBatch): bit-exact
# ---------------------------------------------------------------------------------------------

def test_q8k_quantizer_matches_fixture_bytes(context):
    # Q8KCodecTests.cs:22-35: block bytes identical to the reference quantizer.
    for case in load_json("q8k-v1.json")["cases"]:
        x = np.array(case["input"], np.float32)
        assert np.array_equal(context.quantize_q8k(x), hexbytes(case["block_hex"])), case["name"]
    for case in load_json("q6k-q8k-v1.json")["cases"]:
        x = np.array(case["input"], np.float32)
        assert np.array_equal(context.quantize_q8k(x), hexbytes(case["activation_hex"])), case["name"]


def test_q8k_quantizer_matches_oracle_on_edge_cases(context):
    g = rng(99)
    tiny = TINY
    cases = {
        "normal": g.standard_normal(8960).astype(np.float32),
        "uniform": g.uniform(-1, 1, 1536).astype(np.float32),
        "zeros": np.zeros(512, np.float32),
        "one-zero-block": np.concatenate([np.zeros(256), g.standard_normal(256)]).astype(np.float32),
        "ties": np.tile(np.array([1, -1, 0.5, -0.5], np.float32), 64 * 3),
        "negative-max-first": np.concatenate([[-3.0], g.uniform(-3, 3, 255)]).astype(np.float32),
        "subnormal": np.full(256, tiny, np.float32) * np.sign(g.standard_normal(256)).astype(np.float32),
        "half-steps": (np.arange(256, dtype=np.float32) - 127.5) / 127.0,
        "large": (g.standard_normal(768) * 1e30).astype(np.float32),
        "sin": np.sin(np.arange(768) * 0.01).astype(np.float32),
    }
    for name, x in cases.items():
        assert np.array_equal(context.quantize_q8k(x), O.q8k_quantize_row(x)), name


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("rows,columns", [(8960, 1536), (1536, 8960), (1536, 1536), (256, 1536), (17, 3584),
                                          (4096, 4096), (14336, 4096), (4096, 14336)])
def test_k_integer_batch_is_bit_exact(context, fmt, rows, columns):
    # Q6KQuantizedProductTests.cs:284-308 and KParityTests.cs:214-244: the projection equals the
    # composition of the public codecs, summed block by block; here the oracle's restatement of
    # ExecuteQuantizedTiled, compared bit for bit.
    g = rng(20261014 + rows + 3 * columns)
    w = (g.standard_normal((rows, columns), dtype=np.float32) * 0.02).astype(np.float32)
    x = g.standard_normal(columns, dtype=np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.zeros(rows, np.float32)
    m.execute_batch(x, 1, y)
    expected = O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x))
    assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))
    if rows <= 2048 and columns <= 2048:
        assert np.array_equal(y.view(np.uint32), O.q_matvec_batch(data, rows, columns, int(fmt), x, 1).view(np.uint32))
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
def test_k_integer_product_quantizer_edge_cases(context, fmt):
    # Q8KCodec.QuantizeBlock (Q8KCodec.cs:44-76) inside the integer products: ties of the largest magnitude
    # (the lowest index wins, and its sign sets the scale), the maximum in every lane position of a block,
    # subnormal and huge blocks, zero blocks; outputs bit-exact against the oracle, for the single-position
    # kernel (which quantizes in-kernel) and the matrix-core batch (which quantizes in its pack kernel).
    g = rng(4711)
    rows, columns = 70, 4096
    w = (g.standard_normal((rows, columns)) * 0.05).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    cases = []
    x = np.sign(g.standard_normal(columns)).astype(np.float32)  # all |x| equal: every element ties
    cases.append(x)
    x = g.uniform(-1, 1, columns).astype(np.float32)
    for b in range(16):  # block b: maximum magnitude 3 at element 17b (each lane slot), a later -3 tie
        x[256 * b + 17 * b % 256] = 3.0
        x[256 * b + (17 * b + 100) % 256] = -3.0
    cases.append(x)
    x = g.uniform(-1, 1, columns).astype(np.float32)
    for b in range(16):  # negative maximum first, positive tie later, and a last-element maximum
        x[256 * b + 5] = -2.5
        x[256 * b + 250] = 2.5 if b % 2 else 1.0
        x[256 * b + 255] = 4.0 if b % 3 == 0 else x[256 * b + 255]
    cases.append(x)
    x = (g.standard_normal(columns) * 1e-40).astype(np.float32)  # subnormal blocks
    x[:256] = 0.0
    x[512:768] = np.float32(1e-45)
    cases.append(x)
    x = (g.standard_normal(columns) * 1e30).astype(np.float32)
    x[1024:1280] = 0.0
    cases.append(x)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    for i, x in enumerate(cases):
        y = np.zeros(rows, np.float32)
        m.execute_batch(x, 1, y)
        expected = O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x))
        assert np.array_equal(y.view(np.uint32), expected.view(np.uint32)), f"case {i}"
    xs = np.stack(cases * 4).astype(np.float32)  # 20 positions: the matrix-core path
    y = np.zeros(xs.shape[0] * rows, np.float32)
    m.execute_batch(xs.reshape(-1), xs.shape[0], y)
    expected = O.q_matvec_batch(data, rows, columns, int(fmt), xs.reshape(-1), xs.shape[0])
    assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))
    m.dispose()


@pytest.mark.parametrize("fmt,fixture", [(BQ.Q4_K, "q4k-v1.json"), (BQ.Q6_K, "q6k-v1.json")])
def test_k_integer_batch_multi_position_on_fixture_blocks(context, fmt, fixture):
    # BatchedMatVecTests.cs:45-113: payloads tiled from the fixture blocks, several positions.
    blocks = [hexbytes(c["block_hex"]) for c in load_json(fixture)["cases"]]
    for rows, columns, positions in ((2, 512, 4), (3, 512, 1), (2, 256, 8), (7, 512, 5), (40, 1024, 3)):
        nbr = columns // 256
        data = np.concatenate([blocks[i % len(blocks)] for i in range(rows * nbr)])
        x = np.array([[np.sin(p * 0.37 + c * 0.011) * 1.5 for c in range(columns)] for p in range(positions)],
                     np.float32)
        m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
        y = np.zeros(positions * rows, np.float32)
        m.execute_batch(x.reshape(-1), positions, y)
        expected = O.q_matvec_batch(data, rows, columns, int(fmt), x.reshape(-1), positions)
        assert np.array_equal(y.view(np.uint32), expected.view(np.uint32)), (rows, columns, positions)
        m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("rows,columns,positions", [(17, 512, 16), (129, 768, 37), (300, 1536, 64),
                                                    (1536, 1536, 100), (8960, 1536, 256), (256, 8960, 65)])
def test_k_matrix_core_batch_equals_per_position(context, fmt, rows, columns, positions):
    # BatchedMatVecTests.cs:45-113: a batch equals its positions run one at a time. Sixteen positions and
    # more take the matrix-core kernel, one position the single-position integer kernel (bit-exact against
    # the oracle above), so the two must agree bit for bit. Ragged row and position counts, a zero
    # position, a zero block inside a position and a position of large magnitude are included.
    g = rng(7 + rows + columns + positions)
    w = (g.standard_normal((rows, columns), dtype=np.float32) * 0.02).astype(np.float32)
    x = g.standard_normal((positions, columns), dtype=np.float32)
    x[1] = 0.0
    x[2, 256:512] = 0.0
    x[3] *= 1e20
    data = S.quantize_weights(w, rows, columns, fmt)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.full(positions * rows, np.nan, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    single = np.zeros(rows, np.float32)
    for p in range(positions):
        m.execute_batch(x[p], 1, single)
        assert np.array_equal(y[p * rows:(p + 1) * rows].view(np.uint32), single.view(np.uint32)), p
    if rows * columns * positions <= 1536 * 1536 * 100:
        expected = O.q_matvec_batch(data, rows, columns, int(fmt), x.reshape(-1), positions)
        assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))
    m.dispose()


def _q6k_extreme_blocks(g, rows: int, blocks: int) -> np.ndarray:
    """Q6_K rows whose weight products reach the ends of their range: group scales -128 and 127 with codes 0
    and 63 (sc * (q - 32) from -4064 to 4096, the planes' hi part from -32 to 32), mixed with random blocks;
    finite FP16 d values including subnormal, negative and zero."""
    out = g.integers(0, 256, size=(rows, blocks, 210), dtype=np.uint8)
    kind = g.integers(0, 4, size=(rows, blocks))
    for r in range(rows):
        for b in range(blocks):
            blk = out[r, b]
            if kind[r, b] == 0:    # q = 0 everywhere (q - 32 = -32)
                blk[:192] = 0
            elif kind[r, b] == 1:  # q = 63 everywhere (q - 32 = 31)
                blk[:192] = 0xFF
            if kind[r, b] < 3:
                blk[192:208] = np.where(g.integers(0, 2, 16) == 0, 0x80, 0x7F).astype(np.uint8)  # sc -128 / 127
    d = g.choice(np.array([0x3C00, 0x0001, 0xBC00, 0x0000, 0x2E66, 0x7BFF], np.uint16), size=(rows, blocks))
    out[:, :, 208:210] = d.view(np.uint8).reshape(rows, blocks, 2)
    return np.ascontiguousarray(out.reshape(-1))


@pytest.mark.parametrize("rows,columns,positions", [(70, 1536, 33), (33, 8960, 64)])
def test_k_matrix_core_q6k_extreme_products(context, rows, columns, positions):
    # The Q6_K matrix-core product reads pre-scaled weight planes: its extremes (the largest |sc * (q - 32)|
    # against activation codes of +-127, |Dot| near 2^27) must give the reference's outputs bit for bit, as
    # must the single-position kernel on the resident layout.
    g = rng(31337 + rows + columns)
    data = _q6k_extreme_blocks(g, rows, columns // 256)
    x = g.standard_normal((positions, columns), dtype=np.float32)
    x[0] = np.where(g.integers(0, 2, columns) == 0, -1.0, 1.0)  # every code +-127
    x[1] = 0.0
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, BQ.Q6_K))
    y = np.full(positions * rows, np.nan, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    expected = O.q_matvec_batch(data, rows, columns, int(BQ.Q6_K), x.reshape(-1), positions)
    assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))
    single = np.zeros(rows, np.float32)
    m.execute_batch(x[0], 1, single)
    assert np.array_equal(single.view(np.uint32), expected[:rows].view(np.uint32))
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("positions", [1, 9, 16, 77, 256])
def test_k_group_batch_equals_member_batches(context, fmt, positions):
    # DenseForward.LayerBatch (DenseForward.cs:187-196): q/k/v read one normalized batch. The grouped
    # many-position product (shared Q8_K pack, several members per launch) must equal each member's own
    # ExecuteBatch bit for bit: five members (more than one launch holds), ragged row counts, two inputs
    # (members 0, 1, 3, 4 share one), and zero / huge positions inside the batch.
    columns = 768
    g = rng(100 + positions + int(fmt))
    row_counts = [200, 33, 64, 300, 1]
    x = [g.standard_normal((positions, columns), dtype=np.float32) for _ in range(2)]
    x[0][positions // 2] = 0.0
    x[1][positions - 1] *= 1e15
    mats, datas = [], []
    for r in row_counts:
        w = (g.standard_normal((r, columns), dtype=np.float32) * 0.02).astype(np.float32)
        datas.append(S.quantize_weights(w, r, columns, fmt))
        mats.append(context.create(datas[-1], S.QuantizedMatrixShape(r, columns, fmt)))
    which = [0, 0, 1, 0, 0]
    dx = [context.alloc(4 * a.size) for a in x]
    for p, a in zip(dx, x):
        context.upload(p, a.reshape(-1))
    dy = [context.alloc(4 * positions * r) for r in row_counts]
    group = S.HipGroup(context, mats, [dx[i] for i in which], dy, True)
    try:
        for repeat in range(2):  # the second call reuses the group's workspace
            for p, r in zip(dy, row_counts):
                context.upload(p, np.full(positions * r, np.nan, np.float32))
            group.execute_batch(positions)
            for i, (m, r) in enumerate(zip(mats, row_counts)):
                got = context.download(np.zeros(positions * r, np.float32), dy[i])
                want = np.zeros(positions * r, np.float32)
                m.execute_batch(x[which[i]].reshape(-1), positions, want)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (repeat, i, r)
    finally:
        group.dispose()
        for p in dx + dy:
            context.free(p)
        for m in mats:
            m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("columns,inputs", [(4608, "shared"), (4096, "shared"), (4608, "mixed")])
def test_large_one_position_k_group(context, fmt, columns, inputs):
    # One-position K groups of more members than a launch passes in its arguments (the descriptor array):
    # with one shared input of more than 16 blocks the library quantizes it once per launch and every
    # workgroup copies the bytes; at 16 blocks, or with several inputs, each workgroup quantizes. Every member
    # equals the oracle's ExecuteQuantizedTiled composition bit for bit, on repeated launches and replayed
    # from a captured step with new inputs between the replays.
    g = rng(515 + columns + int(fmt) + (inputs == "mixed"))
    row_counts = [300, 1, 64, 129, 256, 33]
    datas, mats = [], []
    for r in row_counts:
        w = (g.standard_normal((r, columns)) * 0.02).astype(np.float32)
        datas.append(S.quantize_weights(w, r, columns, fmt))
        mats.append(context.create(datas[-1], S.QuantizedMatrixShape(r, columns, fmt)))
    which = [0] * 6 if inputs == "shared" else [0, 1, 0, 1, 1, 0]
    dx = [context.alloc(4 * columns) for _ in range(2)]
    dy = [context.alloc(4 * r) for r in row_counts]
    group = S.HipGroup(context, mats, [dx[i] for i in which], dy, True)
    step = None
    try:
        def check(seed, run):
            x = [rng(seed + i).standard_normal(columns).astype(np.float32) for i in range(2)]
            x[1][:256] = 0.0  # an all-zero activation block
            for p, a in zip(dx, x):
                context.upload(p, a)
            for p, r in zip(dy, row_counts):
                context.upload(p, np.full(r, np.nan, np.float32))
            run()
            context.synchronize()
            for i, r in enumerate(row_counts):
                got = context.download(np.zeros(r, np.float32), dy[i])
                want = O.qk_matvec_quantized_avx2(datas[i], r, columns, int(fmt), O.q8k_quantize_row(x[which[i]]))
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, i, r)

        check(1, group.execute)
        check(2, group.execute)
        step = S.HipStep(context, [group])
        check(3, step.execute)
        check(4, step.execute)
    finally:
        if step is not None:
            step.dispose()
        group.dispose()
        for p in dx + dy:
            context.free(p)
        for m in mats:
            m.dispose()


def test_randomized_shapes_sweep(context):
    # A seeded sweep over every MatVec path and random shapes (rows 1-3000, so rows end inside panels and
    # tiles; ragged Ternary2 columns; odd block counts; long and short rows): the FP32 paths within the
    # 1e-5 * sum|w*x| gate of the oracle's scalar restatement of ExecuteScalarCore / ExecuteScalar, the
    # integer K path (1-15 positions: in-kernel quantization; 16 and more: the matrix-core product) equal to
    # the oracle's ExecuteQuantizedTiled bit for bit.
    g = rng(20261201)
    for case in range(45):
        kind = case % 9
        rows = int(g.integers(1, 3001))
        what = f"case {case}"
        if kind < 3:
            block = (64, 128, 256)[kind]
            columns = int(g.integers(1, 6001))
            what += f" Ternary2 B{block} {rows}x{columns}"
            payload = _t2_random_payload(g, rows, columns, block)
            m = context.create_ternary2(rows, columns, block, payload)
            x = g.standard_normal(columns).astype(np.float32)
            y = run(m, x)
            wq = O.t2_dequantize(payload, rows, columns, block)
            scalar = O.t2_matvec_scalar(payload, rows, columns, block, x)
            assert_within(y, scalar, relative_bound(wq, x) + (columns + 8) * TINY, what)
        elif kind < 7:
            fmt = (BQ.Q8_0, BQ.Q4_0, BQ.Q4_K, BQ.Q6_K)[kind - 3]
            unit = 32 if fmt in (BQ.Q8_0, BQ.Q4_0) else 256
            columns = unit * int(g.integers(1, 6000 // unit + 2))
            what += f" {fmt.name} FP32 {rows}x{columns}"
            w = (g.standard_normal((rows, columns)) * 0.05).astype(np.float32)
            data = S.quantize_weights(w, rows, columns, fmt)
            m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
            x = g.standard_normal(columns).astype(np.float32)
            y = run(m, x)
            wq = O.decode_matrix(data, rows, columns, int(fmt))
            scalar = O.q_matvec_scalar(data, rows, columns, int(fmt), x)
            assert_within(y, scalar, relative_bound(wq, x) + 64 * TINY, what)
        else:
            fmt = BQ.Q4_K if kind == 7 else BQ.Q6_K
            positions = int(g.choice([1, 3, 15, 16, 40]))
            rows = min(rows, 1500)
            columns = 256 * int(g.integers(1, 36))
            what += f" {fmt.name} Q8_K {rows}x{columns} x {positions} positions"
            w = (g.standard_normal((rows, columns)) * 0.05).astype(np.float32)
            data = S.quantize_weights(w, rows, columns, fmt)
            m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
            x = g.standard_normal((positions, columns)).astype(np.float32)
            y = np.zeros(positions * rows, np.float32)
            m.execute_batch(x.reshape(-1), positions, y)
            expected = np.concatenate([O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x[p]))
                                       for p in range(positions)])
            assert np.array_equal(y.view(np.uint32), expected.astype(np.float32).view(np.uint32)), what
        m.dispose()


def test_workspaces_do_not_grow_under_captured_steps():
    # A captured step records the device address of the workspace it launches with: the matrix's Q8_K
    # buffer, the group's, the context's split-attention partials. An eager call that would grow (reallocate)
    # one of them while such a step lives is refused; after the step is destroyed it proceeds.
    ctx = S.HipContext(0)  # fresh: its workspaces start empty
    rows, columns = 64, 512
    g = rng(4242)
    w = (g.standard_normal((rows, columns)) * 0.1).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, BQ.Q4_K)
    m = ctx.create(data, S.QuantizedMatrixShape(rows, columns, BQ.Q4_K))
    x = g.standard_normal((64, columns)).astype(np.float32)
    dx, dy = ctx.alloc(x.nbytes), ctx.alloc(4 * rows * 64)
    ctx.upload(dx, x)
    group = S.HipGroup(ctx, [m], [dx], [dy], True)
    heads, kv_heads, hd, tokens = 2, 1, 64, 64
    wide = 8 * 128  # the buffers fit the wider call below (8 query heads of 128, one KV head)
    dq, dk, dv, do = ctx.alloc(4 * wide), ctx.alloc(4 * tokens * 128), ctx.alloc(4 * tokens * 128), ctx.alloc(4 * wide)
    for p_, n_ in ((dq, wide), (dk, tokens * 128), (dv, tokens * 128)):
        ctx.upload(p_, g.standard_normal(n_).astype(np.float32))
    ops = S.DeviceOps(ctx)
    m.execute_batch_device(dx, 16, dy)      # allocates the 16-position workspaces
    group.execute_batch(16)
    ops.grouped_attention(dq, dk, dv, heads, kv_heads, hd, tokens, do)
    ctx.capture_begin()
    m.execute_batch_device(dx, 16, dy)
    group.execute_batch(16)
    ops.grouped_attention(dq, dk, dv, heads, kv_heads, hd, tokens, do)
    step = ctx.capture_end()
    step.execute()
    with pytest.raises(S.InvalidOperationException):
        m.execute_batch_device(dx, 64, dy)
    with pytest.raises(S.InvalidOperationException):
        group.execute_batch(64)
    with pytest.raises(S.InvalidOperationException):
        ops.grouped_attention(dq, dk, dv, 8, 1, 128, tokens, do)  # wider heads: a larger workspace
    m.execute_batch_device(dx, 16, dy)      # within the current workspace: allowed
    step.execute()
    ctx.synchronize()
    step.dispose()
    m.execute_batch_device(dx, 64, dy)      # the step is gone: the workspace may grow
    group.execute_batch(64)
    ops.grouped_attention(dq, dk, dv, 8, 1, 128, tokens, do)
    ctx.synchronize()
    expected = O.qk_matvec_quantized_avx2(data, rows, columns, int(BQ.Q4_K), O.q8k_quantize_row(x[63]))
    y = ctx.download(np.empty((64, rows), np.float32), dy)
    assert np.array_equal(y[63].view(np.uint32), np.asarray(expected, np.float32).view(np.uint32))
    group.dispose()
    m.dispose()
    for p_ in (dx, dy, dq, dk, dv, do):
        ctx.free(p_)
    ctx.dispose()


def test_k_group_batch_errors(context):
    g = rng(5)
    w = (g.standard_normal((64, 512), dtype=np.float32) * 0.02).astype(np.float32)
    m = context.create(S.quantize_weights(w, 64, 512, BQ.Q4_K), S.QuantizedMatrixShape(64, 512, BQ.Q4_K))
    x, y = context.alloc(4 * 512 * 256), context.alloc(4 * 64 * 256)
    float_group = S.HipGroup(context, [m], [x], [y], False)
    group = S.HipGroup(context, [m], [x], [y], True)
    try:
        with pytest.raises(S.NotSupportedException):
            float_group.execute_batch(16)
        for bad in (0, 257):
            with pytest.raises(S.ArgumentOutOfRangeException):
                group.execute_batch(bad)
    finally:
        float_group.dispose()
        group.dispose()
        context.free(x)
        context.free(y)
        m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
def test_legacy_batch_matches_per_position(context, fmt):
    # BatchedMatVecTests.cs:61-88 (float path): each position within 1e-5 * sum|w x| of the scalar product.
    g = rng(5)
    rows, columns, positions = 37, 288, 6
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    x = g.standard_normal((positions, columns)).astype(np.float32)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.zeros(positions * rows, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    wq = O.decode_matrix(data, rows, columns, int(fmt))
    batch_ref = O.q_matvec_batch(data, rows, columns, int(fmt), x.reshape(-1), positions)
    for p in range(positions):
        bound = relative_bound(wq, x[p])
        assert_within(y[p * rows:(p + 1) * rows], fp64_matvec(wq, x[p]), bound, f"position {p}")
        assert_within(y[p * rows:(p + 1) * rows], batch_ref[p * rows:(p + 1) * rows], bound, f"position {p} batch")
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
@pytest.mark.parametrize("rows,columns,positions", [(37, 288, 32), (100, 1024, 33), (129, 2048, 64),
                                                    (4096, 4096, 256), (11008, 4096, 40), (300, 11008, 100),
                                                    (70, 512, 600)])
def test_legacy_matrix_core_batch(context, fmt, rows, columns, positions):
    # From 32 positions on, Q8_0 / Q4_0 batches run on the matrix cores (exact bf16 splits of x, FP32
    # sums; 256 positions per launch, so 600 positions take three). Every position within 1e-5 * sum |w x|
    # of the FP64 product, sampled positions also of the scalar reference (BatchedMatVecTests.cs:61-88);
    # a zero position, one of large magnitude, and NaN / +Inf inputs, whose non-finite outputs must match the
    # single-position kernel's (the reference's IEEE products).
    g = rng(808 + rows + columns + positions)
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    x = g.standard_normal((positions, columns)).astype(np.float32)
    x[1] = 0.0
    x[2] *= np.float32(1e20)
    x[3, 5] = np.nan
    x[4, columns - 1] = np.inf
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.full(positions * rows, np.nan, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    y = y.reshape(positions, rows)
    wq = O.decode_matrix(data, rows, columns, int(fmt)).astype(np.float64)
    finite = [p for p in range(positions) if p not in (3, 4)]
    xf = x[finite].astype(np.float64)
    exact, bound = np.zeros((positions, rows)), np.zeros((positions, rows))
    exact[finite] = xf @ wq.T
    # Q8Validation.cs:46: the reference's subnormal floor n * float.Epsilon, n = C + C/32 + 2.
    bound[finite] = np.abs(xf) @ np.abs(wq).T * 1e-5 + (columns + columns // 32 + 2) * TINY
    for p in finite:
        assert_within(y[p], exact[p], bound[p], f"position {p} vs FP64")
    for p in sorted({0, 1, 2, positions // 2, positions - 1} - {3, 4}):
        assert_within(y[p], O.q_matvec_scalar(data, rows, columns, int(fmt), x[p]), bound[p], f"position {p} vs scalar")
    single = np.zeros(rows, np.float32)
    for p in (3, 4):
        m.execute_batch(x[p], 1, single)  # one position: the single-position kernel
        assert np.array_equal(np.isnan(y[p]), np.isnan(single)), f"position {p}: NaN pattern"
        inf = np.isinf(single)
        assert np.array_equal(np.isinf(y[p]), inf) and np.array_equal(y[p][inf], single[inf]), f"position {p}: Inf"
    m.dispose()


def _tiny_positions(g, positions, columns, mixed):
    """Activation rows of tiny magnitude (NumericalCorpus.cs:24-27 carries 1e-30, subnormal and 1e-38 cases):
    N(0,1) scaled to 1e-36 and 1e-38, FP32 subnormals, TINY alternating, normal elements mixed with 1e-38 and
    subnormal ones, and magnitudes spread over 2^-150..2^0; with `mixed`, every other position is N(0,1)."""
    x = g.standard_normal((positions, columns)).astype(np.float32)
    kinds = []
    for p in range(positions):
        if mixed and p % 2 == 0:
            kinds.append("normal")
            continue
        kind = ("1e-36", "1e-38", "subnormal", "tiny", "half-1e-38", "spread")[(p // (2 if mixed else 1)) % 6]
        row = g.standard_normal(columns)
        if kind == "1e-36":
            v = row * 1e-36
        elif kind == "1e-38":
            v = row * 1e-38
        elif kind == "subnormal":
            v = g.integers(-(1 << 22), 1 << 22, columns).astype(np.float64) * TINY
        elif kind == "tiny":
            v = np.where(np.arange(columns) % 2 == 0, TINY, -TINY)
        elif kind == "half-1e-38":
            v = np.where(np.arange(columns) % 2 == 0, row, row * 1e-38)
            v[::7] = g.integers(-1000, 1000, v[::7].size) * TINY
        else:
            v = row * np.exp2(g.uniform(-150.0, 0.0, columns))
        x[p] = v.astype(np.float32)
        kinds.append(kind)
    return x, kinds


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
@pytest.mark.parametrize("mixed", [False, True])
def test_legacy_tiny_activations_within_reference_floor(context, fmt, mixed):
    # Positions of 1e-36, 1e-38 and subnormal activations, alone and among normal positions, through the
    # matrix-core batch (>= 32 positions) and the single-position kernels (ExecuteBatch at one position, and
    # the IQuantizedMatrix form): every output within 1e-5 * sum|w x| + n * float.Epsilon (Q8Validation.cs:46,
    # n = C + C/32 + 2) of the FP64 product and of the scalar reference (QuantizedMatVec.cs:45-78).
    g = rng(4242 + int(fmt) + (7 if mixed else 0))
    rows, columns, positions = 300, 1024, 40
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    x, kinds = _tiny_positions(g, positions, columns, mixed)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    y = np.full(positions * rows, np.nan, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    y = y.reshape(positions, rows)
    wq = O.decode_matrix(data, rows, columns, int(fmt)).astype(np.float64)
    floor = (columns + columns // 32 + 2) * TINY
    single = np.zeros(rows, np.float32)
    for p in range(positions):
        xp = x[p].astype(np.float64)
        exact = wq @ xp
        bound = 1e-5 * (np.abs(wq) @ np.abs(xp)) + floor
        scalar = O.q_matvec_scalar(data, rows, columns, int(fmt), x[p])
        what = f"position {p} ({kinds[p]})"
        assert_within(y[p], exact, bound, what + " batch vs FP64")
        assert_within(y[p], scalar, bound, what + " batch vs scalar")
        if kinds[p] != "normal" or p < 2:
            m.execute_batch(x[p], 1, single)
            assert_within(single, exact, bound, what + " single position vs FP64")
            assert_within(single, scalar, bound, what + " single position vs scalar")
            m.execute(x[p], single)
            assert_within(single, scalar, bound, what + " execute vs scalar")
    m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
def test_k_tiny_activations_float_and_integer_paths(context, fmt):
    # The K formats with the same tiny positions: the FP32-activation MatVec (IQuantizedMatrix.Execute,
    # QuantizedMatVec.ExecuteScalar's DotBlock, QuantizedMatVec.cs:56-65) within 1e-5 * sum|w x| + n *
    # float.Epsilon of the scalar reference, and the Q8_K integer path (ExecuteBatch) bit-identical to the
    # reference's ExecuteQuantizedTiled composition, at one position and as a 40-position matrix-core batch.
    g = rng(5151 + int(fmt))
    rows, columns, positions = 256, 1536, 40
    w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    x, kinds = _tiny_positions(g, positions, columns, True)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    wq = O.decode_matrix(data, rows, columns, int(fmt)).astype(np.float64)
    floor = (columns + columns // 256 + 2) * TINY
    y = np.zeros(positions * rows, np.float32)
    m.execute_batch(x.reshape(-1), positions, y)
    single = np.zeros(rows, np.float32)
    for p in range(positions):
        what = f"position {p} ({kinds[p]})"
        ref = O.qk_matvec_quantized_avx2(data, rows, columns, int(fmt), O.q8k_quantize_row(x[p]))
        assert np.array_equal(y[p * rows:(p + 1) * rows].view(np.uint32), ref.view(np.uint32)), what + " batch"
        if kinds[p] == "normal" and p >= 2:
            continue
        m.execute_batch(x[p], 1, single)
        assert np.array_equal(single.view(np.uint32), ref.view(np.uint32)), what + " one position"
        m.execute(x[p], single)
        xp = x[p].astype(np.float64)
        bound = 1e-5 * (np.abs(wq) @ np.abs(xp)) + floor
        assert_within(single, O.q_matvec_scalar(data, rows, columns, int(fmt), x[p]), bound, what + " float")
        assert_within(single, wq @ xp, bound, what + " float vs FP64")
    m.dispose()


# ---------------------------------------------------------------------------------------------
# Contract: errors, output commit, disposal, device and group entry points
# ---------------------------------------------------------------------------------------------

def test_failed_execution_leaves_output_unchanged(context):
    # IQuantizedMatrix.cs:6 and VulkanQ8Tests.cs:73-97 (sentinel output).
    payload, entry = gguf_tensor("q8_0.gguf")
    m = context.create(payload, S.QuantizedMatrixShape(1, 32, BQ.Q8_0))
    sentinel = np.full(1, 123.5, np.float32)
    with pytest.raises(S.ArgumentException):
        m.execute(np.ones(31, np.float32), sentinel)
    bad = np.ones(32, np.float32)
    bad[3] = np.inf
    with pytest.raises(S.ArgumentException):
        m.execute(bad, sentinel)
    assert sentinel[0] == 123.5
    with pytest.raises(S.ArgumentException):
        m.execute(np.ones(32, np.float32), np.zeros(2, np.float32))
    buf = np.ones(64, np.float32)
    with pytest.raises(S.ArgumentException):  # overlapping input and output
        m.execute(buf[:32], buf[31:32])
    m.dispose()
    m.dispose()  # idempotent
    with pytest.raises(S.ObjectDisposedException):
        m.execute(np.ones(32, np.float32), sentinel)


def test_create_rejects_invalid_payloads(context):
    with pytest.raises(S.InvalidDataException):
        context.create(np.frombuffer(b"\x00\x7c" + bytes(32), np.uint8), S.QuantizedMatrixShape(1, 32, BQ.Q8_0))
    with pytest.raises(S.ArgumentException):
        context.create(np.zeros(33, np.uint8), S.QuantizedMatrixShape(1, 32, BQ.Q8_0))
    payload = np.zeros(20, np.uint8)
    payload[:4] = np.frombuffer(np.float32(1).tobytes(), np.uint8)
    payload[4] = 3
    with pytest.raises(S.ArgumentException):
        context.create_ternary2(1, 1, 64, payload)


def _t2_block_offset(columns: int, block: int, row: int, index: int) -> int:
    blocks = -(-columns // block)
    return (row * blocks + index) * (4 + block // 4)


def test_device_checked_uploads_name_the_first_failure(context):
    # Ternary2, bitplane and GGUF-format payloads are checked on the device as they are regrouped; a failure is
    # then named by the host rule: the first failing block in row-major order, its scale checked before its
    # codes (Ternary2Matrix.cs:83-101, TernaryBitplaneMatrix.cs:64-85, QuantizedMatVec.cs:28-42), with the
    # reference's message. A failed upload leaves nothing behind: the next valid one succeeds.
    rows, columns, block = 130, 1000, 128  # ragged last panel and last block
    good = S.Ternary2Matrix.quantize(rng(5).standard_normal((rows, columns)).astype(np.float32), rows, columns,
                                     block).data.copy()

    def expect(payload, error, message):
        with pytest.raises(error) as e:
            context.create_ternary2(rows, columns, block, payload).dispose()
        assert message in str(e.value), str(e.value)

    bad = good.copy()
    bad[_t2_block_offset(columns, block, 70, 3) + 4] |= 3  # code 3 in row 70
    o = _t2_block_offset(columns, block, 100, 0)
    bad[o:o + 4] = np.frombuffer(np.float32(np.nan).tobytes(), np.uint8)  # a later bad scale
    expect(bad, S.ArgumentException, "Invalid weight code or padding.")
    o = _t2_block_offset(columns, block, 70, 3)
    bad[o:o + 4] = np.frombuffer(np.uint32(0x80000000).tobytes(), np.uint8)  # -0 scale in the same block
    expect(bad, S.ArgumentException, "Invalid block scale.")
    pad = good.copy()
    pad[_t2_block_offset(columns, block, 129, 7) + 4 + (1000 - 7 * 128) // 4] |= 1  # a code past column 999
    expect(pad, S.ArgumentException, "Invalid weight code or padding.")
    zero = good.copy()
    o = _t2_block_offset(columns, block, 0, 0)
    zero[o:o + 4] = 0  # scale 0 with nonzero codes
    expect(zero, S.ArgumentException, "Invalid weight code or padding.")
    with context.create_ternary2(rows, columns, block, good) as m:
        y = np.zeros(rows, np.float32)
        x = rng(6).uniform(-1, 1, columns).astype(np.float32)
        m.execute(x, y)
        wq = O.t2_dequantize(good, rows, columns, block)
        assert_within(y, O.t2_matvec_scalar(good, rows, columns, block, x), relative_bound(wq, x), "after failures")

    tb = O.tb_from_t2(good, rows, columns, block)
    overlap = tb.copy()
    o = _t2_block_offset(columns, block, 65, 2)
    overlap[o + 4] |= 1
    overlap[o + 4 + block // 8] |= 1  # weight 0 in both planes
    with pytest.raises(S.ArgumentException) as e:
        context.create_bitplane(rows, columns, block, overlap).dispose()
    assert "Overlapping bits, invalid padding or noncanonical zero." in str(e.value)
    scale = tb.copy()
    scale[o:o + 4] = np.frombuffer(np.float32(-1).tobytes(), np.uint8)
    with pytest.raises(S.ArgumentException) as e:
        context.create_bitplane(rows, columns, block, scale).dispose()
    assert "Invalid bitplane scale." in str(e.value)

    for fmt, at in ((BQ.Q6_K, 208), (BQ.Q4_K, 2), (BQ.Q8_0, 0), (BQ.Q4_0, 0)):
        r, c = 40, 512
        data = S.quantize_weights(rng(7).standard_normal((r, c)).astype(np.float32) * 0.1, r, c, fmt).copy()
        block_bytes = {BQ.Q6_K: 210, BQ.Q4_K: 144, BQ.Q8_0: 34, BQ.Q4_0: 18}[fmt]
        for k in (37, 12):  # blocks 37 and 12 get an FP16 infinity; 12 comes first
            data[k * block_bytes + at:k * block_bytes + at + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
        with pytest.raises(S.InvalidDataException) as e:
            context.create(data, S.QuantizedMatrixShape(r, c, fmt)).dispose()
        assert f"Nonfinite block scale at {12 * block_bytes}." in str(e.value), (fmt, str(e.value))


def test_ternary2_upload_in_several_staged_chunks(context):
    # A payload larger than the 64 MB staging chunk is regrouped panel range by panel range (257 panels of
    # 16,384 columns at B = 256, 240 panels a chunk); every row of both chunks equals the oracle, and a bad code
    # in the second chunk is found.
    rows, columns, block = 257 * 64, 16384, 256
    g = rng(8080)
    payload = _t2_random_payload(g, rows, columns, block)
    assert payload.size > 64 << 20
    x = g.uniform(-1, 1, columns).astype(np.float32)
    with context.create_ternary2(rows, columns, block, payload) as m:
        y = np.zeros(rows, np.float32)
        m.execute(x, y)
    want = O.t2_matvec_scalar(payload, rows, columns, block, x)
    # The bound 1e-5 * sum|w * x| per row, as a MatVec of the payload with every -1 code made +1 over |x| (the
    # whole dequantized matrix would take a gigabyte).
    absolute = payload.copy().reshape(-1, 4 + block // 4)
    absolute[:, 4:] = (absolute[:, 4:] & 0x55) | ((absolute[:, 4:] >> 1) & 0x55)
    bound = 1e-5 * O.t2_matvec_scalar(absolute.reshape(-1), rows, columns, block, np.abs(x)).astype(np.float64)
    assert_within(y, want, bound + columns * TINY, "two staged chunks vs scalar")
    bad = payload.copy()
    bad[_t2_block_offset(columns, block, rows - 1, 63) + 4] |= 3
    with pytest.raises(S.ArgumentException):
        context.create_ternary2(rows, columns, block, bad).dispose()


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_0])
def test_legacy_upload_in_several_staged_chunks(context, fmt):
    # Q8_0 / Q4_0 payloads larger than the 64 MB staging chunk are regrouped block range by block range
    # (16,384 x 4,096 Q8_0: 71 MB, two chunks; Q4_0 32,768 x 4,096: 75 MB); rows on both sides of every chunk
    # boundary and the last row equal the oracle's scalar product within the reference's bound.
    rows = 16384 if fmt == BQ.Q8_0 else 32768
    columns = 4096
    block_bytes = 34 if fmt == BQ.Q8_0 else 18
    g = rng(9393 + int(fmt))
    w = g.standard_normal((rows, columns), dtype=np.float32) * 0.02
    data = S.quantize_weights(w, rows, columns, fmt)
    del w
    assert data.size > 64 << 20
    x = g.standard_normal(columns).astype(np.float32)
    with context.create(data, S.QuantizedMatrixShape(rows, columns, fmt)) as m:
        y = np.zeros(rows, np.float32)
        m.execute(x, y)
    per_chunk = (64 << 20) // block_bytes  # blocks of one staged chunk
    blocks_per_row = columns // 32
    edges = {0, rows - 1}
    for c in range(1, (rows * blocks_per_row + per_chunk - 1) // per_chunk):
        r = c * per_chunk // blocks_per_row
        edges.update({max(r - 1, 0), r, min(r + 1, rows - 1)})
    sample = np.array(sorted(edges))
    row_bytes = blocks_per_row * block_bytes
    sub = np.concatenate([data[r * row_bytes:(r + 1) * row_bytes] for r in sample])
    want = O.q_matvec_scalar(sub, sample.size, columns, int(fmt), x)
    wq = O.decode_matrix(sub, sample.size, columns, int(fmt))
    assert_within(y[sample], want, relative_bound(wq, x) + columns * TINY, f"{fmt.name} rows {sample.tolist()}")


def test_k_batch_rejects_too_many_positions(context):
    data = S.quantize_weights(np.zeros((2, 256), np.float32), 2, 256, BQ.Q4_K)
    m = context.create(data, S.QuantizedMatrixShape(2, 256, BQ.Q4_K))
    with pytest.raises(S.ArgumentOutOfRangeException):
        m.execute_batch(np.zeros(257 * 256, np.float32), 257, np.zeros(257 * 2, np.float32))
    with pytest.raises(S.ArgumentOutOfRangeException):
        m.execute_batch(np.zeros(256, np.float32), 0, np.zeros(2, np.float32))
    m.dispose()


def test_device_and_group_entry_points_match_host_calls(context):
    # One launch over several matrices sharing an input (the q/k/v shape of the decode step) must equal
    # the per-matrix host calls bit for bit, for the FP32 and the Q8_K integer products.
    g = rng(11)
    columns = 1536
    mats = []
    for i in range(3):
        rows = 300 + 64 * i
        w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
        data = S.quantize_weights(w, rows, columns, BQ.Q4_K)
        mats.append(context.create(data, S.QuantizedMatrixShape(rows, columns, BQ.Q4_K)))
    x = g.standard_normal(columns).astype(np.float32)
    dx = context.alloc(x.nbytes)
    context.upload(dx, x)
    for quantized in (False, True):
        ys = [context.alloc(4 * m.rows) for m in mats]
        group = S.HipGroup(context, mats, [dx] * 3, ys, quantized)
        group.execute()
        context.synchronize()
        for m, dy in zip(mats, ys):
            ref = np.zeros(m.rows, np.float32)
            if quantized:
                m.execute_batch(x, 1, ref)
            else:
                m.execute(x, ref)
            got = context.download(np.zeros(m.rows, np.float32), dy)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
            if quantized:
                m.execute_batch_device(dx, 1, dy)
            else:
                m.execute_device(dx, dy)
            context.synchronize()
            got = context.download(np.zeros(m.rows, np.float32), dy)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        group.dispose()
        for dy in ys:
            context.free(dy)
    context.free(dx)
    for m in mats:
        m.dispose()


def test_step_graph_replays_match_eager_groups(context):
    # A two-layer projection skeleton of a decode step (q/k/v sharing one Q8_K input, o, gate/up sharing
    # one input, down in Q6_K), plus a Q8_0 float group and a Ternary2 group (main and fix-up kernels),
    # captured once as a graph. Every replay, with eager launches and synchronisations between replays,
    # must write exactly the bits of the eager launches.
    g = rng(31)
    d, ffn = 512, 1024

    def gguf(rows, columns, fmt):
        w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
        return context.create(S.quantize_weights(w, rows, columns, fmt), S.QuantizedMatrixShape(rows, columns, fmt))

    allocs = []

    def buffer(values):
        p = context.alloc(values.nbytes)
        context.upload(p, values)
        allocs.append(p)
        return p

    mats, groups, outs = [], [], []

    def group(members, inputs, quantized):
        ys = [context.alloc(4 * m.rows) for m in members]
        outs.extend(zip(members, ys))
        groups.append(S.HipGroup(context, members, inputs, ys, quantized))

    for _ in range(2):
        q, k, v, o = gguf(d, d, BQ.Q4_K), gguf(128, d, BQ.Q4_K), gguf(128, d, BQ.Q4_K), gguf(d, d, BQ.Q4_K)
        gate, up, down = gguf(ffn, d, BQ.Q4_K), gguf(ffn, d, BQ.Q4_K), gguf(d, ffn, BQ.Q6_K)
        mats += [q, k, v, o, gate, up, down]
        h, attn, h2 = (buffer(g.standard_normal(d).astype(np.float32)) for _ in range(3))
        act = buffer(g.standard_normal(ffn).astype(np.float32))
        group([q, k, v], [h] * 3, True)
        group([o], [attn], True)
        group([gate, up], [h2] * 2, True)
        group([down], [act], True)
    q8 = [gguf(300, d, BQ.Q8_0), gguf(200, d, BQ.Q8_0)]
    t2 = [context.create_ternary2(4096, 1024, 128, _t2_random_payload(g, 4096, 1024, 128)) for _ in range(2)]
    mats += q8 + t2
    xf = buffer(g.standard_normal(d).astype(np.float32))
    xt = buffer(g.uniform(-1, 1, 1024).astype(np.float32))
    group(q8, [xf, xf], False)
    group(t2, [xt, xt], False)

    def read_all():
        context.synchronize()
        return [context.download(np.zeros(m.rows, np.float32), y).view(np.uint32) for m, y in outs]

    def clear_all():
        for m, y in outs:
            context.upload(y, np.full(m.rows, np.nan, np.float32))

    for grp in groups:
        grp.execute()
    eager = read_all()
    step = S.HipStep(context, groups)
    for replay in range(3):
        clear_all()
        step.execute()
        got = read_all()
        for i, (a, b) in enumerate(zip(got, eager)):
            assert np.array_equal(a, b), f"replay {replay}: output {i} differs from the eager launch"
        groups[replay].execute()  # eager work between replays
        context.synchronize()
    with pytest.raises(S.ArgumentException):
        groups[0].dispose()  # replayed by the step
    with pytest.raises(S.ArgumentException):
        mats[0].dispose()  # launched by a group
    step.dispose()
    for grp in groups:
        grp.dispose()
    for m, y in outs:
        context.free(y)
    for p in allocs:
        context.free(p)
    for m in mats:
        m.dispose()


# ---------------------------------------------------------------------------------------------
# GGUF containers to resident matrices (satori_hip_gguf_matrix_create)
# ---------------------------------------------------------------------------------------------

def _gguf_with(tmp_path, tensors):
    """A canonical GGUF v3 file holding `tensors` = [(name, rows, columns, type id, payload)]."""
    import struct

    def s(v):
        raw = v.encode()
        return struct.pack("<Q", len(raw)) + raw

    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 3))
    out += s("general.architecture") + struct.pack("<I", 8) + s("qwen2")
    out += s("general.alignment") + struct.pack("<II", 4, 32)
    out += s("general.quantization_version") + struct.pack("<II", 4, 2)
    offset, blobs = 0, []
    for name, rows, columns, type_, payload in tensors:
        out += s(name) + struct.pack("<IQQIQ", 2, columns, rows, type_, offset)
        padded = bytes(payload) + bytes(-len(payload) % 32)
        blobs.append(padded)
        offset += len(padded)
    out += bytes(-len(out) % 32)
    path = str(tmp_path / "model.gguf")
    with open(path, "wb") as f:
        f.write(bytes(out) + b"".join(blobs))
    return path


def test_gguf_tensors_upload_to_resident_matrices(context, tmp_path):
    # GgufQuantizedMatrix.CreateExecution (GgufQuantizedMatrix.cs:31-36): the device matrix made from the
    # mapped tensor equals the one made from the same bytes through the factory, for every format, on the
    # FP32 path and on the integer K path (single position and the matrix-core batch).
    g = rng(99)
    specs = [("blk.0.attn_q.weight", 300, 512, BQ.Q4_K, 12), ("blk.0.ffn_down.weight", 129, 768, BQ.Q6_K, 14),
             ("blk.0.attn_k.weight", 70, 256, BQ.Q8_0, 8), ("blk.0.attn_v.weight", 33, 320, BQ.Q4_0, 2)]
    tensors, payloads = [], {}
    for name, rows, columns, fmt, type_ in specs:
        data = S.quantize_weights((g.standard_normal((rows, columns)) * 0.05).astype(np.float32), rows, columns, fmt)
        payloads[name] = data
        tensors.append((name, rows, columns, type_, data))
    path = _gguf_with(tmp_path, tensors)
    with S.GgufFile(path) as f:
        store = S.GgufWeightStore(f, context)
        for name, rows, columns, fmt, _ in specs:
            assert store.has(name)
            m = store.matrix(name)
            ref = context.create(payloads[name], S.QuantizedMatrixShape(rows, columns, fmt))
            x = g.standard_normal(columns).astype(np.float32)
            y, y_ref = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
            m.execute(x, y)
            ref.execute(x, y_ref)
            assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), name
            if fmt in (BQ.Q4_K, BQ.Q6_K):
                for positions in (1, 20):
                    xb = g.standard_normal(positions * columns).astype(np.float32)
                    yb, yb_ref = np.zeros(positions * rows, np.float32), np.zeros(positions * rows, np.float32)
                    store.project_batch(name, xb, positions, yb)
                    ref.execute_batch(xb, positions, yb_ref)
                    assert np.array_equal(yb.view(np.uint32), yb_ref.view(np.uint32)), (name, positions)
            ref.dispose()
        store.dispose()


@pytest.mark.parametrize("fmt,type_,byte", [(BQ.Q4_K, 12, 2), (BQ.Q6_K, 14, 208), (BQ.Q8_0, 8, 0), (BQ.Q4_0, 2, 0)])
def test_gguf_device_scale_check_rejects_nonfinite_scales(context, tmp_path, fmt, type_, byte):
    # QuantizedMatVec.ValidatePayload (QuantizedMatVec.cs:28-42) run on the device copy: a NaN scale in the
    # last block of the last row (Q4_K's dmin, Q6_K's d at byte 208) fails with InvalidData naming its
    # offset, and a clean tensor of the same file still uploads.
    g = rng(7)
    rows, columns = 37, 512
    data = S.quantize_weights((g.standard_normal((rows, columns)) * 0.05).astype(np.float32), rows, columns, fmt)
    bad = data.copy()
    block_bytes = {BQ.Q4_K: 144, BQ.Q6_K: 210, BQ.Q8_0: 34, BQ.Q4_0: 18}[fmt]
    last = bad.size - block_bytes
    bad[last + byte:last + byte + 2] = [0x00, 0x7E]  # FP16 NaN
    path = _gguf_with(tmp_path, [("bad", rows, columns, type_, bad), ("good", rows, columns, type_, data)])
    with S.GgufFile(path) as f:
        handle = ctypes_matrix_from_gguf(context, f, "bad")
        assert handle[0] == S.InvalidDataException.status and str(last) in handle[1]
        m = S.GgufQuantizedMatrix(f, "good").create_execution(context)
        x = g.standard_normal(columns).astype(np.float32)
        y, y_ref = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
        m.execute(x, y)
        with context.create(data, S.QuantizedMatrixShape(rows, columns, fmt)) as ref:
            ref.execute(x, y_ref)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        m.dispose()


def ctypes_matrix_from_gguf(context, f, name):
    """Raw C-ABI call (the Python binding would check the payload on the host first): status and message."""
    import ctypes
    from satori_amd import _ffi
    handle = ctypes.c_void_p()
    status = _ffi.lib().satori_hip_gguf_matrix_create(context.handle, f.handle, f.tensor_index(name),
                                                       ctypes.byref(handle))
    message = _ffi.lib().satori_hip_last_error().decode()
    assert not handle.value or status == 0
    return status, message


def test_golden_gguf_file_through_the_container(context):
    # The reference's q8_0.gguf / q4_0.gguf tensors opened as containers: ones-dot = -8 per row, as the
    # manifest's FP64 decode gives (test_golden_gguf_ones_dot reads the same bytes by offset).
    import os
    from helpers import GOLDEN
    for name in ("q8_0.gguf", "q4_0.gguf"):
        with S.GgufFile(os.path.join(GOLDEN, name)) as f:
            m = S.GgufQuantizedMatrix(f, "weights")
            y = np.zeros(m.shape.rows, np.float32)
            m.execute(np.ones(m.shape.columns, np.float32), y)
            data, _ = gguf_tensor(name)
            expected = O.q_matvec_scalar(data, m.shape.rows, m.shape.columns, int(m.shape.format),
                                         np.ones(m.shape.columns, np.float32))
            assert np.array_equal(y, expected) and y.tolist() == [-8.0], name
            m.dispose()


# ---------------------------------------------------------------------------------------------
# Ternary bitplane layout (executes as its lossless Ternary2 equivalent)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("block", [64, 128, 256])
def test_bitplane_same_corpus_and_results_as_ternary2_including_tails(context, block):
    # TernaryBitplaneAvx2Tests.cs:7-47: the bitplane product equals the Ternary2 product of the same weights
    # (here bit for bit on the device) and stays within the NumericalValidation bound of the FP64 product;
    # corpus cases plus column tails 1..17, 31..33, 63..65, 127..129, 255..257.
    cases = [(name, w, x) for name, w, x in _critical_cases(block)]
    for columns in list(range(1, 18)) + [31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257]:
        w, x = O.corpus_random_matrix(3, columns)
        cases.append((f"C={columns}", w, x))
    for name, w, x in cases:
        rows, columns = w.shape
        t2 = S.Ternary2Matrix.quantize(w, rows, columns, block)
        tb = S.TernaryBitplaneMatrix.from_ternary2(t2)
        y_t2, y_tb = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
        with context.create_ternary2(rows, columns, block, t2.data) as m:
            m.execute(x, y_t2)
        S.TernaryBitplaneMatVec.execute(tb, x, y_tb, context)
        assert np.array_equal(y_t2.view(np.uint32), y_tb.view(np.uint32)), name
        wq = O.t2_dequantize(t2.data, rows, columns, block).reshape(rows, columns)
        assert_within(y_tb, fp64_matvec(wq, x), ternary2_bound(wq, x, block), f"{name} B{block}")
        scalar = O.tb_matvec_scalar(tb.data, rows, columns, block, x)
        assert_within(y_tb, scalar, relative_bound(wq, x) + (columns + 8) * TINY, f"{name} B{block} vs scalar")
        tb.device(context).dispose()


def test_bitplane_file_opens_to_the_same_device_matrix(context, tmp_path):
    # TernaryBitplaneMatrix.Load (TernaryBitplaneMatrix.cs:98-117) then execution: the STB1 file, opened on
    # the device, gives the same outputs as the owned matrix; a corrupt file is InvalidData.
    g = rng(1234)
    rows, columns, block = 4099, 1000, 128
    w = g.standard_normal((rows, columns)).astype(np.float32)
    tb = S.TernaryBitplaneMatrix.from_ternary2(S.Ternary2Matrix.quantize(w, rows, columns, block))
    path = str(tmp_path / "w.stb1")
    tb.save(path)
    x = g.uniform(-1, 1, columns).astype(np.float32)
    y_owned, y_file = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    S.TernaryBitplaneMatVec.execute(tb, x, y_owned, context)
    with context.open_bitplane(path) as m:
        assert (m.rows, m.columns, m.byte_length) == (rows, columns, tb.byte_length)
        m.execute(x, y_file)
    assert np.array_equal(y_owned.view(np.uint32), y_file.view(np.uint32))
    with open(path, "r+b") as f:
        f.seek(32 + 4)  # first block: set a bit in both planes
        f.write(bytes([0xFF]))
        f.seek(32 + 4 + block // 8)
        f.write(bytes([0xFF]))
    with pytest.raises(S.InvalidDataException):
        context.open_bitplane(path)
    tb.device(context).dispose()


# ---------------------------------------------------------------------------------------------
# Decode-step operators (TransformerOps on the device) and embedding-row decode
# ---------------------------------------------------------------------------------------------

def _within_fixture(actual, expected, name):
    # TransformerOpsTests.cs:13-16 / QwenOperatorTests.cs:19-26: |a - e| <= 2e-6 + 2e-6 |e|.
    actual, expected = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    assert np.all(np.isfinite(actual)), name
    err = np.abs(actual - expected)
    assert np.all(err <= 2e-6 + 2e-6 * np.abs(expected)), f"{name}: max err {err.max()}"


def _within_ulp(actual, expected, name, ulps=1):
    # FP64 intermediates that differ only in their last bits (tree sums, device exp/sin/cos/pow) round to
    # FP32 outputs at most one unit in the last place apart.
    a, e = np.asarray(actual, np.float32), np.asarray(expected, np.float32)
    spacing = np.spacing(np.maximum(np.abs(a), np.abs(e)).astype(np.float32)).astype(np.float64)
    err = np.abs(a.astype(np.float64) - e.astype(np.float64))
    assert np.all(err <= ulps * spacing), f"{name}: max err {err.max()} at {np.argmax(err - ulps * spacing)}"


def test_operators_match_reference_fixtures(context):
    # TransformerOpsTests.cs:8-25 and QwenOperatorTests.cs:28-112 on the device.
    T = S.TransformerOps
    d = load_json("transformer-v1.json")
    f = lambda k: np.array(d[k], np.float32)
    out = np.zeros(96, np.float32)
    T.rms_norm(f("x"), f("weights"), 1e-5, out, context)
    _within_fixture(out, d["rms"], "rms")
    x = f("x")
    T.rope(x, 48, 37, context)
    _within_fixture(x, d["rope"], "rope")
    out = np.zeros(8, np.float32)
    T.swiglu(f("gate"), f("up"), out, context)
    _within_fixture(out, d["swiglu"], "swiglu")
    out = np.zeros(96, np.float32)
    T.attention(f("query"), f("keys"), f("values"), 48, 7, out, context)
    _within_fixture(out, d["attention"], "attention")
    d2 = load_json("transformer-v2.json")
    F = lambda v: np.array(v, np.float32)
    g = d2["gqa"]
    out = np.zeros(len(g["query"]), np.float32)
    T.grouped_attention(F(g["query"]), F(g["keys"]), F(g["values"]), g["query_heads"], g["kv_heads"], g["head_dim"],
                        g["tokens"], out, context)
    _within_fixture(out, g["output"], "gqa")
    for key in ("rope_full", "rope_partial"):
        r = d2[key]
        v = F(r["input"])
        T.rope_half(v, r["head_dim"], r["position"], r["base"], r["rotary"], context)
        _within_fixture(v, r["output"], key)
    n = d2["qk_norm"]
    v = F(n["input"])
    T.rms_norm_heads(v, F(n["weights"]), np.float32(n["epsilon"]), len(n["weights"]), context)
    _within_fixture(v, n["output"], "qk_norm")
    b = d2["bias"]
    out = np.zeros(len(b["base"]), np.float32)
    T.add(F(b["base"]), F(b["bias"]), out, context)
    _within_fixture(out, b["output"], "bias")


def test_operators_match_oracle_at_decode_sizes(context):
    # Qwen-1.5B-shaped decode vectors: hidden 1536, FFN 8960, 12 query heads / 2 KV heads of 128 lanes, a KV
    # prefix of 1 .. 2048 tokens, RoPE base 1e6 at a large position. FP32 outputs within one unit in the
    # last place of the oracle's; Add exactly.
    T = S.TransformerOps
    g = rng(808)
    x = (g.standard_normal(1536) * 3).astype(np.float32)
    w = g.uniform(0.5, 1.5, 1536).astype(np.float32)
    out = np.zeros(1536, np.float32)
    T.rms_norm(x, w, 1e-6, out, context)
    _within_ulp(out, O.rms_norm(x, w, np.float32(1e-6)), "rms_norm")
    q = g.standard_normal(12 * 128).astype(np.float32)
    for position in (0, 1, 4095, 100000):
        v = q.copy()
        T.rope_half(v, 128, position, 1e6, 128, context)
        _within_ulp(v, O.rope_half(q, 128, position, 1e6, 128), f"rope_half {position}")
        v = q.copy()
        T.rope(v, 128, position, context)
        _within_ulp(v, O.rope(q, 128, position), f"rope {position}")
    v = q.copy()
    T.rms_norm_heads(v, w[:128], 1e-6, 128, context)
    _within_ulp(v, O.rms_norm_heads(q, w[:128], np.float32(1e-6), 128), "rms_norm_heads")
    gate = (g.standard_normal(8960) * 6).astype(np.float32)
    up = g.standard_normal(8960).astype(np.float32)
    out = np.zeros(8960, np.float32)
    T.swiglu(gate, up, out, context)
    _within_ulp(out, O.swiglu(gate, up), "swiglu")
    T.add(gate, up, out, context)
    assert np.array_equal(out, O.add(gate, up))
    for tokens in (1, 2, 33, 257, 2048, 6912):
        keys = g.standard_normal(tokens * 256).astype(np.float32)
        values = g.standard_normal(tokens * 256).astype(np.float32)
        out = np.zeros(12 * 128, np.float32)
        T.grouped_attention(q, keys, values, 12, 2, 128, tokens, out, context)
        _within_ulp(out, O.grouped_attention(q, keys, values, 12, 2, 128, tokens), f"attention {tokens}")
    # Split prefixes at other head widths: 96 (eighths of 12 lanes), 256, and 80 (eighths that are not whole
    # 16-byte quads: lane-by-lane key loads), with 7 query heads per key/value head.
    for head_dim, tokens in ((96, 100), (256, 65), (80, 300)):
        qq = g.standard_normal(14 * head_dim).astype(np.float32)
        keys = g.standard_normal(tokens * 2 * head_dim).astype(np.float32)
        values = g.standard_normal(tokens * 2 * head_dim).astype(np.float32)
        out = np.zeros(14 * head_dim, np.float32)
        T.grouped_attention(qq, keys, values, 14, 2, head_dim, tokens, out, context)
        _within_ulp(out, O.grouped_attention(qq, keys, values, 14, 2, head_dim, tokens),
                    f"attention {head_dim} x {tokens}")


def test_operator_extremes_and_argument_errors(context):
    # TransformerOpsTests.cs:27-53 and QwenOperatorTests.cs:138-144.
    T = S.TransformerOps
    fmax = np.finfo(np.float32).max
    x = np.array([fmax, -fmax], np.float32)
    out = np.zeros(2, np.float32)
    T.rms_norm(x, np.ones(2, np.float32), 1e-5, out, context)
    assert out.tolist() == [1.0, -1.0]
    out = np.zeros(2, np.float32)
    T.attention(np.array([fmax, fmax], np.float32), np.array([fmax, fmax, -fmax, -fmax], np.float32),
                np.array([3, 4, 100, 200], np.float32), 2, 2, out, context)
    assert out.tolist() == [3.0, 4.0]
    with pytest.raises(S.ArgumentOutOfRangeException):
        T.rope(np.zeros(8, np.float32), 3, 0, context)
    with pytest.raises(S.ArgumentOutOfRangeException):
        T.rope_half(np.zeros(8, np.float32), 8, 0, 10000, 5, context)
    with pytest.raises(S.ArgumentOutOfRangeException):
        T.rms_norm(np.ones(4, np.float32), np.ones(4, np.float32), 0.0, np.zeros(4, np.float32), context)
    with pytest.raises(S.ArgumentException):
        T.grouped_attention(np.zeros(32, np.float32), np.zeros(48, np.float32), np.zeros(48, np.float32), 4, 3, 8, 3,
                            np.zeros(32, np.float32), context)
    # No prefix cap (TransformerOps.cs:140-179): 6,913 tokens of one two-lane head run split, like any length.
    keys = np.linspace(-1, 1, 2 * 6913).astype(np.float32)
    out = np.zeros(2, np.float32)
    T.attention(np.array([0.5, -0.25], np.float32), keys, keys[::-1].copy(), 2, 6913, out, context)
    _within_ulp(out, O.grouped_attention(np.array([0.5, -0.25], np.float32), keys, keys[::-1].copy(), 1, 1, 2, 6913),
                "attention 6913")
    # Partial overlap of device ranges is rejected before anything runs (TransformerOps.cs:7-11).
    import ctypes
    from satori_amd import _ffi
    buf = context.alloc(64)
    status = _ffi.lib().satori_hip_add(context.handle, ctypes.c_void_p(buf), ctypes.c_void_p(buf), 4,
                                       ctypes.c_void_p(buf + 4), None)
    assert status == S.ArgumentException.status
    context.free(buf)


@pytest.mark.parametrize("fmt", [BQ.Q8_0, BQ.Q4_K, BQ.Q6_K, BQ.Q4_0])
def test_embedding_rows_decode_like_the_reference(context, fmt):
    # GgufQuantizedMatrix.ReadRow (GgufQuantizedMatrix.cs:54-61) / QuantizedRow.DecodeRow: every decoded row
    # equals the oracle's decode bit for bit (Q6_K from its regrouped device layout); Q4_0 is not supported.
    g = rng(55)
    rows, columns = 37, 768
    w = (g.standard_normal((rows, columns)) * 0.1).astype(np.float32)
    data = S.quantize_weights(w, rows, columns, fmt)
    m = context.create(data, S.QuantizedMatrixShape(rows, columns, fmt))
    row_bytes = data.size // rows
    out = np.zeros(columns, np.float32)
    if fmt == BQ.Q4_0:
        with pytest.raises(S.NotSupportedException):
            m.read_row(0, out)
    else:
        for r in (0, 1, 17, rows - 1):
            m.read_row(r, out)
            expected = O.q_decode_row(data[r * row_bytes:(r + 1) * row_bytes], columns, int(fmt))
            assert np.array_equal(out.view(np.uint32), expected.view(np.uint32)), r
        with pytest.raises(S.ArgumentOutOfRangeException):
            m.read_row(rows, out)
    m.dispose()


# ---------------------------------------------------------------------------------------------
# A whole decode token on the device (DenseForward.Step + Final), eager and captured
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
def test_group_input_transforms_equal_separate_operators(context, fmt):
    # A K group computing its input from the operators' operands (RmsNorm(a + b), RmsNorm(a), SwiGlu(a, b))
    # equals the operator launch followed by the plain group, bit for bit, and writes a + b once.
    g = rng(31 + int(fmt))
    columns, rows = 1536, [300, 64]
    mats = [context.create(S.quantize_weights((g.standard_normal((r, columns)) * 0.02).astype(np.float32), r,
                                              columns, fmt), S.QuantizedMatrixShape(r, columns, fmt)) for r in rows]
    a, b, w = (g.standard_normal(columns).astype(np.float32) for _ in range(3))
    b[7] = -a[7]  # a zero of the sum
    buffers = []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    da, db, dw, dx = dev(a), dev(b), dev(w), dev(np.zeros(columns, np.float32))
    dres = dev(np.zeros(columns, np.float32))
    ys = [dev(np.zeros(r, np.float32)) for r in rows]
    ops = S.DeviceOps(context)
    plain = S.HipGroup(context, mats, [dx, dx], ys, True)
    fused = S.HipGroup(context, mats, [dx, dx], [dev(np.zeros(r, np.float32)) for r in rows], True)
    fused_out = buffers[-2:]
    try:
        def compare(tag):
            for y0, y1, r in zip(ys, fused_out, rows):
                want = context.download(np.zeros(r, np.float32), y0)
                got = context.download(np.zeros(r, np.float32), y1)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), tag

        # RmsNorm(a + b): the operator adds into a copy of a and normalises into x.
        dsum = dev(a.copy())
        ops.add_rms_norm(dsum, db, dw, 1e-6, columns, dx)
        plain.execute()
        fused.set_input_add_rms_norm(da, db, dw, 1e-6, dres)
        fused.execute()
        compare("add_rms_norm")
        assert np.array_equal(context.download(np.zeros(columns, np.float32), dres).view(np.uint32),
                              context.download(np.zeros(columns, np.float32), dsum).view(np.uint32))
        # RmsNorm(a) without an addend.
        ops.rms_norm(da, dw, 1e-6, columns, dx)
        plain.execute()
        fused.set_input_add_rms_norm(da, 0, dw, 1e-6)
        fused.execute()
        compare("rms_norm")
        # SwiGlu(a, b).
        ops.swiglu(da, db, columns, dx)
        plain.execute()
        fused.set_input_swiglu(da, db)
        fused.execute()
        compare("swiglu")
        # Errors: many positions, overlapping output, unknown kind, FP32-activation groups.
        with pytest.raises(S.NotSupportedException):
            fused.execute_batch(16)
        with pytest.raises(S.ArgumentException):
            fused.set_input_add_rms_norm(da, db, dw, 1e-6, da)
        with pytest.raises(S.ArgumentException):  # an output of the group
            fused.set_input_add_rms_norm(da, db, dw, 1e-6, fused_out[0])
        with pytest.raises(S.ArgumentOutOfRangeException):
            _check_status(S._ffi.lib().satori_hip_group_set_input(fused._handle, 9, None, None, None, 0.0, None))
        float_group = S.HipGroup(context, mats[:1], [dx], [ys[0]], False)
        with pytest.raises(S.NotSupportedException):
            float_group.set_input_swiglu(da, db)
        float_group.dispose()
        fused.set_input_plain()
        fused.execute()
        plain.execute()
        compare("plain again")
    finally:
        plain.dispose()
        fused.dispose()
        for p in buffers:
            context.free(p)
        for m in mats:
            m.dispose()


@pytest.mark.parametrize("fmt", [BQ.Q4_K, BQ.Q6_K])
@pytest.mark.parametrize("columns", [1536, 8960, 29696])
def test_q8k_input_from_the_producer_equals_quantizing_in_the_launch(context, fmt, columns):
    # SwiGlu writing the Q8_K bytes of its output (satori_hip_swiglu_q8k), the device quantizer
    # (satori_hip_quantize_q8k_device) and a group reading those bytes (SATORI_HIP_INPUT_Q8K): the bytes are
    # the oracle's Q8KCodec.QuantizeRow of the FP32 values, and the group's outputs equal the plain group's
    # over the FP32 input bit for bit.
    g = rng(6262 + columns + int(fmt))
    rows = [200, 96]
    mats = [context.create(S.quantize_weights((g.standard_normal((r, columns)) * 0.02).astype(np.float32), r,
                                              columns, fmt), S.QuantizedMatrixShape(r, columns, fmt)) for r in rows]
    gate = (g.standard_normal(columns) * 4).astype(np.float32)
    up = g.standard_normal(columns).astype(np.float32)
    gate[256:512] = -200.0  # a block whose SwiGlu outputs are all (negative) zeros
    buffers = []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    q8k_bytes = columns // 256 * 292
    dgate, dup = dev(gate), dev(up)
    dact, dact2 = dev(np.zeros(columns, np.float32)), dev(np.zeros(columns, np.float32))
    dq, dq2 = dev(np.zeros(q8k_bytes // 4, np.float32)), dev(np.zeros(q8k_bytes // 4, np.float32))
    plain_out = [dev(np.zeros(r, np.float32)) for r in rows]
    q8k_out = [dev(np.zeros(r, np.float32)) for r in rows]
    plain = S.HipGroup(context, mats, [dact, dact], plain_out, True)
    fed = S.HipGroup(context, mats, [dact, dact], q8k_out, True)
    ops = S.DeviceOps(context)
    try:
        ops.swiglu(dgate, dup, columns, dact)
        ops.swiglu_q8k(dgate, dup, columns, dact2, dq)
        act = context.download(np.zeros(columns, np.float32), dact)
        assert np.array_equal(context.download(np.zeros(columns, np.float32), dact2).view(np.uint32), act.view(np.uint32))
        q = context.download(np.zeros(q8k_bytes, np.uint8), dq)
        assert np.array_equal(q, O.q8k_quantize_row(act)), "SwiGlu Q8_K bytes"
        ops.quantize_q8k(dact, columns, 1, dq2)
        assert np.array_equal(context.download(np.zeros(q8k_bytes, np.uint8), dq2), q), "device quantizer"
        ops.swiglu_q8k(dgate, dup, columns, 0, dq2)  # no FP32 output
        assert np.array_equal(context.download(np.zeros(q8k_bytes, np.uint8), dq2), q)
        plain.execute()
        fed.set_input_q8k(dq)
        fed.execute()
        for k, r in enumerate(rows):
            want = context.download(np.zeros(r, np.float32), plain_out[k])
            got = context.download(np.zeros(r, np.float32), q8k_out[k])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"member {k}"
        with pytest.raises(S.NotSupportedException):
            fed.execute_batch(16)
        with pytest.raises(S.ArgumentException):  # not a multiple of 256
            ops.swiglu_q8k(dgate, dup, 300, 0, dq)
    finally:
        plain.dispose()
        fed.dispose()
        for p in buffers:
            context.free(p)
        for m in mats:
            m.dispose()


@pytest.mark.parametrize("fmt,rows,columns,transform,with_q8k", [
    (BQ.Q4_K, 8960, 1536, "add_rms_norm", True),  # the decode step's gate/up (16 rows per workgroup)
    (BQ.Q4_K, 8960, 1536, "add_rms_norm", False),
    (BQ.Q4_K, 8960, 1536, "plain", True),
    (BQ.Q6_K, 1280, 1536, "q8k", True),
    (BQ.Q6_K, 1280, 1536, "q8k", False),
    (BQ.Q4_K, 256, 1536, "plain", True),          # one run of 256 rows, 4 rows per workgroup (64 arrivals)
    (BQ.Q6_K, 512, 29696, "plain", True),         # input staged in chunks of blocks
])
def test_gate_up_group_carrying_swiglu(context, fmt, rows, columns, transform, with_q8k):
    # A gate/up group with the SwiGlu output (satori_hip_group_set_output): the members' outputs equal the
    # plain group's bit for bit, `activated` is the oracle's SwiGlu of those outputs and (with q8k) `q8k` its
    # Q8KCodec.QuantizeRow bytes, on repeated launches (the arrival counts carry over) and in a captured step
    # replayed several times with new inputs between replays. Rows 256..511 of `up` are zero, so that run's
    # SwiGlu values are all zeros (the all-zero Q8_K block).
    g = rng(4242 + rows + columns + int(fmt))
    wg = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    wu = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    if rows >= 512:
        wu[256:512] = 0.0
    mats = [context.create(S.quantize_weights(w, rows, columns, fmt), S.QuantizedMatrixShape(rows, columns, fmt))
            for w in (wg, wu)]
    buffers = []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    q8k_bytes = rows // 256 * 292
    dx = dev(np.zeros(columns, np.float32))
    da, db, dw = (dev(np.zeros(columns, np.float32)) for _ in range(3))
    dres = dev(np.zeros(columns, np.float32))
    dq_in = dev(np.zeros(columns // 256 * 73, np.float32))
    plain_out = [dev(np.zeros(rows, np.float32)) for _ in range(2)]
    paired_out = [dev(np.zeros(rows, np.float32)) for _ in range(2)]
    dact = dev(np.zeros(rows, np.float32))
    dq = dev(np.zeros(q8k_bytes // 4, np.float32))
    ops = S.DeviceOps(context)
    plain = S.HipGroup(context, mats, [dx, dx], plain_out, True)
    paired = S.HipGroup(context, mats, [dx, dx], paired_out, True)
    step = None
    try:
        if transform == "add_rms_norm":
            paired.set_input_add_rms_norm(da, db, dw, 1e-6, dres)
        elif transform == "q8k":
            paired.set_input_q8k(dq_in)
        paired.set_output_swiglu(dact, dq if with_q8k else 0)

        def feed(seed):
            # New operands; x is what the plain group reads (the operator's output for the transforms).
            h = rng(seed)
            a, b = h.standard_normal(columns).astype(np.float32), h.standard_normal(columns).astype(np.float32)
            w = h.uniform(0.5, 1.5, columns).astype(np.float32)
            for p, v in ((da, a), (db, b), (dw, w)):
                context.upload(p, v)
            if transform == "add_rms_norm":
                dsum = dev(a.copy())
                ops.add_rms_norm(dsum, db, dw, 1e-6, columns, dx)
            else:
                context.upload(dx, a)
                if transform == "q8k":
                    context.upload(dq_in, O.q8k_quantize_row(a).view(np.float32))
            context.upload(dact, np.full(rows, np.nan, np.float32))
            context.upload(dq, np.full(q8k_bytes // 4, np.nan, np.float32))
            plain.execute()

        def check(tag):
            outs = []
            for k in range(2):
                want = context.download(np.zeros(rows, np.float32), plain_out[k])
                got = context.download(np.zeros(rows, np.float32), paired_out[k])
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{tag}: member {k}"
                outs.append(want)
            act = O.swiglu(outs[0], outs[1])
            got_act = context.download(np.zeros(rows, np.float32), dact)
            assert np.array_equal(got_act.view(np.uint32), act.view(np.uint32)), f"{tag}: SwiGlu"
            got_q = context.download(np.zeros(q8k_bytes, np.uint8), dq)
            if not with_q8k:
                assert np.isnan(got_q.view(np.float32)).all(), f"{tag}: q8k written without being asked for"
                return
            assert np.array_equal(got_q, O.q8k_quantize_row(act)), f"{tag}: Q8_K bytes"
            if rows >= 512:
                assert not got_q[292:584].any(), f"{tag}: the zero run"

        for seed in (1, 2, 3):  # repeated launches
            feed(seed)
            paired.execute()
            check(f"launch {seed}")
        step = S.HipStep(context, [paired])
        for seed in (4, 5, 6):  # graph replays, eager work between them
            feed(seed)
            step.execute()
            check(f"replay {seed}")
        with pytest.raises(S.NotSupportedException):
            paired.execute_batch(16)
    finally:
        if step is not None:
            step.dispose()
        plain.dispose()
        paired.dispose()
        for p in buffers:
            context.free(p)
        for m in mats:
            m.dispose()


def test_swiglu_output_argument_checks(context):
    # The SwiGlu output's preconditions: two K members with equal row counts, a multiple of 256, quantized
    # activations, no overlap, no SwiGlu input transform; SATORI_HIP_OUTPUT_PLAIN restores the plain launch.
    g = rng(77)
    columns = 1536

    def mat(rows, fmt=BQ.Q4_K):
        w = (g.standard_normal((rows, columns)) * 0.02).astype(np.float32)
        return context.create(S.quantize_weights(w, rows, columns, fmt), S.QuantizedMatrixShape(rows, columns, fmt))

    mats = [mat(512), mat(512), mat(384), mat(300), mat(300)]
    buffers = []

    def dev(n):
        p = context.alloc(4 * n)
        context.upload(p, np.zeros(n, np.float32))
        buffers.append(p)
        return p

    dx, dact, dq = dev(columns), dev(512), dev(2 * 73)
    ys = [dev(512) for _ in range(4)]
    groups = []
    try:
        def group(ms, quantized=True):
            grp = S.HipGroup(context, ms, [dx] * len(ms), ys[:len(ms)], quantized)
            groups.append(grp)
            return grp

        good = group(mats[:2])
        with pytest.raises(S.ArgumentException):  # three members
            group(mats[:3]).set_output_swiglu(dact, dq)
        with pytest.raises(S.ArgumentException):  # different row counts
            group([mats[0], mats[2]]).set_output_swiglu(dact, dq)
        with pytest.raises(S.ArgumentException):  # rows not a multiple of 256
            group(mats[3:5]).set_output_swiglu(dact, dq)
        with pytest.raises(S.NotSupportedException):  # FP32-activation group
            group(mats[:2], False).set_output_swiglu(dact, dq)
        with pytest.raises(S.ArgumentException):  # activated overlaps an output
            good.set_output_swiglu(ys[0], dq)
        with pytest.raises(S.ArgumentException):  # q8k overlaps the input
            good.set_output_swiglu(dact, dx)
        with pytest.raises(S.ArgumentNullException):
            good.set_output_swiglu(0, dq)
        with pytest.raises(S.ArgumentOutOfRangeException):
            _check_status(S._ffi.lib().satori_hip_group_set_output(good._handle, 7, None, None))
        good.set_output_swiglu(dact)  # SwiGlu without its Q8_K bytes
        good.set_output_swiglu(dact, dq)
        with pytest.raises(S.NotSupportedException):
            good.set_input_swiglu(dx, dx)
        good.set_output_plain()
        good.set_input_swiglu(dx, dx)
        with pytest.raises(S.NotSupportedException):
            good.set_output_swiglu(dact, dq)
        # An input transform's operands (and residual_out) are the launch's inputs: neither output buffer may
        # overlap them, whichever of the two calls comes second.
        good.set_input_plain()
        dres, dadd, dnw, dres_out = dev(columns), dev(columns), dev(columns), dev(columns)
        good.set_input_add_rms_norm(dres, dadd, dnw, 1e-6, dres_out)
        for operand in (dres, dadd, dnw, dres_out):
            with pytest.raises(S.ArgumentException):
                good.set_output_swiglu(operand, dq)
        with pytest.raises(S.ArgumentException):  # q8k over the residual
            good.set_output_swiglu(dact, dres)
        good.set_output_swiglu(dact, dq)
        with pytest.raises(S.ArgumentException):  # the residual over activated
            good.set_input_add_rms_norm(dact, dadd, dnw, 1e-6)
        with pytest.raises(S.ArgumentException):  # residual_out over q8k
            good.set_input_add_rms_norm(dres, dadd, dnw, 1e-6, dq)
        with pytest.raises(S.ArgumentException):  # producer Q8_K bytes over activated
            good.set_input_q8k(dact)
        good.set_input_add_rms_norm(dres, dadd, dnw, 1e-6, dres_out)  # disjoint operands are accepted
    finally:
        for grp in groups:
            grp.dispose()
        for p in buffers:
            context.free(p)
        for m in mats:
            m.dispose()


@pytest.mark.parametrize("columns", [1536, 8960, 12288, 16384])
def test_add_rms_norm_q8k_equals_add_rms_norm_then_quantizer(context, columns):
    # satori_hip_add_rms_norm_q8k: residual, normed and the Q8_K bytes equal satori_hip_add_rms_norm followed
    # by the device quantizer bit for bit, and the bytes equal the oracle's Q8KCodec.QuantizeRow of `normed`
    # (12,288 columns is the longest row the single launch keeps in LDS; 16,384 takes the two-launch form).
    g = rng(4545 + columns)
    residual = (g.standard_normal(columns) * 3).astype(np.float32)
    addend = g.standard_normal(columns).astype(np.float32)
    weights = g.uniform(0.5, 1.5, columns).astype(np.float32)
    weights[512:768] = 0.0  # a block whose normalised values are all zeros
    q8k_bytes = columns // 256 * 292
    buffers = []

    def dev(arr):
        p = context.alloc(arr.nbytes)
        context.upload(p, arr)
        buffers.append(p)
        return p

    ops = S.DeviceOps(context)
    try:
        r1, r2, da, dw = dev(residual), dev(residual), dev(addend), dev(weights)
        n1, n2 = dev(np.zeros(columns, np.float32)), dev(np.zeros(columns, np.float32))
        q1, q2 = dev(np.zeros(q8k_bytes // 4, np.float32)), dev(np.full(q8k_bytes // 4, np.nan, np.float32))
        ops.add_rms_norm(r1, da, dw, 1e-6, columns, n1)
        ops.quantize_q8k(n1, columns, 1, q1)
        ops.add_rms_norm_q8k(r2, da, dw, 1e-6, columns, n2, q2)
        down = lambda p, n, t=np.float32: context.download(np.zeros(n, t), p)
        assert np.array_equal(down(r2, columns).view(np.uint32), down(r1, columns).view(np.uint32)), "residual"
        normed = down(n1, columns)
        assert np.array_equal(down(n2, columns).view(np.uint32), normed.view(np.uint32)), "normed"
        q = down(q2, q8k_bytes, np.uint8)
        assert np.array_equal(q, down(q1, q8k_bytes, np.uint8)), "Q8_K bytes"
        assert np.array_equal(q, O.q8k_quantize_row(normed)), "Q8_K bytes against the oracle"
        with pytest.raises(S.ArgumentException):  # not a multiple of 256
            ops.add_rms_norm_q8k(r2, da, dw, 1e-6, columns - 100, n2, q2)
        with pytest.raises(S.ArgumentOutOfRangeException):  # the operator's epsilon rule
            ops.add_rms_norm_q8k(r2, da, dw, 0.0, columns, n2, q2)
    finally:
        for p in buffers:
            context.free(p)


def test_device_q8k_quantizer_positions_match_oracle(context):
    g = rng(808)
    columns, positions = 2048, 5
    x = g.standard_normal((positions, columns)).astype(np.float32)
    x[1] = 0
    x[2, :256] = 1e-30
    dx = context.alloc(x.nbytes)
    dq = context.alloc(positions * columns // 256 * 292)
    try:
        context.upload(dx, x)
        S.DeviceOps(context).quantize_q8k(dx, columns, positions, dq)
        got = context.download(np.zeros(positions * columns // 256 * 292, np.uint8), dq).reshape(positions, -1)
        for p in range(positions):
            assert np.array_equal(got[p], O.q8k_quantize_row(x[p])), p
    finally:
        context.free(dx)
        context.free(dq)


def _check_status(code):
    S._check(code)


def test_device_decode_token_matches_host_composition(context):
    # DenseForward.Step / Final (DenseForward.cs:100-162, 298-306) on a small random model: the device token
    # (eager, and captured then replayed three times with eager work in between) against the same sequence
    # composed on the host from the oracle's operators and integer projections. Eager and replayed logits
    # are bit-identical; against the host they agree to 1e-3 of the largest logit (operator outputs within
    # one unit in the last place can move a Q8_K code of a later projection by one step).
    from satori_amd.decode import DecoderConfig, DeviceDecoder
    g = rng(2718)
    cfg = DecoderConfig(hidden=512, heads=4, kv_heads=2, head_dim=128, ffn=1024, epsilon=1e-6, rope_base=1e6,
                        max_tokens=64)
    vocab, n_layers, position, token = 300, 2, 37, 123
    qw, kvw = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim

    def quant(rows, cols, fmt, scale=0.05):
        return S.quantize_weights((g.standard_normal((rows, cols)) * scale).astype(np.float32), rows, cols, fmt)

    shapes = {"q": (qw, cfg.hidden, BQ.Q4_K), "k": (kvw, cfg.hidden, BQ.Q4_K), "v": (kvw, cfg.hidden, BQ.Q4_K),
              "o": (cfg.hidden, qw, BQ.Q4_K), "gate": (cfg.ffn, cfg.hidden, BQ.Q4_K),
              "up": (cfg.ffn, cfg.hidden, BQ.Q4_K), "down": (cfg.hidden, cfg.ffn, BQ.Q6_K)}
    host_layers, dev_layers, host_vecs, dev_vecs, buffers = [], [], [], [], []

    def dev_vec(a):
        p = context.alloc(a.nbytes)
        context.upload(p, a)
        buffers.append(p)
        return p

    for _ in range(n_layers):
        data = {n: quant(r, c, f) for n, (r, c, f) in shapes.items()}
        host_layers.append(data)
        dev_layers.append({n: context.create(d, S.QuantizedMatrixShape(*shapes[n])) for n, d in data.items()})
        vec = {"attn_norm": g.uniform(0.5, 1.5, cfg.hidden).astype(np.float32),
               "ffn_norm": g.uniform(0.5, 1.5, cfg.hidden).astype(np.float32),
               "q_bias": (g.standard_normal(qw) * 0.1).astype(np.float32),
               "k_bias": (g.standard_normal(kvw) * 0.1).astype(np.float32),
               "v_bias": (g.standard_normal(kvw) * 0.1).astype(np.float32)}
        host_vecs.append(vec)
        dev_vecs.append({k: dev_vec(v) for k, v in vec.items()})
    out_norm = g.uniform(0.5, 1.5, cfg.hidden).astype(np.float32)
    out_data = quant(vocab, cfg.hidden, BQ.Q6_K, 0.1)
    output = context.create(out_data, S.QuantizedMatrixShape(vocab, cfg.hidden, BQ.Q6_K))
    dec = DeviceDecoder(context, cfg, dev_layers, dev_vecs, dev_vec(out_norm), output, output)  # tied embedding
    # A random key/value prefix for positions < `position`, the same on both sides.
    prefix_k = [(g.standard_normal((cfg.max_tokens, kvw)) * 0.5).astype(np.float32) for _ in range(n_layers)]
    prefix_v = [(g.standard_normal((cfg.max_tokens, kvw)) * 0.5).astype(np.float32) for _ in range(n_layers)]
    for layer in range(n_layers):
        context.upload(dec.keys[layer], prefix_k[layer])
        context.upload(dec.values[layer], prefix_v[layer])

    def proj(data, rows, cols, fmt, x):
        return O.qk_matvec_quantized_avx2(data, rows, cols, int(fmt), O.q8k_quantize_row(x))

    row_bytes = out_data.size // vocab
    x = O.q_decode_row(out_data[token * row_bytes:(token + 1) * row_bytes], cfg.hidden, int(BQ.Q6_K))
    for layer in range(n_layers):
        d, vec = host_layers[layer], host_vecs[layer]
        normed = O.rms_norm(x, vec["attn_norm"], np.float32(cfg.epsilon))
        q = O.add(proj(d["q"], qw, cfg.hidden, BQ.Q4_K, normed), vec["q_bias"])
        k = O.add(proj(d["k"], kvw, cfg.hidden, BQ.Q4_K, normed), vec["k_bias"])
        v = O.add(proj(d["v"], kvw, cfg.hidden, BQ.Q4_K, normed), vec["v_bias"])
        q = O.rope_half(q, cfg.head_dim, position, cfg.rope_base, cfg.head_dim)
        k = O.rope_half(k, cfg.head_dim, position, cfg.rope_base, cfg.head_dim)
        keys, values = prefix_k[layer].copy(), prefix_v[layer].copy()
        keys[position], values[position] = k, v
        ctx_vec = O.grouped_attention(q, keys[:position + 1].reshape(-1), values[:position + 1].reshape(-1),
                                      cfg.heads, cfg.kv_heads, cfg.head_dim, position + 1)
        x = O.add(x, proj(d["o"], cfg.hidden, qw, BQ.Q4_K, ctx_vec))
        normed = O.rms_norm(x, vec["ffn_norm"], np.float32(cfg.epsilon))
        act = O.swiglu(proj(d["gate"], cfg.ffn, cfg.hidden, BQ.Q4_K, normed),
                       proj(d["up"], cfg.ffn, cfg.hidden, BQ.Q4_K, normed))
        x = O.add(x, proj(d["down"], cfg.hidden, cfg.ffn, BQ.Q6_K, act))
    expected = proj(out_data, vocab, cfg.hidden, BQ.Q6_K, O.rms_norm(x, out_norm, np.float32(cfg.epsilon)))

    dec.enqueue(token, position)
    eager = dec.read_logits()
    assert np.all(np.isfinite(eager))
    err = np.abs(eager.astype(np.float64) - expected)
    assert err.max() <= 1e-3 * np.abs(expected).max(), f"max err {err.max()} of {np.abs(expected).max()}"
    dec.enqueue(token, position, fused=False)  # the unfused operator sequence gives the same bits
    assert np.array_equal(dec.read_logits().view(np.uint32), eager.view(np.uint32))
    step = dec.capture(token, position)
    for replay in range(3):
        context.upload(dec.logits, np.zeros(vocab, np.float32))
        dec.enqueue(5, 40)  # eager work between replays: another token, a cache slot the step does not read
        step.execute()
        assert np.array_equal(dec.read_logits().view(np.uint32), eager.view(np.uint32)), replay
    # Folded: residual add + RmsNorm inside the projections' launches, eager and replayed.
    dec.enqueue(token, position, folded=True)
    assert np.array_equal(dec.read_logits().view(np.uint32), eager.view(np.uint32))
    folded = dec.capture(token, position, folded=True)
    for replay in range(3):
        context.upload(dec.logits, np.zeros(vocab, np.float32))
        dec.enqueue(7, 41, folded=True)  # eager work between replays
        folded.execute()
        assert np.array_equal(dec.read_logits().view(np.uint32), eager.view(np.uint32)), ("folded", replay)
    assert dec.launches_per_token(folded=True, position=position) == 3 + 6 * n_layers  # inputs inside the attention
    with pytest.raises(S.ArgumentException):
        dev_layers[0]["q"].dispose()  # held by the decoder's group
    with pytest.raises(S.InvalidOperationException):
        context.capture_end()          # nothing is being captured
    folded.dispose()
    step.dispose()
    dec.dispose()
    for layer in dev_layers:
        for m in layer.values():
            m.dispose()
    output.dispose()
    for p in buffers:
        context.free(p)
