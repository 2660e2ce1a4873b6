"""Pins the oracle (C restatement, oracle/dq8_oracle.c) without a GPU.

Each oracle function is checked against something other than itself:
  * the reference's own test vectors and known answers (int8.rs:172-297,
    tensor.rs:605-803, weights.rs:841-866), restated here as data/formulas;
  * an independent numpy restatement (oracle/oracle_np.py), bit for bit;
  * a pure-Python scalar emulation of binary32 arithmetic (each operation
    computed exactly in double and rounded to float32 -- exact for a single
    +, * of two float32 values);
  * closed forms (round-half-away ties, FLT_MIN floor, zero groups).
Planted mistakes (half-to-even rounding, a fused multiply-add, reversed group
order, a transposed weight row) are applied to the numpy restatement and must
fail these checks, so the checks can tell a wrong oracle from a right one.
"""
import struct

import numpy as np
import pytest

import dq8o
import oracle_np as onp

F32 = np.float32
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def f32(v: float) -> float:
    return struct.unpack("f", struct.pack("f", v))[0]


def py_scaled_dot(x, xs, w, ws):
    """Scalar emulation of Kernel::scaled_dot (int8.rs:53-61)."""
    s = 0.0
    for g in range(len(xs)):
        d = 0
        for k in range(64 * g, min(64 * g + 64, len(x))):
            d += int(x[k]) * int(np.int8(np.uint8(w[k]).view(np.int8)))
        p = f32(float(xs[g]) * float(ws[g]))
        t = f32(float(d) * p)
        s = f32(s + t)
    return s


def py_quantize_group(vals):
    """Scalar emulation of one group (tensor.rs:330-338)."""
    m = 0.0
    for v in vals:
        m = max(m, abs(float(v)))
    scale = 1.0 if m == 0.0 else max(f32(m / 127.0), float(FLT_MIN))
    out = []
    for v in vals:
        r = f32(float(v) / scale)
        q = np.sign(r) * np.floor(abs(r) + 0.5)
        out.append(int(min(max(q, -127.0), 127.0)))
    return f32(scale), out


# ----------------------------------------------------------- int8.rs tests


def test_dot_all_lengths_match_integer_reference():
    # int8.rs:177-190: lengths 0..=64, unaligned starts, -128 and 127 present
    for length in range(65):
        a = np.array([(i * 71 + 128) & 0xFF for i in range(length + 1)], np.uint8).view(np.int8)
        b = np.array([(i * 37 + 128) & 0xFF for i in range(length + 1)], np.uint8)
        expected = sum(int(a[i]) * int(b[i:i + 1].view(np.int8)[0]) for i in range(1, length + 1))
        assert dq8o.dot(a[1:], b[1:]) == expected


def test_dot_extremes_known_answers():
    # int8.rs:191-192
    assert dq8o.dot(np.full(64, -128, np.int8), np.full(64, 128, np.uint8)) == 1_048_576
    assert dq8o.dot(np.full(64, -128, np.int8), np.full(64, 127, np.uint8)) == -1_040_384


def _tile_case(width):
    groups = -(-width // 64)

    def bytes_(seed):
        return np.array([(i * 73 + seed * 151) % 256 for i in range(width)], np.uint8)

    def scales(seed):
        out = []
        for g in range(groups):
            k = (g + seed) % 5
            out.append(1e-30 if k == 0 else 3.5e6 if k == 1 else (k + seed / 7.0) / 113.0)
        return np.array(out, np.float32)

    xs = [bytes_(r).view(np.int8) for r in range(4)]
    ws = [bytes_(c) for c in range(4, 8)]
    x_scales = [scales(r) for r in range(4)]
    w_scales = [scales(c) for c in range(4, 8)]
    return xs, x_scales, ws, w_scales


@pytest.mark.parametrize("width", [64, 128, 192, 2048, 100, 1])
def test_scaled_dot_matches_scalar_emulation_on_tile_vectors(width):
    # int8.rs:195-237 data; every (row, column) pair against the scalar emulation
    xs, x_scales, ws, w_scales = _tile_case(width)
    for r in range(4):
        for c in range(4):
            got = dq8o.scaled_dot(xs[r], x_scales[r], ws[c], w_scales[c])
            want = py_scaled_dot(xs[r], x_scales[r], ws[c], w_scales[c])
            assert struct.pack("f", got) == struct.pack("f", want), (width, r, c)


def test_scaled_tile_extremes_known_answer():
    # int8.rs:238-263: every product (-128)(-128) or 127(-128); scales [1.0, 0.5]
    x = [np.full(128, -128, np.int8), np.full(128, 127, np.int8), np.full(128, -128, np.int8),
         np.zeros(128, np.int8)]
    w = [np.full(128, 128, np.uint8), np.full(128, 128, np.uint8), np.full(128, 127, np.uint8),
         np.full(128, 1, np.uint8)]
    s = np.array([1.0, 0.5], np.float32)
    assert dq8o.scaled_dot(x[0], s, w[0], s) == 64.0 * 16384.0 * 1.0 + 64.0 * 16384.0 * 0.25
    for r in range(4):
        for c in range(4):
            assert dq8o.scaled_dot(x[r], s, w[c], s) == np.float32(py_scaled_dot(x[r], s, w[c], s))


# --------------------------------------------------------- tensor.rs tests


@pytest.mark.parametrize("width", [1, 15, 16, 17, 63, 64, 65, 131])
@pytest.mark.parametrize("rows", [1, 19])
def test_integer_projection_matches_independent_fp64_reference(width, rows):
    # tensor.rs:605-662 (bias included)
    output = 31
    groups = -(-width // 64)
    x = np.array([0.0 if i < width else ((i * 43 % 255) - 127.0) / 8.0 for i in range(rows * width)],
                 np.float32).reshape(rows, width)
    values = np.array([(i * 71 + 128) & 0xFF for i in range(output * width)], np.uint8).reshape(output, width)
    scales = np.array([(i % 7 + 1) / 32.0 for i in range(output * groups)], np.float32).reshape(output, groups)
    bias = np.array([i / 16.0 for i in range(output)], np.float32)
    actual = dq8o.linear(x, values, scales, bias=bias)
    q, xs = dq8o.quantize_inputs(x)
    wdeq = values.view(np.int8).astype(np.float64) * np.repeat(scales.astype(np.float64), 64, axis=1)[:, :width]
    for column in range(output):
        for row in range(rows):
            exp = float(bias[column]) + sum(
                float(wdeq[column, k]) * float(q[row, k]) * float(xs[row, k // 64]) for k in range(width))
            assert abs(float(actual[row, column]) - exp) < 1e-3 + abs(exp) * 1e-6


@pytest.mark.parametrize("rows,width,output", [(1, 64, 4), (4, 64, 4), (5, 128, 6), (9, 192, 31), (67, 128, 8),
                                               (7, 100, 9)])
def test_projection_columns_match_per_output_scaled_dots(rows, width, output):
    # tensor.rs:664-732 without the LoRA adapter: columns == scaled_dot + bias, bitwise
    groups = -(-width // 64)
    x = np.array([((i * 43 % 255) - 127.0) / 9.0 for i in range(rows * width)], np.float32).reshape(rows, width)
    values = np.array([(i * 71 + 128) & 0xFF for i in range(output * width)], np.uint8).reshape(output, width)
    scales = np.array([(i % 7 + 1) / 32.0 for i in range(output * groups)], np.float32).reshape(output, groups)
    bias = np.array([i / 16.0 - 0.5 for i in range(output)], np.float32)
    q, xs = dq8o.quantize_inputs(x)
    cols = dq8o.linear_int8(q, xs, values, scales, bias=bias, threads=4)
    for column in range(output):
        for row in range(rows):
            want = np.float32(dq8o.scaled_dot(q[row], xs[row], values[column], scales[column]) + bias[column])
            assert cols[column, row].tobytes() == want.tobytes()


@pytest.mark.parametrize("rows,width", [(3, 100), (70, 1000), (40, 2048)])
def test_parallel_input_quantization_matches_serial(rows, width):
    # tensor.rs:734-766
    def val(i):
        k = i % 17
        return 0.0 if k == 0 else -1e-38 if k == 1 else ((i * 31 % 499) - 249.0) / k

    x = np.array([val(i) for i in range(rows * width)], np.float32).reshape(rows, width)
    a = dq8o.quantize_inputs(x, threads=1)
    b = dq8o.quantize_inputs(x, threads=4)
    assert np.array_equal(a[0], b[0])
    assert a[1].tobytes() == b[1].tobytes()
    assert a[1].shape == (rows, -(-width // 64))


def test_input_quantization_error_bound_zero_and_denormal_groups_and_nonfinite():
    # tensor.rs:768-803
    width = 131
    x = np.array([((i % 79) - 39.0) / 11.0 for i in range(width * 3)], np.float32)
    x[:64] = 0.0
    x[64:128] = np.array([1], np.uint32).view(np.float32)[0]
    x = x.reshape(3, width)
    q, s = dq8o.quantize_inputs(x)
    assert s.shape == (3, 3)
    assert s[0, 0] == 1.0  # zero group: scale 1.0 (tensor.rs:331-332)
    assert s[0, 1] == FLT_MIN  # denormal-only group: floor at f32::MIN_POSITIVE
    for row in range(3):
        for g in range(3):
            scale = s[row, g]
            assert np.isfinite(scale) and scale > 0
            for k in range(64 * g, min(64 * g + 64, width)):
                restored = np.float32(q[row, k]) * scale
                assert abs(float(restored) - float(x[row, k])) <= float(scale) / 2 + 1e-6
    for bad in (np.nan, np.inf, -np.inf):
        assert dq8o.quantize_inputs(np.array([[bad]], np.float32)) is None
        assert dq8o.linear(np.array([[bad]], np.float32), np.array([[1]], np.uint8),
                           np.array([[1.0]], np.float32)) is None


def test_weight_quantization_error_bound_partial_groups_and_zero_rows():
    # weights.rs:841-866 (8-bit bound 127)
    width = 131
    w = np.array([0.0 if i < width else ((i % 113) - 56.0) / 19.0 for i in range(width * 3)],
                 np.float32).reshape(3, width)
    values, scales = dq8o.quantize_weights(w)
    restored = values.view(np.int8).astype(np.float32) * np.repeat(scales, 64, axis=1)[:, :width]
    for r in range(3):
        for g in range(3):
            blk = slice(64 * g, min(64 * g + 64, width))
            m = np.abs(w[r, blk]).max()
            assert np.all(np.abs(w[r, blk] - restored[r, blk]) <= m / (2 * 127.0) + 1e-6)
    assert np.all(scales[0] == 1.0)


def test_benchmark_inputs_formula_projection():
    # tensor.rs:553-603 inputs (weights ((i*71 % 255) - 127) as u8, scales 1/127;
    # x = ((i*43 % 255) - 127) / 127) at a reduced width: oracle == numpy == scalar emulation
    width, output, rows = 256, 8, 3
    values = np.array([((i * 71 % 255) - 127) & 0xFF for i in range(width * output)], np.uint8).reshape(output, width)
    scales = np.full((output, width // 64), 1.0 / 127.0, np.float32)
    x = np.array([((i * 43 % 255) - 127.0) / 127.0 for i in range(rows * width)], np.float32).reshape(rows, width)
    got = dq8o.linear(x, values, scales)
    q, xs = dq8o.quantize_inputs(x)
    for r in range(rows):
        for c in range(output):
            assert np.float32(got[r, c]) == np.float32(py_scaled_dot(q[r], xs[r], values[c], scales[c]) + 0.0)


# ------------------------------------------------------------ closed forms


def test_quantize_closed_forms_round_half_away_and_floors():
    # A group whose absmax is 127 has scale exactly 1.0, so q = round(v) half away from zero.
    g = np.zeros(64, np.float32)
    g[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.49999]
    q, s = dq8o.quantize_inputs(g[None, :])
    assert s[0, 0] == 1.0
    assert list(q[0, :8]) == [127, 3, -3, 1, -1, 2, 127, -126]
    # Absmax below 127 * FLT_MIN: the scale floors at FLT_MIN and q = round(v / FLT_MIN).
    tiny = np.zeros(64, np.float32)
    tiny[0] = np.float32(100) * FLT_MIN
    tiny[1] = np.float32(-3.5) * FLT_MIN
    q, s = dq8o.quantize_inputs(tiny[None, :])
    assert s[0, 0] == FLT_MIN and q[0, 0] == 100 and q[0, 1] == -4
    # A scalar emulation of one group agrees on random data, including ties.
    rng = np.random.default_rng(7)
    for trial in range(50):
        vals = (rng.integers(-600, 600, size=64) / 4.0).astype(np.float32)  # many exact .5 quotients
        if trial % 2:
            vals = rng.standard_normal(64).astype(np.float32) * np.float32(10.0 ** rng.integers(-30, 30))
        q, s = dq8o.quantize_inputs(vals[None, :])
        scale, qs = py_quantize_group(vals)
        assert s[0, 0] == np.float32(scale) and list(q[0]) == qs


def test_linear_with_zero_rows_is_a_no_op():
    out = dq8o.linear(np.zeros((0, 64), np.float32), np.zeros((3, 64), np.uint8), np.ones((3, 1), np.float32))
    assert out.shape == (0, 3)


# ------------------------------------------------------ C == numpy, bitwise


def _random_case(rng, rows, width, output, outliers=False):
    x = rng.standard_normal((rows, width)).astype(np.float32)
    if outliers:
        ch = rng.choice(width, size=max(1, width // 100), replace=False)
        x[:, ch] *= np.float32(20.0)
    w = (rng.standard_normal((output, width)) * 0.02).astype(np.float32)
    return x, w


@pytest.mark.parametrize("rows,width,output", [(1, 1, 1), (3, 63, 5), (19, 64, 31), (7, 65, 9), (33, 131, 17),
                                               (24, 2048, 40), (5, 6144, 7)])
def test_c_oracle_matches_numpy_restatement_bitwise(rows, width, output):
    rng = np.random.default_rng(rows * 1000 + width)
    x, w = _random_case(rng, rows, width, output, outliers=width >= 100)
    cv, cs = dq8o.quantize_weights(w)
    nq, ns = onp.quantize(w)
    assert np.array_equal(cv.view(np.int8), nq) and cs.tobytes() == ns.tobytes()
    cq, cxs = dq8o.quantize_inputs(x, threads=4)
    nxq, nxs = onp.quantize_inputs(x)
    assert np.array_equal(cq, nxq) and cxs.tobytes() == nxs.tobytes()
    assert np.array_equal(dq8o.group_dots(cq, cv), onp.group_dots(nxq, cv))
    bias = rng.standard_normal(output).astype(np.float32)
    cols = dq8o.linear_int8(cq, cxs, cv, cs, bias=bias, threads=3)
    rows_np = onp.linear_rows(nxq, nxs, cv, cs, bias=bias)
    assert cols.T.tobytes() == np.ascontiguousarray(rows_np).tobytes()
    for ep in (0, 1, 2):
        prev = rng.standard_normal((rows, output)).astype(np.float32)
        c_out = dq8o.linear(x, cv, cs, bias=bias, result=prev, epilogue=ep, threads=2)
        n_out = onp.store(prev, rows_np, ep)
        assert c_out.tobytes() == np.ascontiguousarray(n_out).tobytes()


# ----------------------------------------------------------- planted faults


def _mutant_rescale(kind):
    def fn(dots, xs, ws, bias=None):
        rows, n, g = dots.shape
        s = np.zeros((rows, n), np.float32)
        order = range(g - 1, -1, -1) if kind == "reversed" else range(g)
        for gi in order:
            p = xs[:, gi][:, None] * ws[:, gi][None, :]
            if kind == "fma":
                s = (s.astype(np.float64) + dots[:, :, gi].astype(np.float64) * p.astype(np.float64)).astype(np.float32)
            else:
                s = s + dots[:, :, gi].astype(np.float32) * p
        return s
    return fn


@pytest.mark.parametrize("kind", ["reversed", "fma"])
def test_planted_rescale_faults_are_detected(kind):
    xs, x_scales, ws, w_scales = _tile_case(2048)
    q = np.stack(xs)
    w = np.stack(ws)
    dots = onp.group_dots(q, w)
    right = onp.rescale_sum(dots, np.stack(x_scales), np.stack(w_scales))
    wrong = _mutant_rescale(kind)(dots, np.stack(x_scales), np.stack(w_scales))
    emu = np.array([[py_scaled_dot(xs[r], x_scales[r], ws[c], w_scales[c]) for c in range(4)] for r in range(4)],
                   np.float32)
    assert right.tobytes() == emu.tobytes()
    assert wrong.tobytes() != emu.tobytes()


def test_planted_rounding_and_transpose_faults_are_detected():
    g = np.zeros(64, np.float32)
    g[:4] = [127.0, 2.5, -2.5, 0.5]
    half_even = np.clip(np.round(g), -127, 127).astype(np.int8)  # np.round is half-to-even
    q, _ = dq8o.quantize_inputs(g[None, :])
    assert not np.array_equal(half_even, q[0])
    # A transposed weight layout gives different dots on the tensor.rs:664 data.
    x = np.array([((i * 43 % 255) - 127.0) / 9.0 for i in range(5 * 128)], np.float32).reshape(5, 128)
    values = np.array([(i * 71 + 128) & 0xFF for i in range(6 * 128)], np.uint8).reshape(6, 128)
    qx, _ = dq8o.quantize_inputs(x)
    right = dq8o.group_dots(qx, values)
    wrong = onp.group_dots(qx, np.ascontiguousarray(values.reshape(128, 6).T))
    assert not np.array_equal(right, wrong)


# ------------------------------------------------------------ LoRA (FP32)

def py_dot_scores(a, b):
    """Scalar emulation of dot_scores (tensor.rs:6-25, x86-64): eight lanes of
    `lane += a * b`, summed in order from -0.0, then the tail one product at a time."""
    n = len(a)
    chunks = n // 8
    lanes = [0.0] * 8
    for c in range(chunks):
        for i in range(8):
            lanes[i] = f32(lanes[i] + f32(float(a[8 * c + i]) * float(b[8 * c + i])))
    s = -0.0
    for i in range(8):
        s = f32(s + lanes[i])
    for t in range(8 * chunks, n):
        s = f32(s + f32(float(a[t]) * float(b[t])))
    return s


def test_dot_scores_lane_structure_and_tail_order_known_answers():
    # Lane i holds elements i, i+8, ...: 1e8 and -1e8 in lane 0 cancel before
    # the lane sum adds lane 1's 1.0 -> 1.0.  A sequential sum would absorb the
    # 1.0 into 1e8 and return 0.0.
    a = np.zeros(16, np.float32); a[0], a[8], a[1] = 1e8, -1e8, 1.0
    assert dq8o.dot_scores(a, np.ones(16, np.float32)) == 1.0
    # The tail (elements past the last full chunk) is added after the lane sum:
    # (1 + 1e8) - 1e8 = 0.0 in binary32; tail-first order would give 1.0.
    a = np.zeros(10, np.float32); a[0], a[8], a[9] = 1.0, 1e8, -1e8
    assert dq8o.dot_scores(a, np.ones(10, np.float32)) == 0.0
    # Products are rounded before the add (no fused multiply-add): with
    # a = b = 1 + 2^-12, a*b = 1 + 2^-11 + 2^-24 rounds to 1 + 2^-11 (tie to
    # even), so lane + a*b - (1 + 2^-11) is exactly 0; an FMA would keep 2^-24.
    e = np.float32(1 + 2.0 ** -12)
    a = np.array([e] + [0] * 7 + [-1.0] + [0] * 7, np.float32)
    b = np.array([e] + [0] * 7 + [1 + 2.0 ** -11] + [0] * 7, np.float32)
    assert dq8o.dot_scores(a, b) == 0.0
    assert dq8o.dot_scores(np.zeros(0, np.float32), np.zeros(0, np.float32)) == 0.0


@pytest.mark.parametrize("length", list(range(0, 41)) + [63, 64, 65, 131, 2048])
def test_dot_scores_integer_vectors_are_exact(length):
    # Small integers: every partial sum is exact, so any grouping must give the
    # integer dot product (a dropped or doubled term fails).
    a = np.array([(i * 37 % 19) - 9 for i in range(length)], np.float32)
    b = np.array([(i * 11 % 13) - 6 for i in range(length)], np.float32)
    assert float(dq8o.dot_scores(a, b)) == float(sum(int(x) * int(y) for x, y in zip(a, b)))


@pytest.mark.parametrize("length", [0, 1, 7, 8, 9, 15, 16, 17, 40, 63, 64, 65, 131])
def test_dot_scores_matches_scalar_emulation_on_special_values(length):
    # The value mix of tensor.rs:806-829 (-0.0, 1e-30, -3.5e8 and fractions).
    def v(seed):
        out = []
        for i in range(length):
            k = (i + seed) % 11
            out.append(-0.0 if k == 0 else 1e-30 if k == 1 else -3.5e8 if k == 2
                       else ((i * 37 + seed * 101) % 997) / 61.0 - 8.0 + k / 7.0)
        return np.array(out, np.float32)
    a, b = v(1), v(2)
    got = dq8o.dot_scores(a, b)
    assert np.float32(got).tobytes() == np.float32(py_dot_scores(a, b)).tobytes()


def test_dot_scores_within_fp64_bound():
    rng = np.random.default_rng(7)
    for n in [16, 100, 2048]:
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = (n + 2) * 2.0 ** -24 * float(np.sum(np.abs(a.astype(np.float64) * b)))
        assert abs(float(dq8o.dot_scores(a, b)) - exact) <= bound


def test_lora_combine_known_answers():
    # rank 3 is tail-only: 1*1 + 2*1 + 3*1 = 6; 1 + 0.375 * (6 + 0.0) = 3.25
    assert dq8o.lora_combine(1.0, [1.0, 2.0, 3.0], [1.0, 1.0, 1.0], 0.375) == 3.25
    # + 0.0 turns a -0.0 delta into +0.0, so -0.0 + scale * delta is +0.0
    r = dq8o.lora_combine(-0.0, [-0.0], [1.0], 2.0)
    assert r == 0.0 and np.float32(r).tobytes() == np.float32(0.0).tobytes()


@pytest.mark.parametrize("rows,width,output", [(1, 64, 4), (4, 64, 4), (5, 128, 6), (9, 192, 31), (67, 128, 8),
                                               (7, 100, 9)])
def test_projection_with_adapter_matches_per_output_combine(rows, width, output):
    # tensor.rs:664-732 with its rank-3 adapter: the x86 plan of the oracle equals
    # scaled_dot + bias, then Adapter::combine, per output, bitwise.  The middle
    # product is the test's own `mid`, so it enters through an identity A.
    rank = 3
    groups = -(-width // 64)
    x = np.array([((i * 43 % 255) - 127.0) / 9.0 for i in range(rows * width)], np.float32).reshape(rows, width)
    values = np.array([(i * 71 + 128) & 0xFF for i in range(output * width)], np.uint8).reshape(output, width)
    scales = np.array([(i % 7 + 1) / 32.0 for i in range(output * groups)], np.float32).reshape(output, groups)
    bias = np.array([i / 16.0 - 0.5 for i in range(output)], np.float32)
    mid = np.array([(i % 9) / 4.0 - 1.0 for i in range(rows * rank)], np.float32).reshape(rows, rank)
    bw = np.array([(i % 7) / 8.0 for i in range(output * rank)], np.float32).reshape(output, rank)
    q, xs = dq8o.quantize_inputs(x)
    for column in range(output):
        for row in range(rows):
            base = np.float32(dq8o.scaled_dot(q[row], xs[row], values[column], scales[column]) + bias[column])
            want = dq8o.lora_combine(base, mid[row], bw[column], 0.375)
            # the same combine written out: base + scale * (dot_scores + 0.0)
            alt = np.float32(base + np.float32(np.float32(0.375) * np.float32(py_dot_scores(mid[row], bw[column]) + 0.0)))
            assert np.float32(want).tobytes() == alt.tobytes()


@pytest.mark.parametrize("rows", [1, 19, 67])
def test_fused_lora_matches_separate_projections(rows):
    # weights.rs:657-706: the fused plan equals base + scale * delta computed by
    # separate projections, for Write, Add and SwiGlu.
    width, output, rank, scale = 131, 31, 13, 0.375
    x = np.array([((i * 43 % 113) - 56.0) / 32.0 for i in range(rows * width)], np.float32).reshape(rows, width)

    def packed(count):  # bf16-valued weights, as the reference test packs them
        v = np.array([((i * 17 % 89) - 44.0) / 32.0 for i in range(count)], np.float32)
        return (v.view(np.uint32) & 0xFFFF0000).view(np.float32)
    wv, ws = dq8o.quantize_weights(packed(output * width).reshape(output, width))
    a = packed(rank * width).reshape(rank, width)
    b = packed(output * rank).reshape(output, rank)
    bias = np.array([i / 64.0 - 0.25 for i in range(output)], np.float32)
    base = dq8o.linear(x, wv, ws, bias=bias)
    mid = dq8o.linear_f32(x, a)
    delta = dq8o.linear_f32(mid, b)
    expected = (base + (np.float32(scale) * delta).astype(np.float32)).astype(np.float32)
    got = dq8o.linear_lora(x, wv, ws, a, b, scale, bias=bias, threads=4)
    assert got.tobytes() == expected.tobytes()
    original = np.array([i / 16.0 - 3.0 for i in range(rows * output)], np.float32).reshape(rows, output)
    add = dq8o.linear_lora(x, wv, ws, a, b, scale, bias=bias, result=original, epilogue=1)
    assert add.tobytes() == (original + expected).astype(np.float32).tobytes()
    sw = dq8o.linear_lora(x, wv, ws, a, b, scale, bias=bias, result=original, epilogue=2)
    want = np.array([dq8o.silu(o) * e for o, e in zip(original.ravel(), expected.ravel())], np.float32)
    assert sw.ravel().tobytes() == want.tobytes()


def test_lora_mid_is_linear_of_a_and_scale_zero_leaves_base():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 200)).astype(np.float32)
    a = rng.standard_normal((16, 200)).astype(np.float32)
    mid = dq8o.lora_mid(x, a)
    for r in range(5):
        for j in range(16):
            assert np.float32(mid[r, j]).tobytes() == np.float32(py_dot_scores(x[r], a[j]) + 0.0).tobytes()
    wv, ws = dq8o.quantize_weights(rng.standard_normal((9, 200)).astype(np.float32) * 0.02)
    b = rng.standard_normal((9, 16)).astype(np.float32)
    base = dq8o.linear(x, wv, ws)
    assert dq8o.linear_lora(x, wv, ws, a, b, 0.0).tobytes() == (base + np.float32(0.0)).astype(np.float32).tobytes()


def test_planted_dot_scores_faults_are_detected():
    # Sequential summation or a fused multiply-add must fail the known answers above.
    def sequential(a, b):
        s = 0.0
        for x, y in zip(a, b):
            s = f32(s + f32(float(x) * float(y)))
        return s
    a = np.zeros(16, np.float32); a[0], a[8], a[1] = 1e8, -1e8, 1.0
    assert sequential(a, np.ones(16, np.float32)) != 1.0
    e = 1 + 2.0 ** -12
    fused = f32(e * e - (1 + 2.0 ** -11))  # what an FMA would leave in lane 0
    assert fused != 0.0


# ---------------------------------------------------------------- silu / expf
# qwen.rs:194-199 computes silu with f32::exp, i.e. the host libm expf (glibc
# 2.35 on x86-64).  The kernels restate glibc's algorithm; these tests pin the
# restatement (dq8o_expf_restated, the same steps as the kernels) to libm.

def _libm_expf():
    import ctypes
    import ctypes.util
    m = ctypes.CDLL(ctypes.util.find_library("m"))
    m.expf.argtypes = [ctypes.c_float]
    m.expf.restype = ctypes.c_float
    return m.expf


def _exp2_frac_table():
    """2^(j/32), j = 0..31, from 50-digit decimal arithmetic rounded to double."""
    from decimal import Decimal, localcontext
    with localcontext() as c:
        c.prec = 50
        return [float(Decimal(2) ** (Decimal(j) / Decimal(32))) for j in range(32)]


_EXP2_FRAC = _exp2_frac_table()


def _py_expf_unfused(x):
    """glibc's expf steps in plain double arithmetic, without its fused
    multiply-adds (the x86-64 build without FMA3)."""
    tab = _EXP2_FRAC
    inv = float.fromhex("0x1.71547652b82fep+0") * 32
    shift = float.fromhex("0x1.8p+52")
    c0 = float.fromhex("0x1.c6af84b912394p-5") / 32 ** 3
    c1 = float.fromhex("0x1.ebfce50fac4f3p-3") / 32 ** 2
    c2 = float.fromhex("0x1.62e42ff0c52d6p-1") / 32
    z = inv * x
    kd = z + shift
    ki = struct.unpack("<Q", struct.pack("<d", kd))[0]
    kd -= shift
    r = z - kd
    j = ki & 31
    sb = (struct.unpack("<Q", struct.pack("<d", tab[j]))[0] + ((ki - j) << 47)) % (1 << 64)
    s = struct.unpack("<d", struct.pack("<Q", sb))[0]
    y = (c0 * r + c1) * (r * r) + (c2 * r + 1.0)
    return f32(y * s)


def test_restated_expf_matches_libm_on_every_binary32_input():
    assert dq8o.expf_mismatches(0, 1 << 32, threads=8) == 0


def test_expf_known_answers_and_special_values():
    expf = _libm_expf()
    assert dq8o.expf_restated(0.0) == 1.0 and dq8o.expf_restated(-0.0) == 1.0
    assert dq8o.expf_restated(1.0) == F32(float.fromhex("0x1.5bf0a8p+1"))  # e to nearest
    assert dq8o.expf_restated(float("inf")) == np.inf and dq8o.expf_restated(-np.inf) == 0.0
    assert np.isnan(dq8o.expf_restated(float("nan")))
    assert dq8o.expf_restated(89.0) == np.inf and dq8o.expf_restated(-104.0) == 0.0
    # smallest subnormal region and the largest finite result
    for h in ("-0x1.9fe368p+6", "-0x1.9fe36ap+6", "0x1.62e42ep+6", "0x1.62e430p+6"):
        x = f32(float.fromhex(h))
        assert dq8o.expf_restated(x).tobytes() == F32(expf(x)).tobytes()


def test_unfused_expf_agrees_on_ordinary_inputs_but_not_on_glibc_fma_cases():
    # The plain-double form of the same algorithm agrees with libm on random
    # inputs (the constants and table are right) but not where glibc's fused
    # multiply-adds decide the rounding: the restatement must be the fused one.
    expf = _libm_expf()
    rng = np.random.default_rng(3)
    for x in rng.uniform(-80, 80, 2000).astype(np.float32):
        assert _py_expf_unfused(float(x)) == F32(expf(float(x)))
    for h in ("0x1.04845ep+5", "-0x1.f8cbb2p+5"):
        x = f32(float.fromhex(h))
        assert _py_expf_unfused(x) != F32(expf(x))
        assert dq8o.expf_restated(x) == F32(expf(x))


def test_double_exp_rounded_once_is_not_libm_expf():
    # A correctly rounded exp differs from glibc's expf (on 170648 of the
    # 2239889408 inputs in (-104, 89)); one of them:
    import math
    expf = _libm_expf()
    x = f32(float.fromhex("0x1.fefe02p-16"))
    assert F32(math.exp(x)) != F32(expf(x))
    assert dq8o.expf_restated(x) == F32(expf(x))


def test_silu_n_matches_scalar_silu():
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.standard_normal(70000).astype(np.float32) * 20,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 200.0, -200.0], np.float32)])
    y = dq8o.silu_n(x, threads=4)
    want = np.array([dq8o.silu(float(v)) for v in x], np.float32)
    assert y.tobytes() == want.tobytes()
    assert dq8o.silu(0.0) == 0.0 and dq8o.silu(-200.0) == 0.0 and dq8o.silu(200.0) == 200.0


# ------------------------------------------------------ FP32 fallback path
# Projection::apply_quantized takes columns_tiled (tensor.rs:206-269) when
# QuantizedInputs::new returns None: dot_scores over the dequantized weights
# (Data::row, weights.rs:47-78).

def test_dequantize_known_answers_and_bound():
    w = np.array([[1, 255, 127, 129, 0, 128]], np.uint8)  # 1, -1, 127, -127, 0, -128
    ws = np.array([[0.25]], np.float32)
    assert dq8o.dequantize_weights(w, ws).tolist() == [[0.25, -0.25, 31.75, -31.75, 0.0, -32.0]]
    rng = np.random.default_rng(17)
    x = (rng.standard_normal((9, 200)) * 3).astype(np.float32)
    v, s = dq8o.quantize_weights(x)
    d = dq8o.dequantize_weights(v, s)
    for g in range(4):
        blk = slice(64 * g, min(64 * g + 64, 200))
        assert np.all(np.abs(d[:, blk] - x[:, blk]) <= s[:, g:g + 1] / 2 * (1 + 1e-6))


def _fallback_case(rng, rows, width, outputs, rank=0):
    x = (rng.standard_normal((rows, width)) * 2).astype(np.float32)
    v, s = dq8o.quantize_weights((rng.standard_normal((outputs, width)) * 0.1).astype(np.float32))
    bias = rng.standard_normal(outputs).astype(np.float32)
    a = b = None
    if rank:
        a = (rng.standard_normal((rank, width)) * 0.1).astype(np.float32)
        b = (rng.standard_normal((outputs, rank)) * 0.1).astype(np.float32)
    return x, v, s, bias, a, b


@pytest.mark.parametrize("rank", [0, 3, 11])
def test_fallback_outputs_are_dot_scores_of_dequantized_rows(rank):
    rng = np.random.default_rng(rank + 5)
    rows, width, outputs = 4, 75, 6
    x, v, s, bias, a, b = _fallback_case(rng, rows, width, outputs, rank)
    x[1, 30] = np.nan  # the whole projection takes the FP32 path (tensor.rs:318-320)
    got, fp32 = dq8o.apply(x, v, s, bias=bias, a=a, b=b, scale=0.5)
    assert fp32
    d = dq8o.dequantize_weights(v, s)
    for r in range(rows):
        for n in range(outputs):
            want = f32(py_dot_scores(x[r], d[n]) + float(bias[n]))
            if rank:
                mid = [f32(py_dot_scores(x[r], a[j]) + 0.0) for j in range(rank)]
                delta = f32(py_dot_scores(mid, b[n]) + 0.0)
                want = f32(want + f32(0.5 * delta))
            if r == 1:
                assert np.isnan(got[r, n])
            else:
                assert got[r, n] == np.float32(want), (r, n)


def test_finite_inputs_take_the_int8_path_and_the_paths_differ():
    rng = np.random.default_rng(8)
    x, v, s, bias, _, _ = _fallback_case(rng, 5, 130, 7)
    got, fp32 = dq8o.apply(x, v, s, bias=bias)
    assert not fp32
    assert got.tobytes() == dq8o.linear(x, v, s, bias=bias).tobytes()
    # the FP32 path on the same finite input gives different bits, so a device
    # result from the wrong path cannot pass a bitwise check
    d = dq8o.dequantize_weights(v, s)
    fp = np.array([[py_dot_scores(x[r], d[n]) + float(bias[n]) for n in range(7)] for r in range(5)], np.float32)
    assert fp.tobytes() != got.tobytes()


def test_fallback_epilogues_store_like_write_columns():
    rng = np.random.default_rng(9)
    x, v, s, bias, _, _ = _fallback_case(rng, 3, 64, 5)
    x[2, 0] = np.inf
    base = rng.standard_normal((3, 5)).astype(np.float32)
    w, _ = dq8o.apply(x, v, s, bias=bias)
    add, _ = dq8o.apply(x, v, s, bias=bias, result=base, epilogue=1)
    sw, _ = dq8o.apply(x, v, s, bias=bias, result=base, epilogue=2)
    with np.errstate(invalid="ignore"):
        assert np.array_equal(add, (base + w).astype(np.float32), equal_nan=True)
    want = np.array([dq8o.silu(o) * e for o, e in zip(base.ravel(), w.ravel())], np.float32).reshape(3, 5)
    assert np.array_equal(sw, want, equal_nan=True)
