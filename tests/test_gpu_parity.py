"""GPU parity: the HIP path through the C ABI against the oracle, bit for bit.

Quantized int8 tensors, scale bit patterns and per-group i32 dots must be
identical; fp32 outputs of Write/Add/SwiGlu must be identical (the stated
tolerance is max relative error 1e-6; the kernels meet it exactly).  SwiGlu's
silu runs glibc's expf algorithm on the device; the oracle calls libm expf.
"""
import ctypes

import numpy as np
import pytest
import torch

import dq8
import dq8o

pytestmark = pytest.mark.gpu

FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def make_x(rng, rows, width, kind="normal"):
    x = rng.standard_normal((rows, width)).astype(np.float32)
    if kind == "outliers":
        ch = rng.choice(width, size=max(1, width // 100), replace=False)
        x[:, ch] *= np.float32(20.0)
    elif kind == "student":
        z = rng.standard_normal((rows, width))
        chi = rng.chisquare(3, size=(rows, width))
        x = (z / np.sqrt(chi / 3)).astype(np.float32)
    elif kind == "edge":
        x[:, :64] = 0.0  # zero group
        if width > 64:
            x[:, 64:min(128, width)] = np.array([1], np.uint32).view(np.float32)[0]  # denormal-only group
        if width > 130:
            x[:, 128] = 127.0 * FLT_MIN  # tiny group
        x[0, -1] = 2.5  # exact half quotients in some groups
    return x


def tile_rows(rng, m, extra=8, tile=64):
    """Oracle rows of a full-size check: one random row in every 64-row tile,
    the first and last rows, and a few more at random."""
    rows = [int(rng.integers(t, min(t + tile, m))) for t in range(0, m, tile)]
    return np.unique(np.r_[rows, 0, m - 1, rng.choice(m, size=extra, replace=False)])


def make_w(rng, n, k):
    return (rng.standard_normal((n, k)) * 0.02).astype(np.float32)


# ------------------------------------------------------------ quantization

QUANT_SHAPES = [(1, 1), (3, 63), (2, 64), (5, 65), (7, 100), (4, 131), (19, 255), (3, 256), (9, 257), (128, 2048),
                (24, 6144), (33, 4097)]


@pytest.mark.parametrize("rows,width", QUANT_SHAPES)
@pytest.mark.parametrize("kind", ["normal", "outliers", "edge", "student"])
def test_quantize_bit_exact(ctx, rows, width, kind):
    rng = np.random.default_rng(rows * 7919 + width)
    x = make_x(rng, rows, width, kind)
    q, s = ctx.quantize(dev(x))
    want_q, want_s = dq8o.quantize_inputs(x)
    assert np.array_equal(host(q), want_q)
    assert bits_equal(host(s), want_s)


# Widths that are a multiple of 256 run on the chunk-walking quantizer: the
# sizes below give its waves one chunk, and several with a ragged last round.
@pytest.mark.parametrize("rows,width", [(2048, 2048), (1543, 2304), (5, 512)])
@pytest.mark.parametrize("kind", ["normal", "edge", "student"])
def test_quantize_chunk_walk_bit_exact(ctx, rows, width, kind):
    rng = np.random.default_rng(rows + width * 3)
    x = make_x(rng, rows, width, kind)
    q, s = ctx.quantize(dev(x))
    want_q, want_s = dq8o.quantize_inputs(x, threads=8)
    assert np.array_equal(host(q), want_q)
    assert bits_equal(host(s), want_s)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("where", [(0, 0), (2, 511), (1537, 100)])
def test_quantize_chunk_walk_reports_nonfinite(ctx, bad, where):
    rows = 1600 if where[0] >= 3 else 3
    x = np.ones((rows, 512), np.float32)
    x[where] = bad
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.quantize(dev(x), nonfinite=flag)
    assert int(host(flag)[0]) == 1
    with pytest.raises(dq8.NonFinite):
        ctx.quantize(dev(x))


def test_quantize_values_next_to_half_integer_boundaries(ctx):
    # Every element of a group is (k + 0.5) * scale, rounded, and moved by up
    # to 2 ulp either way, for random k in -127..126: the quotient by the scale
    # lands on or next to a rounding boundary, where an approximate quotient
    # could round the other way.  Element 0 of each group sets the scale.
    rng = np.random.default_rng(55)
    rows = []
    for _ in range(64):
        m = np.float32(rng.uniform(0.1, 100.0) * 2.0 ** int(rng.integers(-20, 20)))
        scale = np.float32(m / np.float32(127.0))
        ks = rng.integers(-127, 127, size=63)
        base = ((ks + 0.5) * np.float64(scale)).astype(np.float32)
        vals = (base.view(np.int32) + rng.integers(-2, 3, size=63).astype(np.int32)).view(np.float32)
        rows.append(np.concatenate([[m], np.clip(vals, -m, m)]).astype(np.float32))
    x = np.stack(rows).reshape(16, 256)
    q, s = ctx.quantize(dev(x))
    qh, sh = dq8o.quantize_inputs(x)
    assert np.array_equal(host(q), qh) and bits_equal(host(s), sh)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_quantize_nonfinite_is_reported(ctx, bad):
    x = np.ones((3, 70), np.float32)
    x[2, 69] = bad
    with pytest.raises(dq8.NonFinite):
        ctx.quantize(dev(x))
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.quantize(dev(x), nonfinite=flag)
    assert int(host(flag)[0]) == 1
    flag.zero_()
    ctx.quantize(dev(np.ones((3, 70), np.float32)), nonfinite=flag)
    assert int(host(flag)[0]) == 0


# ----------------------------------------------------------------- weights

WEIGHT_SHAPES = [(1, 1), (31, 131), (64, 64), (65, 100), (100, 2048), (33, 6144)]


@pytest.mark.parametrize("n,k", WEIGHT_SHAPES)
def test_weights_from_f32_bit_exact_and_export(ctx, n, k):
    rng = np.random.default_rng(n * 31 + k)
    w = make_w(rng, n, k)
    w[0, :min(64, k)] = 0.0
    h = ctx.weights_from_f32(dev(w))
    values, scales = h.export()
    want_v, want_s = dq8o.quantize_weights(w)
    assert np.array_equal(host(values), want_v)
    assert bits_equal(host(scales), want_s)


def test_linear_rejects_grids_out_of_range(ctx):
    # m > 2^30 rows, or more than 2^39 outputs in one item: DQ8_ERR_SHAPE before
    # anything is read or launched (the pointers are stand-ins never dereferenced)
    rng = np.random.default_rng(3)
    h = ctx.weights_from_f32(dev(make_w(rng, 2048, 64)))
    lib = dq8.lib()
    fake = 256
    for m in ((1 << 28) + 1, (1 << 30) + 1):
        assert lib.dq8_linear(ctx.handle, h.handle, fake, fake, m, None, fake, 0, 0, None) == dq8.ERR_SHAPE
    torch.cuda.synchronize()


def test_weights_reject_shapes_beyond_the_offset_bounds(ctx):
    # k > 2^26, or a scale table of 4 GiB or more: DQ8_ERR_SHAPE from every
    # weight constructor before anything is read (stand-in pointers)
    lib = dq8.lib()
    fake = 256
    for n, k in ((1, (1 << 26) + 64), (1 << 26, 1 << 10)):
        out = ctypes.c_void_p()
        assert lib.dq8_weights_from_f32(ctx.handle, fake, n, k, None, ctypes.byref(out)) == dq8.ERR_SHAPE
        assert lib.dq8_weights_from_quantized(ctx.handle, fake, fake, n, k, None, ctypes.byref(out)) == dq8.ERR_SHAPE
        assert out.value is None
    torch.cuda.synchronize()


@pytest.mark.parametrize("n,k", WEIGHT_SHAPES)
def test_weights_from_quantized_round_trip(ctx, n, k):
    rng = np.random.default_rng(n + 17 * k)
    values = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    scales = rng.random((n, -(-k // 64))).astype(np.float32)
    h = ctx.weights_from_quantized(dev(values), dev(scales))
    v2, s2 = h.export()
    assert np.array_equal(host(v2), values)
    assert bits_equal(host(s2), scales)


# -------------------------------------------------------------- group dots

DOT_SHAPES = [(1, 64, 1), (5, 100, 9), (24, 2048, 33), (32, 131, 70), (33, 64, 31), (67, 192, 65), (130, 257, 40),
              (24, 6144, 20), (17, 2371, 33), (9, 4160, 18), (48, 2048, 40), (61, 4160, 17)]


@pytest.mark.parametrize("m,k,n", DOT_SHAPES)
def test_group_dots_bit_exact(ctx, m, k, n):
    rng = np.random.default_rng(m * 1009 + k * 7 + n)
    values = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    values[0, :] = 128  # -128 weights
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    q[0, :] = -127
    h = ctx.weights_from_quantized(dev(values), dev(np.ones((n, -(-k // 64)), np.float32)))
    got = host(ctx.group_dots(h, dev(q)))
    assert np.array_equal(got, dq8o.group_dots(q, values))


def test_group_dots_extremes(ctx):
    # int8.rs:191-192 through the MFMA path: -128 * 128 and -128 * 127 sums
    q = np.full((2, 64), -128, np.int8)
    values = np.stack([np.full(64, 128, np.uint8), np.full(64, 127, np.uint8)])
    h = ctx.weights_from_quantized(dev(values), dev(np.ones((2, 1), np.float32)))
    got = host(ctx.group_dots(h, dev(q)))
    assert got[0, 0, 0] == 1_048_576 and got[0, 1, 0] == -1_040_384


# ---------------------------------------------------------------- projection

# Skinny (M <= 32) cases cover both row-tile counts (M <= 16, M <= 32), short K
# (G <= 32, odd G, G = 1) and long K (G > 32: 4-way split groups, partial last
# step, several x-scale chunks, K % 64 != 0).  Long K at 17-32 rows pairs a
# strip's two row-tile blocks 8 apart in runs of 8 strips: 13 and 17 strips
# (200 and 264 outputs) give whole runs followed by a shorter last run.
LINEAR_SHAPES = [(1, 1, 1), (1, 64, 4), (4, 64, 4), (5, 128, 6), (9, 192, 31), (24, 2048, 100), (32, 131, 70),
                 (33, 100, 9), (67, 128, 8), (64, 2048, 64), (128, 2048, 130), (200, 65, 17), (7, 6144, 33),
                 (24, 6144, 70), (17, 2371, 50), (32, 4096, 40), (16, 2112, 33), (2, 2113, 17), (48, 2048, 96),
                 (40, 6144, 50), (63, 131, 33), (34, 4160, 20), (96, 2048, 64), (24, 6144, 200), (17, 4096, 264)]


@pytest.mark.parametrize("m,k,n", LINEAR_SHAPES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_rows_write_bit_exact(ctx, m, k, n, with_bias):
    rng = np.random.default_rng(m * 131 + k * 3 + n)
    x = make_x(rng, m, k, "outliers" if k >= 100 else "normal")
    w = make_w(rng, n, k)
    bias = rng.standard_normal(n).astype(np.float32) if with_bias else None
    wv, ws = dq8o.quantize_weights(w)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    out = ctx.linear(h, q, s, bias=None if bias is None else dev(bias))
    want = dq8o.linear(x, wv, ws, bias=bias, threads=4)
    assert bits_equal(host(out), want)


@pytest.mark.parametrize("m,k,n", [(5, 128, 6), (24, 2048, 100), (67, 128, 8), (130, 257, 40), (48, 2048, 40)])
def test_linear_columns_layout_bit_exact(ctx, m, k, n):
    rng = np.random.default_rng(m + k + n)
    x = make_x(rng, m, k)
    w = make_w(rng, n, k)
    wv, ws = dq8o.quantize_weights(w)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    cols = ctx.linear(h, q, s, layout=dq8.COLUMNS)
    qh, sh = dq8o.quantize_inputs(x)
    assert bits_equal(host(cols), dq8o.linear_int8(qh, sh, wv, ws, threads=4))


@pytest.mark.parametrize("m,k,n", [(3, 131, 31), (24, 2048, 64), (67, 192, 65), (45, 6144, 40)])
def test_linear_add_epilogue_bit_exact(ctx, m, k, n):
    rng = np.random.default_rng(3 * m + k + n)
    x = make_x(rng, m, k)
    w = make_w(rng, n, k)
    prev = rng.standard_normal((m, n)).astype(np.float32)
    wv, ws = dq8o.quantize_weights(w)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    out = dev(prev)
    ctx.linear(h, q, s, out=out, epilogue=dq8.ADD)
    assert bits_equal(host(out), dq8o.linear(x, wv, ws, result=prev, epilogue=1, threads=4))


@pytest.mark.parametrize("m,k,n,ep", [(130, 16384, 200, dq8.WRITE), (300, 12288, 130, dq8.ADD),
                                      (24, 16384, 100, dq8.WRITE), (20, 32768, 48, dq8.ADD), (9, 20480, 40, dq8.WRITE)])
def test_linear_long_k_bit_exact(ctx, m, k, n, ep):
    # K far beyond the model's 6144 (192 to 512 groups): the wide kernel's operand
    # rings and x-scale chunk buffers, and the skinny long-K ring and in-order
    # hand-off, wrap many times; the group offsets reach the largest values tested
    rng = np.random.default_rng(m + k + 7 * n)
    x = make_x(rng, m, k, "student")
    w = make_w(rng, n, k)
    wv, ws = dq8o.quantize_weights(w)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    if ep == dq8.ADD:
        prev = rng.standard_normal((m, n)).astype(np.float32)
        out = dev(prev)
        ctx.linear(h, q, s, out=out, epilogue=dq8.ADD)
        want = dq8o.linear(x, wv, ws, result=prev, epilogue=1, threads=4)
    else:
        out = ctx.linear(h, q, s)
        want = dq8o.linear(x, wv, ws, threads=4)
    assert bits_equal(host(out), want)


@pytest.mark.parametrize("m,k,n", [(3, 131, 31), (24, 2048, 64), (67, 192, 65), (50, 2048, 70)])
def test_linear_swiglu_epilogue(ctx, m, k, n):
    rng = np.random.default_rng(5 * m + k + n)
    x = make_x(rng, m, k)
    w = make_w(rng, n, k)
    gate = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    wv, ws = dq8o.quantize_weights(w)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    out = dev(gate)
    ctx.linear(h, q, s, out=out, epilogue=dq8.SWIGLU)
    got = host(out)
    want = dq8o.linear(x, wv, ws, result=gate, epilogue=2, threads=4)
    assert bits_equal(got, want)
    print(f"swiglu bit-identical fraction {np.mean(got == want):.6f}")


# Inputs where glibc's fused expf steps decide the rounding, where a correctly
# rounded exp differs from glibc's, the overflow/underflow edges of exp(-x),
# signed zeros, subnormals, infinities and NaN.
SILU_EDGES = ["-0x1.04845ep+5", "0x1.f8cbb2p+5", "-0x1.fefe02p-16", "0x1.9fe368p+6", "0x1.9fe36ap+6",
              "-0x1.62e42ep+6", "-0x1.62e430p+6", "0x1.a0p+6", "-0x1.64p+6", "0x0p+0", "-0x0p+0", "0x1p-149",
              "-0x1p-149", "0x1.fffffcp-127", "inf", "-inf", "nan", "0x1.fffffep+127", "-0x1.fffffep+127"]


@pytest.mark.parametrize("m,seed", [(64, 1), (24, 2), (8, 3)])
def test_swiglu_silu_matches_libm_over_a_bit_pattern_sweep(ctx, m, seed):
    # Zero weights and a bias of 1 make every stored value silu(old) * 1, so
    # the epilogue's silu is compared with the oracle's (libm expf) on 2^17
    # columns of pseudo-random bit patterns per row plus the edge cases above.
    n = 1 << 17
    i = np.arange(m * n, dtype=np.uint64)
    bits = ((i * np.uint64(2654435761 + 2 * seed)) + np.uint64(seed * 977)) & np.uint64(0xFFFFFFFF)
    gate = bits.astype(np.uint32).view(np.float32)
    gate[:len(SILU_EDGES)] = [float.fromhex(h) if "x" in h else float(h) for h in SILU_EDGES]
    gate = gate.reshape(m, n)
    wv, ws = dq8o.quantize_weights(np.zeros((n, 64), np.float32))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(np.ones((m, 64), np.float32)))
    out = dev(gate)
    ctx.linear(h, q, s, out=out, bias=dev(np.ones(n, np.float32)), epilogue=dq8.SWIGLU)
    got = host(out)
    want = dq8o.silu_n(gate, threads=8)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert got[~nan].tobytes() == want[~nan].tobytes()


def test_linear_f32in_and_nonfinite_fallback(ctx):
    rng = np.random.default_rng(11)
    x = make_x(rng, 40, 300)
    w = make_w(rng, 50, 300)
    wv, ws = dq8o.quantize_weights(w)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    assert bits_equal(host(ctx.linear_f32in(h, dev(x))), dq8o.linear(x, wv, ws, threads=4))
    x[3, 7] = np.nan
    sentinel = dev(np.full((40, 50), 7.0, np.float32))
    with pytest.raises(dq8.NonFinite):
        ctx.linear_f32in(h, dev(x), out=sentinel)
    assert np.all(host(sentinel) == 7.0)  # left untouched for the caller's FP32 path


def test_reference_fp64_case_through_gpu(ctx):
    # tensor.rs:605-662 vectors (first row all zeros, distinct group scales, biases)
    for width in (1, 15, 16, 17, 63, 64, 65, 131):
        for rows in (1, 19):
            output = 31
            groups = -(-width // 64)
            x = np.array([0.0 if i < width else ((i * 43 % 255) - 127.0) / 8.0 for i in range(rows * width)],
                         np.float32).reshape(rows, width)
            values = np.array([(i * 71 + 128) & 0xFF for i in range(output * width)], np.uint8).reshape(output, width)
            scales = np.array([(i % 7 + 1) / 32.0 for i in range(output * groups)], np.float32).reshape(output, groups)
            bias = np.array([i / 16.0 for i in range(output)], np.float32)
            h = ctx.weights_from_quantized(dev(values), dev(scales))
            out = ctx.linear_f32in(h, dev(x), bias=dev(bias))
            assert bits_equal(host(out), dq8o.linear(x, values, scales, bias=bias)), (width, rows)


def test_linear_batch_mixed_kinds_matches_single_calls(ctx):
    rng = np.random.default_rng(99)
    items, wants = [], []
    for (m, k, n) in [(24, 2048, 96), (24, 2048, 40), (70, 256, 64), (5, 100, 9), (130, 131, 33)]:
        x = make_x(rng, m, k)
        w = make_w(rng, n, k)
        wv, ws = dq8o.quantize_weights(w)
        h = ctx.weights_from_quantized(dev(wv), dev(ws))
        q, s = ctx.quantize(dev(x))
        out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        items.append(dq8.Item(h, q, s, out))
        wants.append(dq8o.linear(x, wv, ws, threads=4))
    ctx.linear_batch(items)
    for it, want in zip(items, wants):
        assert bits_equal(host(it.out), want)


def test_linear_batch_question_layer_set(ctx):
    # One continuation question (M=24) against a scaled-down layer set: short-K
    # and long-K skinny projections in one grouped launch, with bias and epilogues.
    rng = np.random.default_rng(24)
    m = 24
    items, wants = [], []
    for (k, n, ep) in [(256, 96, dq8.WRITE), (256, 40, dq8.WRITE), (256, 200, dq8.WRITE), (2048, 64, dq8.WRITE),
                       (2048, 96, dq8.SWIGLU), (6144, 64, dq8.ADD), (2240, 33, dq8.WRITE)]:
        x = make_x(rng, m, k)
        w = make_w(rng, n, k)
        bias = rng.standard_normal(n).astype(np.float32)
        wv, ws = dq8o.quantize_weights(w)
        h = ctx.weights_from_quantized(dev(wv), dev(ws))
        q, s = ctx.quantize(dev(x))
        base = rng.standard_normal((m, n)).astype(np.float32)
        out = dev(base.copy())
        items.append(dq8.Item(h, q, s, out, bias=dev(bias), epilogue=ep))
        wants.append(dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=4))
    ctx.linear_batch(items)
    for it, want in zip(items, wants):
        assert bits_equal(host(it.out), want)


# A question's projections at full size: q, k, v, o, GDN in/out, FFN gate, up
# (SwiGlu onto gate's output) and down (Add).  About 930 one-wave strips, so the
# grouped launch keeps the short-K skinny path (small launches take the 4-wave
# path); 9 rows take the 16-row kernel, 24 the 32-row one.
FULL_LAYER = [("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048), ("gdn_in", 8224, 2048),
              ("gdn_out", 2048, 2048), ("gate", 6144, 2048), ("up", 6144, 2048), ("down", 2048, 6144)]


@pytest.mark.parametrize("m", [24, 9])
def test_linear_batch_full_layer_set(ctx, m):
    rng = np.random.default_rng(m + 1000)
    weights = {}
    for name, n, k in FULL_LAYER:
        wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
        weights[name] = (wv, ws, ctx.weights_from_quantized(dev(wv), dev(ws)))
    x = make_x(rng, m, 2048, kind="student")
    xd = make_x(rng, m, 6144)
    q, s = ctx.quantize(dev(x))
    qd, sd = ctx.quantize(dev(xd))
    resid = rng.standard_normal((m, 2048)).astype(np.float32)
    outs = {name: dev(np.zeros((m, n), np.float32)) for name, n, _ in FULL_LAYER}
    outs["down"] = dev(resid.copy())
    items = [dq8.Item(weights[name][2], qd if name == "down" else q, sd if name == "down" else s, outs[name],
                      epilogue=dq8.ADD if name == "down" else dq8.WRITE)
             for name, _, _ in FULL_LAYER if name != "up"]
    ctx.linear_batch(items)
    # up after gate: its SwiGlu reads gate's stored output
    ctx.linear_batch([dq8.Item(weights["up"][2], q, s, outs["gate"], epilogue=dq8.SWIGLU)])
    for name, _, _ in FULL_LAYER:
        wv, ws, _ = weights[name]
        if name == "up":
            continue
        if name == "down":
            want = dq8o.linear(xd, wv, ws, result=resid, epilogue=1, threads=8)
        elif name == "gate":
            gate = dq8o.linear(x, wv, ws, threads=8)
            want = dq8o.linear(x, weights["up"][0], weights["up"][1], result=gate, epilogue=2, threads=8)
        else:
            want = dq8o.linear(x, wv, ws, threads=8)
        assert bits_equal(host(outs[name]), want), name


@pytest.mark.parametrize("m", [24, 9, 32])
def test_linear_batch_short_k_units_dealt(ctx, m):
    # The layer set's eight short-K projections in one grouped launch, no long-K
    # item: 1730 units of 16 columns dealt 6 or 7 to a block and one or two to a
    # wave, so 16- and 32-column pieces start at even and odd units.
    rng = np.random.default_rng(m + 2000)
    short = [(name, n, k) for name, n, k in FULL_LAYER if k == 2048]
    x = make_x(rng, m, 2048, kind="student")
    q, s = ctx.quantize(dev(x))
    items, want = [], {}
    for name, n, k in short:
        wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
        bias = rng.standard_normal(n).astype(np.float32) if name in ("o", "gdn_in") else None
        out = dev(np.zeros((m, n), np.float32))
        items.append(dq8.Item(ctx.weights_from_quantized(dev(wv), dev(ws)), q, s, out,
                              bias=None if bias is None else dev(bias)))
        want[name] = (out, dq8o.linear(x, wv, ws, bias=bias, threads=8))
    ctx.linear_batch(items)
    for name, (out, w) in want.items():
        assert bits_equal(host(out), w), name


def test_skinny_short_path_single_projection_with_lora(ctx):
    # 8224 outputs = 257 one-wave strips: a single projection on the short-K path,
    # with a rank-16 adapter
    rng = np.random.default_rng(8224)
    m, k, n, rank = 24, 2048, 8224, 16
    x, wv, ws, a, b, bias = _lora_case(rng, m, k, n, rank)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.25)
    got = host(ctx.linear_lora(h, q, s, lora, bias=dev(bias)))
    assert bits_equal(got, dq8o.linear_lora(x, wv, ws, a, b, 0.25, bias=bias, threads=8))
    assert bits_equal(host(ctx.linear(h, q, s, bias=dev(bias))), dq8o.linear(x, wv, ws, bias=bias, threads=8))


@pytest.mark.parametrize("tokens", [[24, 24], [24, 24, 24, 24], [24, 17, 31, 9, 24, 5, 30, 24], [24] * 16, [40]])
def test_questions_stacked_rows_match_per_question_launches(ctx, tokens):
    # Continuation of several questions (lib.rs:512-528 runs them one after
    # another): stacking their token rows into one projection launch must give
    # each question the bits of its own launch, since every row is computed on
    # its own.  A scaled-down layer set with long K, all three epilogues and a
    # LoRA adapter; the stacked result is also checked against the oracle.
    rng = np.random.default_rng(sum(tokens) + len(tokens))
    total = sum(tokens)
    starts = np.cumsum([0] + tokens)
    layer = [(2048, 96, dq8.WRITE, False), (6144, 64, dq8.ADD, False), (2048, 160, dq8.SWIGLU, False),
             (256, 40, dq8.WRITE, True)]
    stacked, per_q, wants = [], [[] for _ in tokens], []
    for (k, n, ep, lora) in layer:
        x = make_x(rng, total, k)
        wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
        h = ctx.weights_from_quantized(dev(wv), dev(ws))
        bias = rng.standard_normal(n).astype(np.float32)
        base = (rng.standard_normal((total, n)) * 2).astype(np.float32)
        a = b = None
        if lora:
            a = (rng.standard_normal((8, k)) * 0.05).astype(np.float32)
            b = (rng.standard_normal((n, 8)) * 0.05).astype(np.float32)
        q, s = ctx.quantize(dev(x))
        out = dev(base.copy())
        ad = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.5) if lora else None
        stacked.append(dq8.Item(h, q, s, out, bias=dev(bias), epilogue=ep, lora=ad))
        if lora:
            wants.append(dq8o.linear_lora(x, wv, ws, a, b, 0.5, bias=bias, result=base, epilogue=ep, threads=4))
        else:
            wants.append(dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=4))
        for i in range(len(tokens)):
            r0, r1 = starts[i], starts[i + 1]
            qi, si = ctx.quantize(dev(x[r0:r1]))
            oi = dev(base[r0:r1].copy())
            adi = dq8.Lora(ctx.lora_mid(dev(x[r0:r1]), dev(a)), dev(b), 0.5) if lora else None
            per_q[i].append(dq8.Item(h, qi, si, oi, bias=dev(bias), epilogue=ep, lora=adi))
    ctx.linear_batch(stacked)
    for items in per_q:
        ctx.linear_batch(items)
    for j, want in enumerate(wants):
        got = host(stacked[j].out)
        assert bits_equal(got, want)
        for i in range(len(tokens)):
            assert bits_equal(host(per_q[i][j].out), got[starts[i]:starts[i + 1]])


@pytest.mark.parametrize("ep,lora", [(dq8.WRITE, False), (dq8.SWIGLU, False), (dq8.ADD, True)])
def test_linear_large_grid_bit_exact(ctx, ep, lora):
    # 2048 rows x 4096 outputs: 1024 blocks of the wide kernel with uniform K,
    # the launch shape that keeps the two-group ring (small launches and
    # mixed-K launches take the three-group ring, covered above).
    rng = np.random.default_rng(4096 + ep)
    m, k, n = 2048, 256, 4096
    x = make_x(rng, m, k)
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    bias = rng.standard_normal(n).astype(np.float32)
    base = (rng.standard_normal((m, n)) * 2).astype(np.float32)
    q, s = ctx.quantize(dev(x))
    out = dev(base.copy())
    if lora:
        a = (rng.standard_normal((8, k)) * 0.05).astype(np.float32)
        b = (rng.standard_normal((n, 8)) * 0.05).astype(np.float32)
        ctx.linear_lora(h, q, s, dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.5), out=out, bias=dev(bias),
                        epilogue=ep)
        want = dq8o.linear_lora(x, wv, ws, a, b, 0.5, bias=bias, result=base, epilogue=ep, threads=8)
    else:
        ctx.linear(h, q, s, out=out, bias=dev(bias), epilogue=ep)
        want = dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=8)
    assert bits_equal(host(out), want)


def test_config1_single_linear_seed0_bit_exact(ctx):
    # M=128 tokens, K=2048, N=2048; weights N(0, 0.02^2), activations N(0, 1); seed 0
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((2048, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal((128, 2048)).astype(np.float32)
    h = ctx.weights_from_f32(dev(w))
    q, s = ctx.quantize(dev(x))
    dots = host(ctx.group_dots(h, q))
    out = host(ctx.linear(h, q, s))
    wv, ws = dq8o.quantize_weights(w)
    qh, sh = dq8o.quantize_inputs(x)
    assert np.array_equal(host(q), qh) and bits_equal(host(s), sh)
    ev, es = h.export()
    assert np.array_equal(host(ev), wv) and bits_equal(host(es), ws)
    assert np.array_equal(dots, dq8o.group_dots(qh, wv))
    assert bits_equal(out, dq8o.linear(x, wv, ws, threads=8))


# ------------------------------------------------------------------- LoRA

# The LDS-staged kernels take k % 4 == 0 with 16-byte aligned rows; other
# shapes take the plain-memory kernel.  Shapes cover ranks past one block of 16
# adapter rows (full and partial), partial tiles of 256 inputs, k % 8 == 4
# over several tiles, k with no full chunk of 8 (tail only) and full size.
LORA_MID_SHAPES = [(1, 64, 1), (5, 131, 13), (24, 2048, 16), (67, 100, 3), (130, 2048, 16), (9, 7, 9), (4, 6144, 8),
                   (130, 2048, 40), (9, 256, 64), (300, 1000, 24), (16, 8, 17), (33, 4, 5), (8, 2052, 16),
                   (2048, 2048, 16), (17, 264, 33),
                   # m <= 32: whole rows staged in LDS (4 x rows + 2 adapter rows per block) up to
                   # k = 6656, beyond that the tiled kernel
                   (32, 3328, 16), (32, 3332, 7), (20, 6656, 16), (5, 6660, 3), (31, 2048, 5), (32, 6144, 64)]


@pytest.mark.parametrize("m,k,rank", LORA_MID_SHAPES)
def test_lora_mid_bit_exact(ctx, m, k, rank):
    rng = np.random.default_rng(m * 7 + k + rank)
    x = make_x(rng, m, k)
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    got = host(ctx.lora_mid(dev(x), dev(a)))
    assert bits_equal(got, dq8o.lora_mid(x, a, threads=4))


def test_lora_mid_batch_matches_single_calls(ctx):
    # adapters in one call: few-rows items share grouped launches (35 of them:
    # two launches), items with more rows or k > 6656 share grouped launches of
    # the tiled kernel, the rest (k % 4 != 0, unaligned x) run on their own and
    # rank 0 / m 0 do nothing; every result equals its single call and the oracle
    rng = np.random.default_rng(40)
    shapes = [(24, 2048, 16), (24, 6144, 16), (9, 512, 8), (32, 3332, 7), (1, 64, 1)] * 7 + \
             [(40, 256, 16), (24, 131, 5), (24, 2048, 0), (0, 2048, 16), (17, 6660, 3), (130, 2048, 16),
              (64, 6144, 40), (2048, 2048, 16)]
    pairs, wants = [], []
    for m, k, rank in shapes:
        x = make_x(rng, m, k)
        a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
        pairs.append((dev(x), dev(a)))
        wants.append(dq8o.lora_mid(x, a, threads=4) if m and rank else np.zeros((m, rank), np.float32))
    xf = torch.zeros(24 * 2048 + 1, dtype=torch.float32, device="cuda")
    xu = xf[1:].view(24, 2048)
    xu.copy_(pairs[0][0])
    pairs.append((xu, pairs[0][1]))
    wants.append(wants[0])
    got = ctx.lora_mid_batch(pairs)
    for (x, a), g, want in zip(pairs, got, wants):
        assert bits_equal(host(g), want)
        if x.shape[0] and a.shape[0]:
            assert bits_equal(host(ctx.lora_mid(x, a)), want)


def test_lora_mid_batch_rejects_before_running(ctx):
    # one bad item (lora_A narrower than x): nothing is written, status SHAPE
    good = (dev(np.ones((4, 64), np.float32)), dev(np.ones((2, 64), np.float32)))
    mid = torch.full((4, 2), -1.0, device="cuda")
    lib = dq8.lib()
    arr = (dq8._MidItem * 2)()
    arr[0] = dq8._MidItem(good[0].data_ptr(), 4, 64, good[1].data_ptr(), 2, mid.data_ptr())
    arr[1] = dq8._MidItem(good[0].data_ptr(), 4, 0, good[1].data_ptr(), 2, mid.data_ptr())
    assert lib.dq8_lora_mid_batch(ctx.handle, arr, 2, None) == dq8.ERR_SHAPE
    torch.cuda.synchronize()
    assert (host(mid) == -1.0).all()


def same_nan(got, want):
    """Bit-equal outside NaNs, NaN at the same positions (payloads differ between x86 and the GPU)."""
    got, want = np.asarray(got), np.asarray(want)
    nan = np.isnan(want)
    return got.shape == want.shape and np.array_equal(np.isnan(got), nan) and \
        got[~nan].tobytes() == want[~nan].tobytes()


@pytest.mark.parametrize("m,k,rank", [(24, 2048, 16), (37, 520, 20), (9, 131, 5)])
def test_lora_mid_special_values(ctx, m, k, rank):
    # denormal inputs, products that underflow into (or below) the denormal
    # range, zeros of both signs (rows of -0.0 products sum to +0.0 lane sums),
    # overflow to infinity and NaN inputs, each in its own rows
    rng = np.random.default_rng(k + rank)
    x = make_x(rng, m, k)
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    tiny = np.array([1, 7, 0x7FFFFF, 0x400000], np.uint32).view(np.float32)
    x[0] = rng.choice(tiny, size=k) * rng.choice([-1, 1], size=k).astype(np.float32)
    x[1] = (rng.standard_normal(k) * 1e-20).astype(np.float32)
    a[0] = (rng.standard_normal(k) * 1e-20).astype(np.float32)
    x[2] = -0.0
    x[3, ::3] = -0.0
    x[4] = 0.0
    x[5, k // 2] = 3e38
    a[1 % rank, k // 2] = 1e5
    x[6, k // 3] = np.inf
    x[7, 1] = np.nan
    a[rank - 1, k - 1] = -np.inf
    x[8] = np.float32(1e19) * rng.choice([-1, 1], size=k).astype(np.float32)
    got = host(ctx.lora_mid(dev(x), dev(a)))
    want = dq8o.lora_mid(x, a, threads=4)
    assert same_nan(got, want)
    assert np.isinf(want).any() and np.isnan(want).any()


@pytest.mark.parametrize("m,k,rank", [(24, 2048, 16), (130, 1000, 40), (8, 4, 3)])
def test_lora_mid_unaligned_buffers(ctx, m, k, rank):
    # x and A that are not 16-byte aligned take the plain-memory kernel; both
    # kernels give the oracle's bits
    rng = np.random.default_rng(m + k)
    x = make_x(rng, m, k)
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    want = dq8o.lora_mid(x, a, threads=4)
    xf = torch.zeros(m * k + 1, dtype=torch.float32, device="cuda")
    af = torch.zeros(rank * k + 3, dtype=torch.float32, device="cuda")
    xs, as_ = xf[1:].view(m, k), af[3:].view(rank, k)
    xs.copy_(dev(x))
    as_.copy_(dev(a))
    assert xs.data_ptr() % 16 != 0 and as_.data_ptr() % 16 != 0
    assert bits_equal(host(ctx.lora_mid(xs, as_)), want)
    assert bits_equal(host(ctx.lora_mid(dev(x), dev(a))), want)


# (m, k, n, rank): skinny (m <= 32, short and long K) and wide kernels; ranks
# with full chunks of 8, tails, both, and rank 0.
LORA_SHAPES = [(1, 64, 4, 3), (5, 131, 31, 13), (24, 2048, 96, 16), (17, 6144, 40, 8), (32, 256, 70, 1),
               (67, 131, 31, 13), (130, 2048, 100, 16), (64, 192, 65, 24), (19, 128, 9, 0), (48, 2048, 96, 16),
               (37, 6144, 40, 8), (130, 16384, 100, 16), (24, 12288, 64, 16), (300, 20480, 40, 8)]


def _lora_case(rng, m, k, n, rank):
    x = make_x(rng, m, k)
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((n, rank)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    return x, wv, ws, a, b, bias


@pytest.mark.parametrize("m,k,n,rank", LORA_SHAPES)
def test_linear_lora_bit_exact(ctx, m, k, n, rank):
    rng = np.random.default_rng(m * 31 + k + n * 3 + rank)
    x, wv, ws, a, b, bias = _lora_case(rng, m, k, n, rank)
    scale = 0.375
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    mid = ctx.lora_mid(dev(x), dev(a))
    lora = dq8.Lora(mid, dev(b), scale)
    want = dq8o.linear_lora(x, wv, ws, a, b, scale, bias=bias, threads=4)
    got = host(ctx.linear_lora(h, q, s, lora, bias=dev(bias)))
    assert bits_equal(got, want)
    # Add epilogue and the column layout (linear_int8's own return, tensor.rs:438)
    base = rng.standard_normal((m, n)).astype(np.float32)
    out = dev(base.copy())
    ctx.linear_lora(h, q, s, lora, out=out, bias=dev(bias), epilogue=dq8.ADD)
    assert bits_equal(host(out), dq8o.linear_lora(x, wv, ws, a, b, scale, bias=bias, result=base, epilogue=1))
    cols = host(ctx.linear_lora(h, q, s, lora, bias=dev(bias), layout=dq8.COLUMNS))
    assert bits_equal(cols, np.ascontiguousarray(want.T))


@pytest.mark.parametrize("m", [130, 24])
@pytest.mark.parametrize("rank", [16, 15, 5, 1])
@pytest.mark.parametrize("aligned", [True, False])
def test_linear_lora_operand_staging(ctx, m, rank, aligned):
    # Both kernels load the adapter operands (mid and lora_B rows) before the
    # products: 16-byte loads when rank == 16 and both buffers are 16-byte
    # aligned, element loads otherwise; ragged m and n clamp the rows.  130
    # rows take the wide kernel (operands staged in LDS), 24 the skinny one.
    rng = np.random.default_rng(rank * 2 + aligned + m)
    k, n = 256, 200
    x, wv, ws, a, b, bias = _lora_case(rng, m, k, n, rank)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    mid0 = ctx.lora_mid(dev(x), dev(a))
    if aligned:
        mid, bt = mid0, dev(b)
    else:
        mf = torch.zeros(m * rank + 1, dtype=torch.float32, device="cuda")
        bf = torch.zeros(n * rank + 3, dtype=torch.float32, device="cuda")
        mid, bt = mf[1:].view(m, rank), bf[3:].view(n, rank)
        mid.copy_(mid0)
        bt.copy_(dev(b))
        assert mid.data_ptr() % 16 != 0 and bt.data_ptr() % 16 != 0
    got = host(ctx.linear_lora(h, q, s, dq8.Lora(mid, bt, 0.625), bias=dev(bias)))
    assert bits_equal(got, dq8o.linear_lora(x, wv, ws, a, b, 0.625, bias=bias, threads=4))


def test_linear_lora_swiglu_epilogue(ctx):
    rng = np.random.default_rng(11)
    m, k, n, rank = 24, 2048, 96, 16
    x, wv, ws, a, b, bias = _lora_case(rng, m, k, n, rank)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 2.0)
    gate = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    out = dev(gate.copy())
    ctx.linear_lora(h, q, s, lora, out=out, bias=dev(bias), epilogue=dq8.SWIGLU)
    want = dq8o.linear_lora(x, wv, ws, a, b, 2.0, bias=bias, result=gate, epilogue=2)
    assert bits_equal(host(out), want)


@pytest.mark.parametrize("rows", [1, 19, 67])
def test_reference_fused_lora_case(ctx, rows):
    # weights.rs:657-706: input 131, output 31, rank 13, scale 0.375, bf16-valued
    # weights and LoRA matrices, a bias; Write, Add and SwiGlu.
    width, output, rank, scale = 131, 31, 13, 0.375
    x = np.array([((i * 43 % 113) - 56.0) / 32.0 for i in range(rows * width)], np.float32).reshape(rows, width)

    def packed(count):
        v = np.array([((i * 17 % 89) - 44.0) / 32.0 for i in range(count)], np.float32)
        return (v.view(np.uint32) & 0xFFFF0000).view(np.float32)
    wv, ws = dq8o.quantize_weights(packed(output * width).reshape(output, width))
    a = packed(rank * width).reshape(rank, width)
    b = packed(output * rank).reshape(output, rank)
    bias = np.array([i / 64.0 - 0.25 for i in range(output)], np.float32)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), scale)
    expected = dq8o.linear_lora(x, wv, ws, a, b, scale, bias=bias)
    assert bits_equal(host(ctx.linear_lora(h, q, s, lora, bias=dev(bias))), expected)
    original = np.array([i / 16.0 - 3.0 for i in range(rows * output)], np.float32).reshape(rows, output)
    out = dev(original.copy())
    ctx.linear_lora(h, q, s, lora, out=out, bias=dev(bias), epilogue=dq8.ADD)
    assert bits_equal(host(out), (original + expected).astype(np.float32))


@pytest.mark.parametrize("rows,width,output", [(1, 64, 4), (4, 64, 4), (5, 128, 6), (9, 192, 31), (67, 128, 8),
                                               (7, 100, 9)])
def test_reference_adapter_tile_case(ctx, rows, width, output):
    # tensor.rs:664-732: the projection with a rank-3 adapter whose middle
    # product is given; every output = Adapter::combine(scaled_dot + bias).
    rank = 3
    groups = -(-width // 64)
    x = np.array([((i * 43 % 255) - 127.0) / 9.0 for i in range(rows * width)], np.float32).reshape(rows, width)
    values = np.array([(i * 71 + 128) & 0xFF for i in range(output * width)], np.uint8).reshape(output, width)
    scales = np.array([(i % 7 + 1) / 32.0 for i in range(output * groups)], np.float32).reshape(output, groups)
    bias = np.array([i / 16.0 - 0.5 for i in range(output)], np.float32)
    mid = np.array([(i % 9) / 4.0 - 1.0 for i in range(rows * rank)], np.float32).reshape(rows, rank)
    bw = np.array([(i % 7) / 8.0 for i in range(output * rank)], np.float32).reshape(output, rank)
    h = ctx.weights_from_quantized(dev(values), dev(scales))
    q, s = ctx.quantize(dev(x))
    got = host(ctx.linear_lora(h, q, s, dq8.Lora(dev(mid), dev(bw), 0.375), bias=dev(bias)))
    qh, sh = dq8o.quantize_inputs(x)
    for column in range(output):
        for row in range(rows):
            base = np.float32(dq8o.scaled_dot(qh[row], sh[row], values[column], scales[column]) + bias[column])
            want = dq8o.lora_combine(base, mid[row], bw[column], 0.375)
            assert got[row, column].tobytes() == np.float32(want).tobytes()


def test_linear_batch_with_and_without_lora(ctx):
    rng = np.random.default_rng(5)
    items, wants = [], []
    for (m, k, n, rank) in [(24, 2048, 96, 16), (24, 2048, 40, 0), (24, 6144, 33, 8), (70, 256, 64, 16),
                            (70, 256, 40, None)]:
        x, wv, ws, a, b, bias = _lora_case(rng, m, k, n, rank or 0)
        h = ctx.weights_from_quantized(dev(wv), dev(ws))
        q, s = ctx.quantize(dev(x))
        out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        if rank is None:
            items.append(dq8.Item(h, q, s, out, bias=dev(bias)))
            wants.append(dq8o.linear(x, wv, ws, bias=bias, threads=4))
        else:
            lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), -1.5)
            items.append(dq8.Item(h, q, s, out, bias=dev(bias), lora=lora))
            wants.append(dq8o.linear_lora(x, wv, ws, a, b, -1.5, bias=bias, threads=4))
    ctx.linear_batch(items)
    for it, want in zip(items, wants):
        assert bits_equal(host(it.out), want)


# ------------------------------------------- fused re-quantization, FFN chain

@pytest.mark.parametrize("m,k,n,ep", [(70, 256, 128, dq8.WRITE), (130, 2048, 200, dq8.SWIGLU), (24, 2048, 96, dq8.SWIGLU),
                                      (64, 192, 65, dq8.ADD), (2048, 2048, 384, dq8.SWIGLU), (5, 131, 31, dq8.WRITE)])
def test_linear_q_quantizes_the_stored_result(ctx, m, k, n, ep):
    rng = np.random.default_rng(m + 3 * k + n)
    x = make_x(rng, m, k)
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    base = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    out, qo, so = ctx.linear_q(h, q, s, out=dev(base.copy()), epilogue=ep)
    got = host(out)
    want = dq8o.linear(x, wv, ws, result=base, epilogue=ep, threads=4)
    assert bits_equal(got, want)
    # the quantization is of the stored result, bit for bit (QuantizedInputs::new)
    qh, sh = dq8o.quantize_inputs(got)
    assert np.array_equal(host(qo), qh) and bits_equal(host(so), sh)


def test_linear_q_reports_nonfinite_results(ctx):
    rng = np.random.default_rng(2)
    m, k, n = 70, 256, 64
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(make_x(rng, m, k)))
    base = np.zeros((m, n), np.float32)
    base[3, 5] = np.inf  # Add keeps the infinity in the stored result
    with pytest.raises(dq8.NonFinite):
        ctx.linear_q(h, q, s, out=dev(base.copy()), epilogue=dq8.ADD)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.linear_q(h, q, s, out=dev(base.copy()), epilogue=dq8.ADD, nonfinite=flag)
    assert int(flag.item()) == 1
    flag.zero_()
    ctx.linear_q(h, q, s, out=dev(np.zeros((m, n), np.float32)), epilogue=dq8.ADD, nonfinite=flag)
    assert int(flag.item()) == 0


@pytest.mark.parametrize("m,hidden,inter,lora", [(130, 256, 384, False), (24, 256, 384, True), (512, 2048, 6144, False),
                                                 (96, 192, 320, True), (200, 256, 300, False), (65, 512, 128, False)])
def test_ffn_chain_matches_the_reference_sequence(ctx, m, hidden, inter, lora):
    # qwen.rs:486-492: h = silu(gate(x)) * up(x); residual += down(h), with h
    # re-quantized per token.  h and the residual are both bit-exact.
    rng = np.random.default_rng(m + hidden + inter)
    x = make_x(rng, m, hidden)
    gv, gs = dq8o.quantize_weights(make_w(rng, inter, hidden))
    uv, us = dq8o.quantize_weights(make_w(rng, inter, hidden))
    dv, ds = dq8o.quantize_weights(make_w(rng, hidden, inter))
    G, U, D = (ctx.weights_from_quantized(dev(v), dev(s)) for v, s in ((gv, gs), (uv, us), (dv, ds)))
    q, s = ctx.quantize(dev(x))
    resid0 = rng.standard_normal((m, hidden)).astype(np.float32)
    resid = dev(resid0.copy())
    kw = {}
    if lora:
        r = 8
        ga, gb = (rng.standard_normal((r, hidden)) * 0.05).astype(np.float32), (rng.standard_normal((inter, r)) * 0.05).astype(np.float32)
        ua, ub = (rng.standard_normal((r, hidden)) * 0.05).astype(np.float32), (rng.standard_normal((inter, r)) * 0.05).astype(np.float32)
        da, db = (rng.standard_normal((r, inter)) * 0.05).astype(np.float32), (rng.standard_normal((hidden, r)) * 0.05).astype(np.float32)
        kw = dict(gate_lora=dq8.Lora(ctx.lora_mid(dev(x), dev(ga)), dev(gb), 0.5),
                  up_lora=dq8.Lora(ctx.lora_mid(dev(x), dev(ua)), dev(ub), 0.5),
                  down_lora=(dev(da), dev(db), 0.5))
    h = host(ctx.ffn(G, U, D, q, s, resid, **kw))
    if lora:
        gate = dq8o.linear_lora(x, gv, gs, ga, gb, 0.5, threads=4)
        want_h = dq8o.linear_lora(x, uv, us, ua, ub, 0.5, result=gate, epilogue=2, threads=4)
        want_r = dq8o.linear_lora(want_h, dv, ds, da, db, 0.5, result=resid0, epilogue=1, threads=8)
    else:
        gate = dq8o.linear(x, gv, gs, threads=4)
        want_h = dq8o.linear(x, uv, us, result=gate, epilogue=2, threads=4)
        want_r = dq8o.linear(want_h, dv, ds, result=resid0, epilogue=1, threads=8)
    assert bits_equal(h, want_h)
    assert bits_equal(host(resid), want_r)


@pytest.mark.parametrize("m,hidden,inter", [(130, 256, 384), (40, 256, 384), (24, 128, 96), (300, 1024, 520),
                                             (1000, 2048, 2048), (65, 128, 100), (129, 256, 72)])
def test_ffn_gate_up_equals_write_then_swiglu(ctx, m, hidden, inter):
    # dq8_ffn_gate_up stores what the crate's gate Write and up SwiGlu apply
    # calls store (qwen.rs:489-490): the same bits as two dq8_linear calls and as
    # the oracle, with and without biases; more than 64 rows take the one-launch
    # pair path, fewer the two launches.  With quantize=True, h is also
    # quantized (qwen.rs:491): the same bytes and scales as dq8_quantize(h) and
    # as the oracle's QuantizedInputs::new(h), for widths that end in a partial
    # group and widths that are not a multiple of 16 (byte stores).
    rng = np.random.default_rng(m * 7 + inter)
    x = make_x(rng, m, hidden, "outliers")
    gv, gs = dq8o.quantize_weights(make_w(rng, inter, hidden))
    uv, us = dq8o.quantize_weights(make_w(rng, inter, hidden))
    G, U = ctx.weights_from_quantized(dev(gv), dev(gs)), ctx.weights_from_quantized(dev(uv), dev(us))
    q, s = ctx.quantize(dev(x))
    gb = (rng.standard_normal(inter) * 0.5).astype(np.float32)
    ub = (rng.standard_normal(inter) * 0.5).astype(np.float32)
    for biases in ((None, None), (gb, ub), (None, ub)):
        db = tuple(None if b is None else dev(b) for b in biases)
        got = host(ctx.ffn_gate_up(G, U, q, s, biases=db))
        h = ctx.linear(G, q, s, bias=db[0])
        ctx.linear(U, q, s, out=h, bias=db[1], epilogue=dq8.SWIGLU)
        assert bits_equal(got, host(h))
        gate = dq8o.linear(x, gv, gs, bias=biases[0], threads=8)
        want_h = dq8o.linear(x, uv, us, bias=biases[1], result=gate, epilogue=2, threads=8)
        assert bits_equal(got, want_h)
        hf, hq, hs = ctx.ffn_gate_up(G, U, q, s, biases=db, quantize=True)
        assert bits_equal(host(hf), want_h)
        rq, rs = ctx.quantize(hf)
        assert np.array_equal(host(hq), host(rq)) and bits_equal(host(hs), host(rs))
        oq, os_ = dq8o.quantize_inputs(want_h, threads=8)
        assert np.array_equal(host(hq), oq) and bits_equal(host(hs), os_)


@pytest.mark.parametrize("m", [200, 24])
@pytest.mark.parametrize("given", [False, True])
def test_ffn_gate_up_quantize_reports_a_non_finite_h(ctx, m, given):
    # h overflowing to infinity in one column: QuantizedInputs::new(h) is None
    # (tensor.rs:321-339), reported as dq8_quantize reports it: NonFinite
    # without a flag, 1 ORed into the flag with one; h itself is still stored.
    hidden, inter = 256, 384
    rng = np.random.default_rng(m + given)
    x = rng.standard_normal((m, hidden)).astype(np.float32)
    gv, gs = dq8o.quantize_weights((rng.standard_normal((inter, hidden)) * 0.05).astype(np.float32))
    uv, us = dq8o.quantize_weights((rng.standard_normal((inter, hidden)) * 0.05).astype(np.float32))
    G, U = ctx.weights_from_quantized(dev(gv), dev(gs)), ctx.weights_from_quantized(dev(uv), dev(us))
    gb = np.zeros(inter, np.float32)
    ub = np.zeros(inter, np.float32)
    gb[300], ub[300] = 1e30, 1e30
    q, s = ctx.quantize(dev(x))
    gate = dq8o.linear(x, gv, gs, bias=gb, threads=4)
    want_h = dq8o.linear(x, uv, us, bias=ub, result=gate, epilogue=2, threads=4)
    assert np.isinf(want_h[:, 300]).all()
    h = torch.empty((m, inter), dtype=torch.float32, device="cuda")
    if given:
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ctx.ffn_gate_up(G, U, q, s, h=h, biases=(dev(gb), dev(ub)), quantize=True, nonfinite=flag)
        assert int(host(flag)[0]) == 1
    else:
        with pytest.raises(dq8.NonFinite):
            ctx.ffn_gate_up(G, U, q, s, h=h, biases=(dev(gb), dev(ub)), quantize=True)
    assert bits_equal(host(h), want_h)
    # a finite h afterwards: the flag is not left set by the earlier call
    hf, hq, hs = ctx.ffn_gate_up(G, U, q, s, quantize=True)
    assert np.array_equal(host(hq), dq8o.quantize_inputs(host(hf), threads=4)[0])


@pytest.mark.parametrize("kind", ["student", "edge"])
def test_ffn_full_size_sampled_rows(ctx, kind):
    # One FFN of the 24-layer stack at full size: 2048 tokens, 2048 -> 6144
    # gate/up (one launch of 3072 blocks storing h), h re-quantized, 6144 ->
    # 2048 down Add (qwen.rs:486-492).  Rows are independent, so the oracle
    # recomputes sampled rows of h and of the residual, one in every 64-row tile.
    rng = np.random.default_rng(6144 + len(kind))
    m, hidden, inter = 2048, 2048, 6144
    x = make_x(rng, m, hidden, kind)
    gv, gs = dq8o.quantize_weights(make_w(rng, inter, hidden))
    uv, us = dq8o.quantize_weights(make_w(rng, inter, hidden))
    dv, ds = dq8o.quantize_weights(make_w(rng, hidden, inter))
    gb = (rng.standard_normal(inter) * 0.1).astype(np.float32)
    G, U, D = (ctx.weights_from_quantized(dev(v), dev(s)) for v, s in ((gv, gs), (uv, us), (dv, ds)))
    q, s = ctx.quantize(dev(x))
    resid0 = rng.standard_normal((m, hidden)).astype(np.float32)
    resid = dev(resid0.copy())
    h = host(ctx.ffn(G, U, D, q, s, resid, biases=(dev(gb), None, None)))
    rows = tile_rows(rng, m)
    gate = dq8o.linear(x[rows], gv, gs, bias=gb, threads=8)
    want_h = dq8o.linear(x[rows], uv, us, result=gate, epilogue=2, threads=8)
    assert bits_equal(h[rows], want_h)
    want_r = dq8o.linear(want_h, dv, ds, result=resid0[rows], epilogue=1, threads=8)
    assert bits_equal(host(resid)[rows], want_r)


def test_full_size_gdn_in_projection_properties(ctx):
    # The headline stack's largest projection at full size (2048 tokens x
    # 2048 -> 8224, 2112 wide blocks).  The oracle checks sampled rows, one in
    # every 64-row tile and 32 more; the
    # rest is pinned by properties that hold bit for bit: rows are independent
    # (a row permutation of x permutes the result), and output columns are
    # independent (the weights split in two launches give the same columns).
    rng = np.random.default_rng(8224)
    m, k, n = 2048, 2048, 8224
    x = make_x(rng, m, k, "outliers")
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    full = host(ctx.linear(h, q, s))
    rows = tile_rows(rng, m, extra=32)
    assert bits_equal(full[rows], dq8o.linear(x[rows], wv, ws, threads=8))
    perm = rng.permutation(m)
    qp, sp = ctx.quantize(dev(x[perm]))
    assert bits_equal(host(ctx.linear(h, qp, sp)), full[perm])
    cut = 3000
    h1 = ctx.weights_from_quantized(dev(wv[:cut]), dev(ws[:cut]))
    h2 = ctx.weights_from_quantized(dev(wv[cut:]), dev(ws[cut:]))
    assert bits_equal(np.concatenate([host(ctx.linear(h1, q, s)), host(ctx.linear(h2, q, s))], axis=1), full)


def test_ffn_gate_up_quantize_edge_groups(ctx):
    # The pair launch's quantization of h on edge groups.  Weight rows 0-191 are
    # zero, so those columns of h come from the biases alone: columns 0-63 give
    # silu(-1000) * 0 = -0 (an all-zero group, scale 1); 64-127 silu(-80) ~
    # -1.5e-33 times up biases from 1e-10 to 8e-6 (subnormal h only, scale
    # FLT_MIN, bytes 0 and -1); 128-191 1e18 * 1e18..2e18 (h near 1e36);
    # 192-255 ordinary values.  h, its bytes and scales must equal the
    # oracle's h and QuantizedInputs::new(h).
    m, hidden, inter = 130, 256, 256
    rng = np.random.default_rng(4242)
    x = rng.standard_normal((m, hidden)).astype(np.float32)
    wg = (rng.standard_normal((inter, hidden)) * 0.01).astype(np.float32)
    wu = (rng.standard_normal((inter, hidden)) * 0.01).astype(np.float32)
    wg[:192] = 0.0
    wu[:192] = 0.0
    gv, gs = dq8o.quantize_weights(wg)
    uv, us = dq8o.quantize_weights(wu)
    i64 = np.arange(64, dtype=np.float64)
    gb = np.zeros(inter, np.float32)
    ub = np.zeros(inter, np.float32)
    gb[:64], gb[64:128], gb[128:192] = -1000.0, -80.0, 1e18
    ub[64:128] = (1e-10 * 10.0 ** (i64 * 4.9 / 63)).astype(np.float32)
    ub[128:192] = (1e18 * (1.0 + i64 / 64)).astype(np.float32)
    G, U = ctx.weights_from_quantized(dev(gv), dev(gs)), ctx.weights_from_quantized(dev(uv), dev(us))
    q, s = ctx.quantize(dev(x))
    gate = dq8o.linear(x, gv, gs, bias=gb, threads=8)
    want_h = dq8o.linear(x, uv, us, bias=ub, result=gate, epilogue=2, threads=8)
    tiny = np.finfo(np.float32).tiny
    assert np.all(want_h[:, :64] == 0)
    assert np.all(np.abs(want_h[:, 64:128]) < tiny) and np.any(np.abs(want_h[:, 64:128]) > tiny / 2)
    assert np.all(np.abs(want_h[:, 128:192]) > 1e35) and np.all(np.isfinite(want_h))
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    h, hq, hs = ctx.ffn_gate_up(G, U, q, s, biases=(dev(gb), dev(ub)), quantize=True, nonfinite=flag)
    assert bits_equal(host(h), want_h)
    oq, os_ = dq8o.quantize_inputs(want_h, threads=8)
    assert np.array_equal(host(hq), oq) and bits_equal(host(hs), os_)
    assert np.all(host(hs)[:, 0] == 1.0) and np.all(host(hs)[:, 1] == tiny) and np.any(oq[:, 64:128] != 0)
    assert int(host(flag)[0]) == 0


def _adapter(ctx, rng, m, k, n, rank, scale, x, placed):
    """A LoRA pair for ffn_gate_up: host matrices (a, b) and the device Lora.
    placed "aligned" keeps torch's allocations; "offset" moves mid and b one
    and three floats past 16-byte alignment."""
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((n, rank)) * 0.05).astype(np.float32)
    mid0 = ctx.lora_mid(dev(x), dev(a)) if rank else torch.zeros((m, 0), dtype=torch.float32, device="cuda")
    if placed == "aligned":
        return a, b, dq8.Lora(mid0, dev(b), scale)
    mf = torch.zeros(m * rank + 1, dtype=torch.float32, device="cuda")
    bf = torch.zeros(n * rank + 3, dtype=torch.float32, device="cuda")
    mid, bt = mf[1:].view(m, rank), bf[3:].view(n, rank)
    mid.copy_(mid0)
    bt.copy_(dev(b))
    assert mid.data_ptr() % 16 != 0 and bt.data_ptr() % 16 != 0
    return a, b, dq8.Lora(mid, bt, scale)


# (rows, hidden, intermediate, gate adapter, up adapter); an adapter is (rank,
# placement) or None.  Rank 16 with aligned buffers (the reference checkpoints'
# rank) and rank 0 run in the one-launch pair path; other ranks and offset
# buffers go to separate gate and up launches.
PAIR_LORA_CASES = [(130, 256, 384, (16, "aligned"), (16, "aligned")),
                   (130, 256, 384, (16, "aligned"), None),
                   (130, 256, 384, None, (16, "aligned")),
                   (65, 128, 100, (16, "aligned"), (16, "aligned")),
                   (129, 256, 72, (16, "aligned"), (0, "aligned")),
                   (300, 1024, 520, (16, "aligned"), (16, "aligned")),
                   (300, 1024, 520, (13, "aligned"), (16, "aligned")),
                   (300, 1024, 520, (16, "offset"), (16, "aligned")),
                   (1000, 2048, 2048, (16, "aligned"), (16, "aligned")),
                   (200, 2048, 6144, (16, "aligned"), (16, "aligned"))]


def test_ffn_gate_up_with_adapters_full_size(ctx):
    # The 2048-token stack's FFN shape (2048 x 2048 -> 2 x 6144, rank-16
    # adapters on gate and up, biases, h quantized in the launch): the pair
    # launch equals the separate gate Write and up SwiGlu launches with their
    # adapters on every output, and the oracle on one row of every 64-row tile.
    m, hidden, inter, rank = 2048, 2048, 6144, 16
    rng = np.random.default_rng(2049)
    x = make_x(rng, m, hidden, "student")
    gv, gs = dq8o.quantize_weights(make_w(rng, inter, hidden))
    uv, us = dq8o.quantize_weights(make_w(rng, inter, hidden))
    G, U = ctx.weights_from_quantized(dev(gv), dev(gs)), ctx.weights_from_quantized(dev(uv), dev(us))
    q, s = ctx.quantize(dev(x))
    gb = (rng.standard_normal(inter) * 0.5).astype(np.float32)
    ub = (rng.standard_normal(inter) * 0.5).astype(np.float32)
    ga, gbm = (rng.standard_normal((rank, hidden)) * 0.05).astype(np.float32), \
        (rng.standard_normal((inter, rank)) * 0.05).astype(np.float32)
    ua, ubm = (rng.standard_normal((rank, hidden)) * 0.05).astype(np.float32), \
        (rng.standard_normal((inter, rank)) * 0.05).astype(np.float32)
    gl = dq8.Lora(ctx.lora_mid(dev(x), dev(ga)), dev(gbm), 0.625)
    ul = dq8.Lora(ctx.lora_mid(dev(x), dev(ua)), dev(ubm), -1.5)
    h, hq, hs = ctx.ffn_gate_up(G, U, q, s, biases=(dev(gb), dev(ub)), quantize=True, loras=(gl, ul))
    sep = ctx.linear_lora(G, q, s, gl, bias=dev(gb))
    ctx.linear_lora(U, q, s, ul, out=sep, bias=dev(ub), epilogue=dq8.SWIGLU)
    assert bits_equal(host(h), host(sep))
    rq, rs = ctx.quantize(sep)
    assert np.array_equal(host(hq), host(rq)) and bits_equal(host(hs), host(rs))
    rows = tile_rows(rng, m)
    gate = dq8o.linear_lora(x[rows], gv, gs, ga, gbm, 0.625, bias=gb, threads=8)
    want = dq8o.linear_lora(x[rows], uv, us, ua, ubm, -1.5, bias=ub, result=gate, epilogue=2, threads=8)
    assert bits_equal(host(h)[rows], want)


@pytest.mark.parametrize("m,hidden,inter,gl,ul", PAIR_LORA_CASES)
def test_ffn_gate_up_with_adapters(ctx, m, hidden, inter, gl, ul):
    # dq8_ffn_gate_up_lora: each projection's adapter term (Adapter::combine,
    # tensor.rs:109-117, after the bias, 438) before silu(gate) * up
    # (qwen.rs:489-490).  The same bits as the gate Write and up SwiGlu calls
    # with their adapters and as the oracle; with quantize=True h's bytes and
    # scales equal QuantizedInputs::new(h).
    rng = np.random.default_rng(m * 13 + inter + hidden)
    x = make_x(rng, m, hidden, "outliers")
    gv, gs = dq8o.quantize_weights(make_w(rng, inter, hidden))
    uv, us = dq8o.quantize_weights(make_w(rng, inter, hidden))
    G, U = ctx.weights_from_quantized(dev(gv), dev(gs)), ctx.weights_from_quantized(dev(uv), dev(us))
    q, s = ctx.quantize(dev(x))
    gb = (rng.standard_normal(inter) * 0.5).astype(np.float32)
    ub = (rng.standard_normal(inter) * 0.5).astype(np.float32)
    ad = [None if spec is None else _adapter(ctx, rng, m, hidden, inter, spec[0], sc, x, spec[1])
          for spec, sc in ((gl, 0.625), (ul, -1.5))]
    loras = tuple(None if a is None else a[2] for a in ad)
    got = host(ctx.ffn_gate_up(G, U, q, s, biases=(dev(gb), dev(ub)), loras=loras))
    h = (ctx.linear_lora(G, q, s, loras[0], bias=dev(gb)) if loras[0] is not None
         else ctx.linear(G, q, s, bias=dev(gb)))
    if loras[1] is not None:
        ctx.linear_lora(U, q, s, loras[1], out=h, bias=dev(ub), epilogue=dq8.SWIGLU)
    else:
        ctx.linear(U, q, s, out=h, bias=dev(ub), epilogue=dq8.SWIGLU)
    assert bits_equal(got, host(h))
    if ad[0] is not None:
        gate = dq8o.linear_lora(x, gv, gs, ad[0][0], ad[0][1], 0.625, bias=gb, threads=8)
    else:
        gate = dq8o.linear(x, gv, gs, bias=gb, threads=8)
    if ad[1] is not None:
        want_h = dq8o.linear_lora(x, uv, us, ad[1][0], ad[1][1], -1.5, bias=ub, result=gate, epilogue=2, threads=8)
    else:
        want_h = dq8o.linear(x, uv, us, bias=ub, result=gate, epilogue=2, threads=8)
    assert bits_equal(got, want_h)
    hf, hq, hs = ctx.ffn_gate_up(G, U, q, s, biases=(dev(gb), dev(ub)), quantize=True, loras=loras)
    assert bits_equal(host(hf), want_h)
    oq, os_ = dq8o.quantize_inputs(want_h, threads=8)
    assert np.array_equal(host(hq), oq) and bits_equal(host(hs), os_)


# 65-512 rows whose wide launch would be small run as 32-row chunks on the
# skinny kernel (dq8_linear and grouped calls through run_linear, dq8_apply
# through its own launch); shapes on both sides of the rule's limits.
SMALL_CALLS = [(65, 2048, 300, dq8.WRITE), (96, 6144, 2048, dq8.ADD), (128, 2048, 2048, dq8.SWIGLU),
               (128, 2048, 8224, dq8.WRITE), (200, 4096, 100, dq8.ADD), (256, 2048, 512, dq8.WRITE),
               (384, 2048, 2048, dq8.SWIGLU), (512, 2048, 2048, dq8.WRITE), (512, 6144, 1024, dq8.ADD),
               (513, 2048, 256, dq8.WRITE), (192, 2048, 6144, dq8.SWIGLU), (192, 6144, 2048, dq8.ADD),
               (256, 6144, 2048, dq8.ADD)]


@pytest.mark.parametrize("m,k,n,ep", SMALL_CALLS)
def test_small_calls_bit_exact(ctx, m, k, n, ep):
    rng = np.random.default_rng(m * 7 + k + n + ep)
    x = make_x(rng, m, k, "student")
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    bias = rng.standard_normal(n).astype(np.float32)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    base = rng.standard_normal((m, n)).astype(np.float32)
    got = host(ctx.linear(h, q, s, out=dev(base.copy()), bias=dev(bias), epilogue=ep))
    want = dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=8)
    assert bits_equal(got, want)
    # the same rows through dq8_apply (fp32 input, quantized inside, its own launch)
    got_a = host(ctx.apply(h, dev(x), out=dev(base.copy()), bias=dev(bias), epilogue=ep))
    assert bits_equal(got_a, want)


@pytest.mark.parametrize("m", [100, 300])
def test_small_call_with_adapter_and_group(ctx, m):
    # An adapter through the chunked path (its middle-product rows follow the
    # chunks), and a grouped call whose items are all small.
    rng = np.random.default_rng(m + 5)
    k, n, rank = 2048, 640, 16
    x = make_x(rng, m, k, "outliers")
    wv, ws = dq8o.quantize_weights(make_w(rng, n, k))
    a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((n, rank)) * 0.05).astype(np.float32)
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.5)
    got = host(ctx.linear_lora(h, q, s, lora, epilogue=dq8.WRITE))
    assert bits_equal(got, dq8o.linear_lora(x, wv, ws, a, b, 0.5, threads=8))
    w2v, w2s = dq8o.quantize_weights(make_w(rng, 512, k))
    h2 = ctx.weights_from_quantized(dev(w2v), dev(w2s))
    o1 = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    o2 = torch.zeros((m, 512), dtype=torch.float32, device="cuda")
    ctx.linear_batch([dq8.Item(h, q, s, o1), dq8.Item(h2, q, s, o2)])
    assert bits_equal(host(o1), dq8o.linear(x, wv, ws, threads=8))
    assert bits_equal(host(o2), dq8o.linear(x, w2v, w2s, threads=8))
