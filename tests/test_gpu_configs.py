"""GPU parity at the benchmark workloads' full sizes, and edge inputs through
the projection kernels.

  - one layer's projection set at the 4096-token window with 1% of the input
    channels scaled x20 (GQA q/k/v/o, Gated DeltaNet in/out);
  - a full Gated DeltaNet layer and a full GQA layer of the 24-layer stack at
    2048 tokens with Student-t(3) activations, every launch of the benchmark
    step (grouped q/k/v, o, GDN in/out, FFN gate Write, up SwiGlu, the
    re-quantized h and down Add into the residual);
  - zero, denormal-only and 127*FLT_MIN groups of x (tensor.rs:766-803) and of
    the weights through the wide and skinny kernels, so that x-scale * w-scale
    products are subnormal or underflow;
  - non-finite weights rejected by every weight entry point (weights.rs:170-187).

Full-size results are checked against the oracle on sampled rows, at least one
in every 64-row tile (rows are independent: each is quantized and multiplied
on its own) and, for the rest,
through properties that hold bit for bit: a row permutation of the input
permutes the output rows, and splitting the weight rows over two handles gives
the same columns.
"""
import numpy as np
import pytest
import torch

import dq8
import dq8o

pytestmark = pytest.mark.gpu

FLT_MIN = np.float32(np.finfo(np.float32).tiny)
DENORM = np.array([1], np.uint32).view(np.float32)[0]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def normal(rng, rows, width):
    return rng.standard_normal((rows, width)).astype(np.float32)


def outliers(rng, rows, width):
    """N(0, 1) with 1% of the channels (rounded down) scaled x20 across all tokens."""
    x = normal(rng, rows, width)
    ch = rng.choice(width, size=width // 100, replace=False)
    x[:, ch] *= np.float32(20.0)
    return x


def student(rng, rows, width):
    z = rng.standard_normal((rows, width))
    chi = rng.chisquare(3, size=(rows, width))
    return (z / np.sqrt(chi / 3)).astype(np.float32)


def tile_rows(rng, m, extra=8, tile=64):
    """Oracle rows of a full-size check: one random row in every 64-row tile
    of the output (each wide launch's row tiles, and with them every XCD
    region and column chunk of the tile walk), the first and last rows, and a
    few more at random."""
    rows = [int(rng.integers(t, min(t + tile, m))) for t in range(0, m, tile)]
    return np.unique(np.r_[rows, 0, m - 1, rng.choice(m, size=extra, replace=False)])


def weights(ctx, rng, n, k):
    wv, ws = dq8o.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    return wv, ws, ctx.weights_from_quantized(dev(wv), dev(ws))


# ------------------------------------------------------------ non-finite weights

@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_weights_from_f32_rejects_nonfinite(ctx, bad):
    # Data::read rejects "non-finite weights" before Data::quantize ever sees
    # them (weights.rs:170-187): every weight entry point returns NONFINITE
    w = (np.random.default_rng(5).standard_normal((70, 130)) * 0.02).astype(np.float32)
    w[69, 129] = bad
    with pytest.raises(dq8.NonFinite):
        ctx.weights_from_f32(dev(w))
    with pytest.raises(dq8.NonFinite):
        ctx.weights_from_raw(dev(w))
    w[69, 129] = 0.5
    h = ctx.weights_from_f32(dev(w))  # the same context still works afterwards
    values, scales = h.export()
    wv, ws = dq8o.quantize_weights(w)
    assert np.array_equal(host(values), wv) and bits_equal(host(scales), ws)


# ------------------------------------------------------------ edge groups

def edge_x(rng, rows, width):
    """x with a zero group, a denormal-only group (scale FLT_MIN, so the
    product with a weight scale is subnormal), a group whose absmax is
    127*FLT_MIN (scale FLT_MIN exactly) and exact-half quotients."""
    x = normal(rng, rows, width)
    x[:, 0:64] = 0.0
    x[:, 64:128] = DENORM
    x[1::3, 64:128] = -DENORM * 3
    x[:, 128:192] = 0.0
    x[:, 128] = np.float32(127.0) * FLT_MIN
    x[:, 130] = -np.float32(63.5) * FLT_MIN
    x[::2, 200] = np.float32(2.5)
    return x


def edge_w(rng, n, k):
    """weights with a row group of denormals (w scale FLT_MIN: products with x
    scales underflow to subnormals or zero), a zero group and tiny groups."""
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0
    w[1, :] = DENORM * 5
    w[2, 64:128] = np.float32(127.0) * FLT_MIN
    w[3, 128:192] = -DENORM
    w[4, :] = np.float32(1e30)  # large scales: products near the top of the range
    return w


# m = 9 and 24: the skinny kernel (16- and 32-row); 48: two skinny row chunks;
# 96 and 200: the wide kernel
@pytest.mark.parametrize("m", [9, 24, 48, 96, 200])
@pytest.mark.parametrize("ep", [dq8.WRITE, dq8.ADD, dq8.SWIGLU])
@pytest.mark.parametrize("k", [2048, 6144])
def test_edge_groups_through_projection_kernels(ctx, m, ep, k):
    rng = np.random.default_rng(m * 10 + ep + k)
    n = 96
    x = edge_x(rng, m, k)
    wv, ws = dq8o.quantize_weights(edge_w(rng, n, k))
    assert ws[1, 0] == FLT_MIN  # the denormal row's scale is the floor
    qh, sh = dq8o.quantize_inputs(x)
    assert sh[0, 1] == FLT_MIN and sh[0, 2] == FLT_MIN and sh[0, 0] == 1.0
    p = np.float32(sh[0, 1]) * np.float32(ws[0, 1])  # a subnormal x-scale * w-scale product
    assert 0 < p < FLT_MIN
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    assert np.array_equal(host(q), qh) and bits_equal(host(s), sh)
    bias = rng.standard_normal(n).astype(np.float32)
    base = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    out = dev(base.copy())
    ctx.linear(h, q, s, out=out, bias=dev(bias), epilogue=ep)
    want = dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=8)
    assert bits_equal(host(out), want)
    # the same through the column-major layout of linear_int8 (Write only)
    if ep == dq8.WRITE:
        cols = ctx.linear(h, q, s, layout=dq8.COLUMNS)
        assert bits_equal(host(cols), dq8o.linear_int8(qh, sh, wv, ws, threads=8))


# ------------------------------------------------------------ config 3: 4096-token layer set

LAYER3 = [("q", 2048), ("k", 512), ("v", 512), ("o", 2048), ("gdn_in", 4 * 2048 + 2 * 16), ("gdn_out", 2048)]


def test_layer_projection_set_4096_tokens_with_outlier_channels(ctx):
    # GQA q (16 heads x 128), k/v (4 KV heads x 128) in one grouped launch, o;
    # Gated DeltaNet in (q, k, v, z + b, a) and out.  x feeds q/k/v/GDN in;
    # o and GDN out read their own (attention / recurrence output) inputs.
    rng = np.random.default_rng(4096)
    m, hidden = 4096, 2048
    W = {name: weights(ctx, rng, n, hidden) for name, n in LAYER3}
    x, xo, xg = (outliers(rng, m, hidden) for _ in range(3))
    inputs = {"q": x, "k": x, "v": x, "gdn_in": x, "o": xo, "gdn_out": xg}
    qs = {}
    for key, arr in (("x", x), ("o", xo), ("g", xg)):
        qs[key] = ctx.quantize(dev(arr))
    src = {"q": "x", "k": "x", "v": "x", "gdn_in": "x", "o": "o", "gdn_out": "g"}
    outs = {name: torch.zeros((m, n), dtype=torch.float32, device="cuda") for name, n in LAYER3}
    ctx.linear_batch([dq8.Item(W[nm][2], *qs["x"], outs[nm]) for nm in ("q", "k", "v")])
    for nm in ("gdn_in", "o", "gdn_out"):
        ctx.linear(W[nm][2], *qs[src[nm]], out=outs[nm])
    got = {nm: host(o) for nm, o in outs.items()}
    rows = tile_rows(rng, m)
    for nm, _ in LAYER3:
        wv, ws, _ = W[nm]
        want = dq8o.linear(inputs[nm][rows], wv, ws, threads=16)
        assert bits_equal(got[nm][rows], want), nm
    # every other row: a row permutation of x permutes the results (rows are
    # computed independently), checked on the largest projection
    perm = rng.permutation(m)
    qp, sp = ctx.quantize(dev(x[perm]))
    assert bits_equal(host(ctx.linear(W["gdn_in"][2], qp, sp)), got["gdn_in"][perm])
    # and the columns of k/v: the weight rows split over two handles
    wv, ws, _ = W["k"]
    h1 = ctx.weights_from_quantized(dev(wv[:200]), dev(ws[:200]))
    h2 = ctx.weights_from_quantized(dev(wv[200:]), dev(ws[200:]))
    both = np.concatenate([host(ctx.linear(h1, *qs["x"])), host(ctx.linear(h2, *qs["x"]))], axis=1)
    assert bits_equal(both, got["k"])


# ------------------------------------------------------------ config 5: full layers at 2048 tokens

def _ffn_check(ctx, rng, W, m, rows, x_ffn):
    """The step's FFN launches (gate Write, up SwiGlu, quantize h, down Add)
    against the oracle on sampled rows."""
    gate = torch.empty((m, 6144), dtype=torch.float32, device="cuda")
    resid0 = rng.standard_normal((m, 2048)).astype(np.float32)
    resid = dev(resid0)
    q, s = ctx.quantize(dev(x_ffn))
    ctx.linear(W["gate"][2], q, s, out=gate)
    ctx.linear(W["up"][2], q, s, out=gate, epilogue=dq8.SWIGLU)
    qh, sh = ctx.quantize(gate)
    ctx.linear(W["down"][2], qh, sh, out=resid, epilogue=dq8.ADD)
    h = host(gate)
    g_want = dq8o.linear(x_ffn[rows], W["gate"][0], W["gate"][1], threads=16)
    h_want = dq8o.linear(x_ffn[rows], W["up"][0], W["up"][1], result=g_want, epilogue=2, threads=16)
    assert bits_equal(h[rows], h_want), "h = silu(gate) * up"
    qhh, shh = dq8o.quantize_inputs(h[rows])
    assert np.array_equal(host(qh)[rows], qhh) and bits_equal(host(sh)[rows], shh), "re-quantized h"
    r_want = dq8o.linear(h[rows], W["down"][0], W["down"][1], result=resid0[rows], epilogue=1, threads=16)
    assert bits_equal(host(resid)[rows], r_want), "residual += down(h)"


def test_stack_gdn_layer_2048_tokens_student_t(ctx):
    rng = np.random.default_rng(2048)
    m = 2048
    W = {nm: weights(ctx, rng, n, k) for nm, n, k in
         [("in", 8224, 2048), ("out", 2048, 2048), ("gate", 6144, 2048), ("up", 6144, 2048), ("down", 2048, 6144)]}
    x, xm, xf = (student(rng, m, 2048) for _ in range(3))
    rows = tile_rows(rng, m)
    q, s = ctx.quantize(dev(x))
    mixer = host(ctx.linear(W["in"][2], q, s))
    assert bits_equal(mixer[rows], dq8o.linear(x[rows], W["in"][0], W["in"][1], threads=16)), "GDN in"
    qm, sm = ctx.quantize(dev(xm))
    out = host(ctx.linear(W["out"][2], qm, sm))
    assert bits_equal(out[rows], dq8o.linear(xm[rows], W["out"][0], W["out"][1], threads=16)), "GDN out"
    _ffn_check(ctx, rng, W, m, rows, xf)


def test_stack_gqa_layer_2048_tokens_student_t(ctx):
    rng = np.random.default_rng(2049)
    m = 2048
    W = {nm: weights(ctx, rng, n, k) for nm, n, k in
         [("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048), ("gate", 6144, 2048),
          ("up", 6144, 2048), ("down", 2048, 6144)]}
    x, xo, xf = (student(rng, m, 2048) for _ in range(3))
    rows = tile_rows(rng, m)
    q, s = ctx.quantize(dev(x))
    outs = {nm: torch.zeros((m, W[nm][0].shape[0]), dtype=torch.float32, device="cuda") for nm in ("q", "k", "v")}
    ctx.linear_batch([dq8.Item(W[nm][2], q, s, outs[nm]) for nm in ("q", "k", "v")])
    for nm in ("q", "k", "v"):
        assert bits_equal(host(outs[nm])[rows], dq8o.linear(x[rows], W[nm][0], W[nm][1], threads=16)), nm
    qo, so = ctx.quantize(dev(xo))
    o = host(ctx.linear(W["o"][2], qo, so))
    assert bits_equal(o[rows], dq8o.linear(xo[rows], W["o"][0], W["o"][1], threads=16)), "o"
    _ffn_check(ctx, rng, W, m, rows, xf)
