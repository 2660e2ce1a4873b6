"""GPU parity at the edges of the fp32 rescale and of silu.

  - Overflowing scale products (int8.rs:53-61): finite x and w groups whose
    x-scale * w-scale product exceeds FLT_MAX, so p = +inf and t = dot * p is
    +-inf, or NaN where the group's dot is 0; groups whose p is finite but
    dot * p overflows; and rows where two such groups of opposite sign meet
    (inf - inf = NaN).  They run through every projection path: the wide
    kernel, the 16- and 32-row skinny kernels, the two-chunk split, the
    dealt short-K units and the 4-wave long-K strips, and the SwiGLU pair
    launch, with the Write, Add and SwiGlu stores.
  - silu (qwen.rs:194-199) on every one of the 2^32 binary32 inputs, through
    the SwiGlu store of the wide kernel and through the pair launch, against
    the oracle's silu (libm expf, as the reference's f32::exp): 0 mismatches.

NaN results are compared by position: the oracle (x86) and the GPU produce
different NaN payloads for inf - inf and 0 * inf, and the reference's outputs
carry no meaning in a NaN's payload.
"""
import numpy as np
import pytest
import torch

import dq8
import dq8o

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same_bits(a, b):
    """Bit-equal outside NaNs, NaN at the same positions."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if a.shape != b.shape:
        return False
    nan = np.isnan(b)
    return np.array_equal(np.isnan(a), nan) and a[~nan].tobytes() == b[~nan].tobytes()


BIG_X, BIG_W = np.float32(1e20), np.float32(1e25)  # scales 7.9e17 and 7.9e22: the product overflows


def overflow_x(rng, m, k):
    """Rows 3i: group 0 of random large values; rows 3i+1: group 0 = [A, -A,
    0, ...] (a zero dot against the [B, B, 0, ...] weight rows) and group 1
    large; rows 3i+2: ~1e19 in group 0 (finite p against ~1.6e21 weights,
    dot * p overflows)."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    sign = np.where(rng.random((m, 64)) < 0.5, -1, 1).astype(np.float32)
    mag = rng.uniform(0.5, 1.0, (m, 64)).astype(np.float32)
    r0, r1, r2 = np.arange(0, m, 3), np.arange(1, m, 3), np.arange(2, m, 3)
    x[r0, :64] = (sign * mag * BIG_X)[r0]
    x[r1, :64] = 0.0
    x[r1, 0], x[r1, 1] = BIG_X, -BIG_X
    x[r1, 64:128] = (sign * mag * BIG_X)[r1]
    x[r2, :64] = (sign * mag * np.float32(1e19))[r2]
    return x


def overflow_w(rng, n, k):
    """Rows 5j: group 0 large; 5j+1: group 0 = [B, B, 0, ...]; 5j+2: groups 0
    and 1 large with opposite signs; 5j+3: group 0 ~1.6e21; 5j+4: ordinary."""
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    sign = np.where(rng.random((n, 128)) < 0.5, -1, 1).astype(np.float32)
    mag = rng.uniform(0.5, 1.0, (n, 128)).astype(np.float32)
    j = np.arange(n)
    r0, r1, r2, r3 = j[j % 5 == 0], j[j % 5 == 1], j[j % 5 == 2], j[j % 5 == 3]
    w[r0, :64] = (sign[:, :64] * mag[:, :64] * BIG_W)[r0]
    w[r1, :64] = 0.0
    w[r1, 0] = w[r1, 1] = BIG_W
    w[r2, :64] = (mag[:, :64] * BIG_W)[r2]
    w[r2, 64:128] = -(mag[:, 64:] * BIG_W)[r2]
    w[r3, :64] = (sign[:, :64] * mag[:, :64] * np.float32(1.6e21))[r3]
    return w


def check_overflow_cases(want):
    """The oracle's results hold +inf, -inf and NaN, so every case is live."""
    assert np.isposinf(want).any() and np.isneginf(want).any() and np.isnan(want).any()
    assert np.isfinite(want).any()


# m = 9 and 24: the skinny kernel (16- and 32-row); 48: two skinny row chunks;
# 96 and 200: the wide kernel.  n = 100 columns run on the 4-wave strips (few
# strips); k = 6144 is long K.
@pytest.mark.parametrize("m", [9, 24, 48, 96, 200])
@pytest.mark.parametrize("ep", [dq8.WRITE, dq8.ADD, dq8.SWIGLU])
@pytest.mark.parametrize("k", [2048, 6144])
def test_overflowing_scale_products(ctx, m, ep, k):
    rng = np.random.default_rng(31 * m + 7 * ep + k)
    n = 100
    x = overflow_x(rng, m, k)
    wv, ws = dq8o.quantize_weights(overflow_w(rng, n, k))
    qh, sh = dq8o.quantize_inputs(x)
    with np.errstate(over="ignore"):
        assert np.isinf(np.float32(sh[0, 0]) * np.float32(ws[0, 0]))  # the product overflows
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    assert np.array_equal(host(q), qh) and host(s).tobytes() == sh.tobytes()
    bias = rng.standard_normal(n).astype(np.float32)
    base = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    base[:, ::7] = 0.0  # silu(0) * inf = NaN in the SwiGlu store
    out = dev(base.copy())
    ctx.linear(h, q, s, out=out, bias=dev(bias), epilogue=ep)
    want = dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=8)
    check_overflow_cases(want)
    assert same_bits(host(out), want)
    if ep == dq8.WRITE:  # the column-major layout of linear_int8
        cols = ctx.linear(h, q, s, layout=dq8.COLUMNS)
        assert same_bits(host(cols), dq8o.linear_int8(qh, sh, wv, ws, threads=8))
    h.free()


@pytest.mark.parametrize("m", [9, 24])
def test_overflowing_scale_products_on_dealt_short_k_units(ctx, m):
    # 6144 columns at short K: 192 strips, so the skinny launch deals its
    # 16-column units over the blocks instead of the 4-wave strips.
    rng = np.random.default_rng(6144 + m)
    n, k = 6144, 2048
    x = overflow_x(rng, m, k)
    wv, ws = dq8o.quantize_weights(overflow_w(rng, n, k))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(x))
    got = host(ctx.linear(h, q, s))
    want = dq8o.linear(x, wv, ws, threads=8)
    check_overflow_cases(want)
    assert same_bits(got, want)
    h.free()


def test_overflowing_scale_products_through_the_pair_launch(ctx):
    # gate and up of one FFN in one wide launch (h = silu(gate) * up), with
    # the overflowing groups in both projections; h's quantization reports
    # the non-finite h through the device flag.
    rng = np.random.default_rng(4242)
    m, k, n = 130, 2048, 320
    x = overflow_x(rng, m, k)
    gv, gs = dq8o.quantize_weights(overflow_w(rng, n, k))
    wu = overflow_w(rng, n, k)[::-1].copy()
    wu[n // 2:] = rng.standard_normal((n - n // 2, k)) * np.float32(0.02)  # up columns with ordinary weights
    uv, us = dq8o.quantize_weights(wu)
    G = ctx.weights_from_quantized(dev(gv), dev(gs))
    U = ctx.weights_from_quantized(dev(uv), dev(us))
    q, s = ctx.quantize(dev(x))
    h = host(ctx.ffn_gate_up(G, U, q, s))
    gate = dq8o.linear(x, gv, gs, threads=8)
    want = dq8o.linear(x, uv, us, result=gate, epilogue=2, threads=8)
    check_overflow_cases(want)
    assert same_bits(h, want)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    h2, hq, hs = ctx.ffn_gate_up(G, U, q, s, quantize=True, nonfinite=flag)
    assert same_bits(host(h2), want) and int(host(flag)[0]) == 1
    G.free()
    U.free()


# ------------------------------------------------------------ silu on all 2^32 inputs

def _pattern_chunk(start, count):
    """float32 tensor on the GPU holding the bit patterns start .. start+count-1."""
    i = torch.arange(start, start + count, dtype=torch.int64, device="cuda")
    return (i - (i >= 2 ** 31).to(torch.int64) * 2 ** 32).to(torch.int32).view(torch.float32)


def _mismatches(got, want):
    nan = np.isnan(want)
    bad = np.isnan(got) != nan
    bad |= ~nan & (got.view(np.uint32) != want.view(np.uint32))
    return int(bad.sum())


def test_silu_on_every_binary32_input_through_the_swiglu_store(ctx):
    # Zero weights and a bias of 1 give y = 1 for every output, so the wide
    # kernel's SwiGlu store writes silu(old) * 1 = silu(old) over an output
    # that was filled with bit patterns: 64 launches of 4096 x 16384 cover
    # all 2^32 of them.
    m, n = 4096, 16384
    per = m * n
    wv, ws = dq8o.quantize_weights(np.zeros((n, 64), np.float32))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    q, s = ctx.quantize(dev(np.ones((m, 64), np.float32)))
    bias = dev(np.ones(n, np.float32))
    pinned = torch.empty(per, dtype=torch.float32, pin_memory=True)
    total = 0
    for c in range(2 ** 32 // per):
        out = _pattern_chunk(c * per, per).view(m, n)
        ctx.linear(h, q, s, out=out, bias=bias, epilogue=dq8.SWIGLU)
        pinned.copy_(out.view(-1))
        torch.cuda.synchronize()
        got = pinned.numpy()
        pat = (np.arange(per, dtype=np.uint32) + np.uint32(c * per)).view(np.float32)
        total += _mismatches(got, dq8o.silu_n(pat, threads=16))
    assert total == 0
    h.free()


def test_silu_on_every_binary32_input_through_the_pair_launch(ctx):
    # Gate and up weights are zero, the gate bias holds the bit patterns and
    # the up bias is 1: every row of h is silu(0 + pattern) * 1.  (0 + -0 is
    # +0, so -0 itself cannot reach this silu; everything else does.)  512
    # launches of 65 rows x 2^23 columns cover all 2^32 patterns.
    m, n = 65, 1 << 23
    zv, zs = dq8o.quantize_weights(np.zeros((1, 64), np.float32))
    G = ctx.weights_from_quantized(torch.zeros((n, 64), dtype=torch.uint8, device="cuda"),
                                   torch.ones((n, 1), dtype=torch.float32, device="cuda"))
    U = ctx.weights_from_quantized(torch.zeros((n, 64), dtype=torch.uint8, device="cuda"),
                                   torch.ones((n, 1), dtype=torch.float32, device="cuda"))
    assert zv.tobytes() == bytes(64) and zs[0, 0] == 1.0  # what the zero weights quantize to
    q, s = ctx.quantize(dev(np.ones((m, 64), np.float32)))
    up_bias = torch.ones(n, dtype=torch.float32, device="cuda")
    hbuf = torch.empty((m, n), dtype=torch.float32, device="cuda")
    pinned = torch.empty(2 * n, dtype=torch.float32, pin_memory=True)
    total = 0
    for c in range(2 ** 32 // n):
        gate_bias = _pattern_chunk(c * n, n)
        ctx.ffn_gate_up(G, U, q, s, h=hbuf, biases=(gate_bias, up_bias))
        pinned[:n].copy_(hbuf[0])
        pinned[n:].copy_(hbuf[m - 1])
        torch.cuda.synchronize()
        got = pinned.numpy()
        pat = (np.arange(n, dtype=np.uint32) + np.uint32(c * n)).view(np.float32)
        with np.errstate(invalid="ignore"):
            want = dq8o.silu_n(np.float32(0.0) + pat, threads=16)
        total += _mismatches(got[:n], want) + _mismatches(got[n:], want)
    assert total == 0
    G.free()
    U.free()
