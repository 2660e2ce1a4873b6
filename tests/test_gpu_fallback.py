"""GPU parity of the FP32 path (Projection::columns_tiled, tensor.rs:206-269)
that Projection::apply_quantized takes for non-finite inputs (tensor.rs:197-201):
dq8_linear_fp32 (the path itself), dq8_apply (the device picks the path) and the
FFN chain's down projection on a non-finite h.  Finite results are bit-exact
against the oracle; NaN positions must match (NaN payloads are not compared)."""
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


def same(got, want):
    got, want = np.asarray(got), np.asarray(want)
    nan = np.isnan(want)
    return got.shape == want.shape and np.array_equal(np.isnan(got), nan) and \
        got[~nan].tobytes() == want[~nan].tobytes()


def oracle_fp32(x, v, s, bias=None, a=None, b=None, scale=0.0, result=None, epilogue=0):
    """columns_tiled over dequantized weights, adapter, store (composed from pinned parts)."""
    vals = dq8o.linear_f32(x, dq8o.dequantize_weights(v, s), bias=bias, threads=8)
    if a is not None:
        delta = dq8o.linear_f32(dq8o.lora_mid(x, a, threads=8), b, threads=8)
        vals = (vals + (np.float32(scale) * delta).astype(np.float32)).astype(np.float32)
    if epilogue == 0:
        return vals
    base = np.asarray(result, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        if epilogue == 1:
            return (base + vals).astype(np.float32)
    return np.array([dq8o.silu(o) * e for o, e in zip(base.ravel(), vals.ravel())], np.float32).reshape(vals.shape)


def case(rng, m, k, n, rank=0):
    x = (rng.standard_normal((m, k)) * 2).astype(np.float32)
    v, s = dq8o.quantize_weights((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    bias = rng.standard_normal(n).astype(np.float32)
    a = b = None
    if rank:
        a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
        b = (rng.standard_normal((n, rank)) * 0.05).astype(np.float32)
    return x, v, s, bias, a, b


SHAPES = [(1, 1, 1, 0), (5, 7, 3, 0), (33, 100, 70, 3), (70, 131, 65, 0), (24, 2048, 96, 16), (130, 257, 200, 8),
          (3, 64, 300, 1), (64, 6144, 40, 0)]


@pytest.mark.parametrize("m,k,n,rank", SHAPES)
@pytest.mark.parametrize("ep", [dq8.WRITE, dq8.ADD, dq8.SWIGLU])
def test_linear_fp32_is_columns_tiled(ctx, m, k, n, rank, ep):
    rng = np.random.default_rng(m * 13 + k + n + rank + ep)
    x, v, s, bias, a, b = case(rng, m, k, n, rank)
    h = ctx.weights_from_quantized(dev(v), dev(s))
    base = (rng.standard_normal((m, n)) * 2).astype(np.float32)
    lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.75) if rank else None
    got = host(ctx.linear_fp32(h, dev(x), out=dev(base.copy()), bias=dev(bias), lora=lora, epilogue=ep))
    want = oracle_fp32(x, v, s, bias, a, b, 0.75, base, ep)
    assert got.tobytes() == want.tobytes()


def test_linear_fp32_columns_layout(ctx):
    rng = np.random.default_rng(2)
    x, v, s, bias, _, _ = case(rng, 37, 300, 90)
    h = ctx.weights_from_quantized(dev(v), dev(s))
    got = host(ctx.linear_fp32(h, dev(x), bias=dev(bias), layout=dq8.COLUMNS))
    assert got.tobytes() == np.ascontiguousarray(oracle_fp32(x, v, s, bias).T).tobytes()


@pytest.mark.parametrize("m,k,n,rank", [(24, 2048, 96, 0), (130, 257, 200, 8), (48, 6144, 64, 16), (3, 131, 31, 0)])
@pytest.mark.parametrize("bad", [None, np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("ep", [dq8.WRITE, dq8.ADD])
def test_apply_takes_the_path_the_crate_takes(ctx, m, k, n, rank, bad, ep):
    rng = np.random.default_rng(m + k + n + rank)
    x, v, s, bias, a, b = case(rng, m, k, n, rank)
    if bad is not None:
        x[m // 2, k // 3] = bad
    h = ctx.weights_from_quantized(dev(v), dev(s))
    base = rng.standard_normal((m, n)).astype(np.float32)
    lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.5) if rank else None
    got = host(ctx.apply(h, dev(x), out=dev(base.copy()), bias=dev(bias), lora=lora, epilogue=ep))
    want, fp32 = dq8o.apply(x, v, s, bias=bias, a=a, b=b, scale=0.5, result=base, epilogue=ep, threads=8)
    assert fp32 == (bad is not None)
    assert same(got, want)
    # the same call again (the context flag is reset per call)
    got2 = host(ctx.apply(h, dev(x), out=dev(base.copy()), bias=dev(bias), lora=lora, epilogue=ep))
    assert got2.tobytes() == got.tobytes()


@pytest.mark.parametrize("m", [24, 130])
def test_ffn_with_a_non_finite_h_takes_the_fp32_down(ctx, m):
    # qwen.rs:486-492 with h overflowing to infinity: the crate's down
    # projection finds QuantizedInputs::new(h) = None and runs columns_tiled.
    hidden, inter = 256, 384
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, hidden)).astype(np.float32)
    gv, gs = dq8o.quantize_weights((rng.standard_normal((inter, hidden)) * 0.05).astype(np.float32))
    uv, us = dq8o.quantize_weights((rng.standard_normal((inter, hidden)) * 0.05).astype(np.float32))
    dv, ds = dq8o.quantize_weights((rng.standard_normal((hidden, inter)) * 0.05).astype(np.float32))
    gb = np.zeros(inter, np.float32)
    ub = np.zeros(inter, np.float32)
    gb[7], ub[7] = 1e30, 1e30  # column 7 of h: silu(~1e30) * ~1e30 = inf
    G, U, D = (ctx.weights_from_quantized(dev(v), dev(s)) for v, s in ((gv, gs), (uv, us), (dv, ds)))
    q, s = ctx.quantize(dev(x))
    resid0 = rng.standard_normal((m, hidden)).astype(np.float32)
    resid = dev(resid0.copy())
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    h = host(ctx.ffn(G, U, D, q, s, resid, biases=(dev(gb), dev(ub), None), nonfinite=flag))
    gate = dq8o.linear(x, gv, gs, bias=gb, threads=4)
    want_h = dq8o.linear(x, uv, us, bias=ub, result=gate, epilogue=2, threads=4)
    assert np.isinf(want_h[:, 7]).all()
    assert same(h, want_h)
    want_r, fp32 = dq8o.apply(want_h, dv, ds, result=resid0, epilogue=1, threads=8)
    assert fp32
    assert same(host(resid), want_r)
    assert int(host(flag)[0]) == 1
