"""dq8_apply_noalloc through the C ABI: the same bits as dq8_apply on
consecutive calls (the second smaller, then a non-finite input that takes the
FP32 path on the device), and inputs beyond its fixed scratch rejected with
ERR_LIMIT before anything is enqueued."""
import ctypes

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
    a, b = np.asarray(a), np.asarray(b)
    nan = np.isnan(b)
    return a.shape == b.shape and np.array_equal(np.isnan(a), nan) and a[~nan].tobytes() == b[~nan].tobytes()


def noalloc(ctx, w, x, out, bias=None, lora=None, epilogue=dq8.WRITE):
    lo = ctx._lora(lora, x.shape[0], w.n) if lora is not None else None
    return dq8.lib().dq8_apply_noalloc(ctx.handle, w.handle, x.data_ptr(), x.shape[0],
                                       None if bias is None else bias.data_ptr(),
                                       ctypes.byref(lo) if lo is not None else None, out.data_ptr(), dq8.ROWS,
                                       epilogue, torch.cuda.current_stream().cuda_stream)


def test_apply_noalloc_matches_apply_on_consecutive_calls(ctx):
    rng = np.random.default_rng(707)
    cases = [
        # (m, k, n, epilogue, non-finite input, adapter rank)
        (1024, 2048, 512, dq8.ADD, False, 0),   # wide kernel, 1024 x 2048 quantized into the scratch
        (24, 6144, 96, dq8.SWIGLU, False, 8),   # smaller: skinny kernel, long K, with an adapter
        (70, 300, 40, dq8.WRITE, True, 0),      # a NaN: the device flag picks the FP32 path
    ]
    for m, k, n, ep, bad, rank in cases:
        x = rng.standard_normal((m, k)).astype(np.float32)
        if bad:
            x[5, 17] = np.nan
        wv, ws = dq8o.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        h = ctx.weights_from_quantized(dev(wv), dev(ws))
        bias = rng.standard_normal(n).astype(np.float32)
        base = rng.standard_normal((m, n)).astype(np.float32)
        lora = None
        if rank:
            a = (rng.standard_normal((rank, k)) * 0.05).astype(np.float32)
            b = (rng.standard_normal((n, rank)) * 0.05).astype(np.float32)
            lora = dq8.Lora(ctx.lora_mid(dev(x), dev(a)), dev(b), 0.5)
        want = dev(base.copy())
        ctx.apply(h, dev(x), out=want, bias=dev(bias), lora=lora, epilogue=ep)
        got = dev(base.copy())
        assert noalloc(ctx, h, dev(x), got, bias=dev(bias), lora=lora, epilogue=ep) == dq8.OK
        g, w_ = host(got), host(want)
        assert same_bits(g, w_), (m, k, n)
        if bad:
            assert np.isnan(g[5]).all() and not np.isnan(g[4]).any()
        elif not rank:
            assert same_bits(g, dq8o.linear(x, wv, ws, bias=bias, result=base, epilogue=ep, threads=8))
        h.free()


def test_apply_noalloc_rejects_inputs_beyond_its_scratch(ctx):
    # 4096 x 4160: 4096 * 65 * 64 bytes of quantized rows alone exceed 16 MiB
    m, k, n = 4096, 4160, 8
    wv, ws = dq8o.quantize_weights(np.ones((n, k), np.float32))
    h = ctx.weights_from_quantized(dev(wv), dev(ws))
    x = torch.ones((m, k), dtype=torch.float32, device="cuda")
    out = torch.full((m, n), 3.0, dtype=torch.float32, device="cuda")
    assert noalloc(ctx, h, x, out) == dq8.ERR_LIMIT
    assert (host(out) == 3.0).all()
    # the largest the scratch holds: 2048 x 6144 (12 MiB of rows, 0.75 MiB of scales)
    m, k = 2048, 6144
    wv, ws = dq8o.quantize_weights(np.full((n, k), 0.5, np.float32))
    h2 = ctx.weights_from_quantized(dev(wv), dev(ws))
    x = torch.ones((m, k), dtype=torch.float32, device="cuda")
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    assert noalloc(ctx, h2, x, out) == dq8.OK
    want = ctx.apply(h2, x)
    assert host(out).tobytes() == host(want).tobytes()
    h.free()
    h2.free()


def test_apply_noalloc_captures_on_a_fresh_context_and_replays_bit_exact():
    # A new context has no workspace at all, so dq8_apply would have to
    # allocate (and refuses under capture); dq8_apply_noalloc captures as it
    # is and its replays equal the oracle.  Shapes: a 128-row small call whose
    # int8 path runs as skinny row chunks over the scratch-held inputs, a
    # 2048-row wide launch, and a 24-row skinny call.
    rng = np.random.default_rng(909)
    c = dq8.Context(0)
    try:
        cases = [(128, 2048, 2048), (2048, 2048, 512), (24, 6144, 256)]
        stream = torch.cuda.Stream()
        for m, k, n in cases:
            x0 = rng.standard_normal((m, k)).astype(np.float32)
            wv, ws = dq8o.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
            bias0 = rng.standard_normal(n).astype(np.float32)
            h = c.weights_from_quantized(dev(wv), dev(ws))
            x, bias = dev(x0), dev(bias0)
            out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            status = []
            with torch.cuda.graph(g, stream=stream):
                status.append(noalloc(c, h, x, out, bias=bias))
            assert status == [dq8.OK], (m, k, n)
            want = dq8o.linear(x0, wv, ws, bias=bias0, threads=8)
            for replay in range(3):
                out.fill_(-1.0)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                assert same_bits(host(out), want), (m, k, n, replay)
                # eager work between the replays, on the same shared scratch
                eager = torch.zeros((m, n), dtype=torch.float32, device="cuda")
                assert noalloc(c, h, dev(rng.standard_normal((m, k)).astype(np.float32)), eager) == dq8.OK
                torch.cuda.synchronize()
            del g
            h.free()
    finally:
        torch.cuda.synchronize()
        c.close()
