"""HIP graph capture of the library's asynchronous calls.

A step of quantize / linear (wide and skinny) / grouped launch / SwiGlu / Add /
LoRA (single and grouped middle products) / FFN chain / apply (device-side path
choice) is captured once on a side stream and replayed several times, with eager
work and synchronizations in between.  Every replay must reproduce the eager results bit for bit (NaN
positions for the non-finite apply)."""
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


def bits_equal(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def test_captured_step_replays_bit_exact(ctx):
    rng = np.random.default_rng(77)
    M, H, F = 130, 256, 384
    mk = lambda n, k: ctx.weights_from_quantized(*(dev(t) for t in dq8o.quantize_weights(
        (rng.standard_normal((n, k)) * 0.05).astype(np.float32))))
    wq, wg, wu, wd = mk(H, H), mk(F, H), mk(F, H), mk(H, F)
    x0 = rng.standard_normal((M, H)).astype(np.float32)
    xs0 = rng.standard_normal((24, H)).astype(np.float32)
    xn0 = x0.copy()
    xn0[3, 5] = np.nan
    res0 = rng.standard_normal((M, H)).astype(np.float32)
    a = (rng.standard_normal((8, H)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((F, 8)) * 0.05).astype(np.float32)

    x, xs, xn, A, B = dev(x0), dev(xs0), dev(xn0), dev(a), dev(b)
    res_init = dev(res0)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    q = torch.empty((M, H), dtype=torch.int8, device="cuda")
    s = torch.empty((M, H // 64), dtype=torch.float32, device="cuda")
    qs = torch.empty((24, H), dtype=torch.int8, device="cuda")
    ss = torch.empty((24, H // 64), dtype=torch.float32, device="cuda")
    mid = torch.empty((M, 8), dtype=torch.float32, device="cuda")
    x24 = dev(rng.standard_normal((24, H)).astype(np.float32))

    def step(o):
        """Writes every result into the dict of buffers o."""
        o["res"].copy_(res_init)
        ctx.quantize(x, q, s, nonfinite=flag)
        ctx.quantize(xs, qs, ss, nonfinite=flag)
        ctx.linear(wq, q, s, out=o["wide"])
        ctx.linear(wq, qs, ss, out=o["skinny"])
        ctx.linear_batch([dq8.Item(wg, q, s, o["g1"]), dq8.Item(wg, qs, ss, o["g2"])])
        ctx.lora_mid(x, A, mid=mid)
        ctx.lora_mid_batch([(x, A), (x24, A), (xs, A)], mids=[o["mb0"], o["mb1"], o["mb2"]])
        ctx.linear_lora(wg, q, s, dq8.Lora(mid, B, 0.5), out=o["lora"])
        ctx.ffn(wg, wu, wd, q, s, o["res"], h=o["h"])
        ctx.apply(wq, xn, out=o["apply"])

    def buffers():
        z = lambda *shape: torch.zeros(shape, dtype=torch.float32, device="cuda")
        return {"res": z(M, H), "wide": z(M, H), "skinny": z(24, H), "g1": z(M, F), "g2": z(24, F),
                "lora": z(M, F), "h": z(M, F), "apply": z(M, H), "mb0": z(M, 8), "mb1": z(24, 8), "mb2": z(24, 8)}

    stream = torch.cuda.Stream()
    eager, graph_out = buffers(), buffers()
    with torch.cuda.stream(stream):
        step(eager)          # eager reference (also grows every workspace before capture)
        step(graph_out)
    torch.cuda.synchronize()
    want = {k: v.cpu().numpy() for k, v in eager.items()}
    assert np.isnan(want["apply"][3]).all() and not np.isnan(want["apply"][4]).any()

    g = torch.cuda.CUDAGraph()
    for t in graph_out.values():
        t.zero_()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=stream):
        step(graph_out)
    for replay in range(4):
        for t in graph_out.values():
            t.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k, v in graph_out.items():
            got = v.cpu().numpy()
            nan = np.isnan(want[k])
            assert np.array_equal(np.isnan(got), nan), (replay, k)
            assert got[~nan].tobytes() == want[k][~nan].tobytes(), (replay, k)
        # eager work between replays
        with torch.cuda.stream(stream):
            step(eager)
        torch.cuda.synchronize()


def test_capture_does_not_grow_and_earlier_graphs_survive_growth():
    # A fresh context has no workspace: a captured dq8_apply that would have
    # to allocate one returns CAPTURE and enqueues nothing.  After dq8_reserve
    # the same calls capture; an eager call at a larger size then grows the
    # workspace, and the earlier graph (which holds the old buffer) still
    # replays bit-exact, because outgrown buffers are kept until destroy.
    rng = np.random.default_rng(91)
    c = dq8.Context(0)
    try:
        H, F = 256, 384
        mk = lambda n, k: (lambda v, s: (v, s, c.weights_from_quantized(dev(v), dev(s))))(
            *dq8o.quantize_weights((rng.standard_normal((n, k)) * 0.05).astype(np.float32)))
        wq, wg, wu, wd = mk(H, H), mk(F, H), mk(F, H), mk(H, F)
        x0 = rng.standard_normal((24, H)).astype(np.float32)
        res0 = rng.standard_normal((24, H)).astype(np.float32)
        x, res_init = dev(x0), dev(res0)
        q = torch.empty((24, H), dtype=torch.int8, device="cuda")
        s = torch.empty((24, H // 64), dtype=torch.float32, device="cuda")
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        out = torch.zeros((24, H), dtype=torch.float32, device="cuda")
        res = torch.zeros((24, H), dtype=torch.float32, device="cuda")
        h = torch.zeros((24, F), dtype=torch.float32, device="cuda")
        stream = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with pytest.raises(dq8.Dq8Error) as err:
            with torch.cuda.graph(g, stream=stream):
                c.apply(wq[2], x, out=out)
        assert err.value.status == dq8.ERR_CAPTURE
        torch.cuda.synchronize()
        c.reserve(24, F)

        def step():
            res.copy_(res_init)
            c.apply(wq[2], x, out=out)
            c.quantize(x, q, s, nonfinite=flag)
            c.ffn(wg[2], wu[2], wd[2], q, s, res, h=h)

        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            step()
        want_out = dq8o.linear(x0, wq[0], wq[1], threads=4)
        gate = dq8o.linear(x0, wg[0], wg[1], threads=4)
        want_h = dq8o.linear(x0, wu[0], wu[1], result=gate, epilogue=2, threads=4)
        want_res = dq8o.linear(want_h, wd[0], wd[1], result=res0, epilogue=1, threads=4)
        big = rng.standard_normal((512, H)).astype(np.float32)
        for replay in range(3):
            out.fill_(-1.0)
            h.fill_(-1.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert bits_equal(host(out), want_out), replay
            assert bits_equal(host(h), want_h), replay
            assert bits_equal(host(res), want_res), replay
            # eager calls at a larger size grow the workspace between replays
            got = c.apply(wq[2], dev(big))
            assert bits_equal(host(got), dq8o.linear(big, wq[0], wq[1], threads=4)), replay
            qb, sb = c.quantize(dev(big))
            c.ffn(wg[2], wu[2], wd[2], qb, sb, torch.zeros((big.shape[0], H), dtype=torch.float32, device="cuda"))
            torch.cuda.synchronize()
            big = rng.standard_normal((512 * (replay + 2), H)).astype(np.float32)
        del g
    finally:
        torch.cuda.synchronize()
        c.close()


def test_synchronizing_calls_refuse_capture_and_enqueue_nothing(ctx):
    # Calls that report a non-finite input by synchronizing (no flag pointer
    # given) return CAPTURE on a capturing stream before enqueuing anything,
    # so the capture stays usable: the same stream then captures and replays
    # the flag-pointer forms of the same calls, bit-exact to eager.
    rng = np.random.default_rng(93)
    H, F, M = 256, 384, 130
    mk = lambda n, k: ctx.weights_from_quantized(*(dev(t) for t in dq8o.quantize_weights(
        (rng.standard_normal((n, k)) * 0.05).astype(np.float32))))
    wq, wg, wu = mk(H, H), mk(F, H), mk(F, H)
    x = dev(rng.standard_normal((M, H)).astype(np.float32))
    q, s = ctx.quantize(x)
    out = torch.zeros((M, H), dtype=torch.float32, device="cuda")
    h = torch.zeros((M, F), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    refusing = [lambda: ctx.quantize(x), lambda: ctx.linear_q(wq, q, s, out=out),
                lambda: ctx.ffn_gate_up(wg, wu, q, s, h=h, quantize=True), lambda: ctx.linear_f32in(wq, x, out=out)]
    for call in refusing:
        g = torch.cuda.CUDAGraph()
        with pytest.raises(dq8.Dq8Error) as err:
            with torch.cuda.graph(g, stream=stream):
                call()
        assert err.value.status == dq8.ERR_CAPTURE
    torch.cuda.synchronize()
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    qo = torch.empty((M, H), dtype=torch.int8, device="cuda")
    so = torch.empty((M, H // 64), dtype=torch.float32, device="cuda")
    hq = torch.empty((M, F), dtype=torch.int8, device="cuda")
    hs = torch.empty((M, F // 64), dtype=torch.float32, device="cuda")

    def step():
        ctx.quantize(x, qo, so, nonfinite=flag)
        lib = dq8.lib()
        assert lib.dq8_ffn_gate_up(ctx.handle, wg.handle, wu.handle, qo.data_ptr(), so.data_ptr(), M, None, None,
                                   h.data_ptr(), hq.data_ptr(), hs.data_ptr(), flag.data_ptr(),
                                   stream.cuda_stream) == 0

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    want = [host(t) for t in (qo, so, h, hq, hs)]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    for _ in range(3):
        for t in (qo, so, h, hq, hs):
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip((qo, so, h, hq, hs), want):
            assert bits_equal(host(a), b)
    assert int(host(flag)[0]) == 0


def test_reserve_while_another_stream_captures_globally_keeps_that_capture():
    # dq8_reserve grows the workspace from the NULL stream.  While a side
    # stream captures in global mode, a plain allocation would invalidate that
    # capture (HIP reports the NULL stream as not capturing meanwhile); the
    # library allocates in relaxed mode, so the reserve succeeds, the capture
    # ends and replays, and the reserved workspace then lets a captured
    # dq8_apply of that size run without allocating.
    rng = np.random.default_rng(95)
    c = dq8.Context(0)
    try:
        x = torch.zeros(16, dtype=torch.float32, device="cuda")
        stream = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        status = []
        with torch.cuda.graph(g, stream=stream, capture_error_mode="global"):
            x.add_(1.0)
            status.append(dq8.lib().dq8_reserve(c.handle, 300, 256, 0))
        assert status == [dq8.OK]
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        assert host(x).tolist() == [2.0] * 16
        wv, ws = dq8o.quantize_weights((rng.standard_normal((64, 256)) * 0.05).astype(np.float32))
        w = c.weights_from_quantized(dev(wv), dev(ws))
        a0 = rng.standard_normal((300, 256)).astype(np.float32)
        a, out = dev(a0), torch.zeros((300, 64), dtype=torch.float32, device="cuda")
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2, stream=stream):
            c.apply(w, a, out=out)
        g2.replay()
        torch.cuda.synchronize()
        assert bits_equal(host(out), dq8o.linear(a0, wv, ws, threads=4))
        del g, g2
        w.free()
    finally:
        torch.cuda.synchronize()
        c.close()
