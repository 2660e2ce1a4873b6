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
