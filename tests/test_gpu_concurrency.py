"""Two contexts on two streams at once, sharing weight handles (immutable
after creation): results equal the single-stream ones bit for bit."""
import numpy as np
import pytest
import torch

import dq8
import dq8o

pytestmark = pytest.mark.gpu


def test_two_contexts_on_two_streams_share_weights():
    rng = np.random.default_rng(21)
    a_ctx, b_ctx = dq8.Context(0), dq8.Context(0)
    try:
        w1 = (rng.standard_normal((384, 2048)) * 0.05).astype(np.float32)
        w2 = (rng.standard_normal((2048, 384)) * 0.05).astype(np.float32)
        v1, s1 = dq8o.quantize_weights(w1)
        v2, s2 = dq8o.quantize_weights(w2)
        h1 = a_ctx.weights_from_quantized(torch.from_numpy(v1).cuda(), torch.from_numpy(s1).cuda())
        h2 = a_ctx.weights_from_quantized(torch.from_numpy(v2).cuda(), torch.from_numpy(s2).cuda())
        xs = [rng.standard_normal((m, 2048)).astype(np.float32) for m in (24, 130, 512, 48)]
        xn = xs[1].copy()
        xn[7, 9] = np.inf
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        outs = {}
        for rep in range(3):
            for i, x in enumerate(xs + [xn]):
                ctx, st = (a_ctx, sa) if i % 2 == 0 else (b_ctx, sb)
                with torch.cuda.stream(st):
                    xd = torch.from_numpy(x).cuda()
                    y = ctx.apply(h1, xd)            # quantize + int8 (or FP32) on the context's workspace
                    z = ctx.apply(h2, y)             # a second projection on the first one's result
                    outs[(rep, i)] = (y, z)
        torch.cuda.synchronize()
        for i, x in enumerate(xs + [xn]):
            y_want, _ = dq8o.apply(x, v1, s1, threads=8)
            z_want, _ = dq8o.apply(y_want, v2, s2, threads=8)
            for rep in range(3):
                y, z = (t.cpu().numpy() for t in outs[(rep, i)])
                for got, want in ((y, y_want), (z, z_want)):
                    nan = np.isnan(want)
                    assert np.array_equal(np.isnan(got), nan)
                    assert got[~nan].tobytes() == want[~nan].tobytes(), (rep, i)
    finally:
        a_ctx.close()
        b_ctx.close()
