#!/usr/bin/env python3
"""Benchmark of the MI355X int8 projection path (one JSON line on stdout).

Headline workload (a "step"): the full projection stack of a 24-layer,
2048-hidden model for one 2048-token prefill -- 18 Gated DeltaNet layers and 6
GQA layers in D,D,D,F order, each followed by a 2048<->6144 SwiGLU FFN:
  GDN  in 2048->8224 (q,k,v,z + b,a concatenated), out 2048->2048
  GQA  q 2048->2048, k 2048->512, v 2048->512 (one grouped launch), o 2048->2048
  FFN  gate 2048->6144 (Write), up 2048->6144 (SwiGlu into gate),
       down 6144->2048 (Add into the residual) on the re-quantized gate
Every projection input is quantized inside the step (as the reference's timed
region does); weights are repacked once before timing.  Weights ~N(0, 0.02^2),
activations Student-t(3), seeded; all inputs are resident in HBM.

Secondary workload (reported under "skinny"): 16 questions x 24 tokens, each
question one grouped skinny launch over one layer's projection set (q, k, v, o,
GDN in/out, FFN gate/up/down), rotating 5 weight copies (> 256 MB MALL) so
weight bytes come from HBM.  "questions_stacked" runs the same questions layer
by layer with their rows stacked into one 384-row launch per layer set.

"roofline" is for the dominant kernel (the wide projection kernel): achieved
= algorithmic int8 ops per launch / its average launch time from HIP events on
the launch stream.  "cpu_baseline" times the oracle (the C restatement of the
reference's x86 path) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "decider-engine_amd"))

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E, 8 TB/s
HIDDEN, FFN_DIM, GDN_IN = 2048, 6144, 4 * 2048 + 2 * 16
LAYER_KINDS = ["gdn", "gdn", "gdn", "gqa"] * 6


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--tokens", type=int, default=2048)
    p.add_argument("--questions", type=int, default=16)
    p.add_argument("--question-tokens", type=int, default=24)
    p.add_argument("--weight-copies", type=int, default=5)
    p.add_argument("--skinny-reps", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="time eager submission only (no HIP graph replay)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--lora-rank", type=int, default=16,
                   help="rank of the LoRA adapters of the stack's second pass (0: skip it)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device copy (for rocprof counter calibration)")
    return p.parse_args()


def student_t(torch, gen, shape, device):
    z = torch.randn(shape, generator=gen, device=device)
    chi = (torch.randn((3,) + tuple(shape), generator=gen, device=device) ** 2).sum(0)
    return (z / torch.sqrt(chi / 3.0)).contiguous()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every box here has one GPU)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import dq8

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.add(src, 0.0, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4}))
        return
    ctx = dq8.Context(0)
    lib = dq8.lib()
    # all work on one side stream (default priority): it can be graph-captured
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    sh = stream.cuda_stream
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)

    def weights(n, k):
        w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).contiguous()
        h = ctx.weights_from_f32(w)
        del w
        return h

    M = args.tokens
    # ---------------------------------------------------------- the stack
    layers = []
    for kind in LAYER_KINDS:
        L = {"kind": kind}
        if kind == "gdn":
            L["in"] = weights(GDN_IN, HIDDEN)
            L["out"] = weights(HIDDEN, HIDDEN)
        else:
            L["q"] = weights(HIDDEN, HIDDEN)
            L["k"] = weights(512, HIDDEN)
            L["v"] = weights(512, HIDDEN)
            L["o"] = weights(HIDDEN, HIDDEN)
        L["gate"] = weights(FFN_DIM, HIDDEN)
        L["up"] = weights(FFN_DIM, HIDDEN)
        L["down"] = weights(HIDDEN, FFN_DIM)
        L["x"] = student_t(torch, gen, (M, HIDDEN), dev)      # mixer input
        L["mix"] = student_t(torch, gen, (M, HIDDEN), dev)    # attention / recurrence output
        L["ffn"] = student_t(torch, gen, (M, HIDDEN), dev)    # post-norm FFN input
        layers.append(L)
    groups = lambda k: (k + 63) // 64
    qx = torch.empty((M, HIDDEN), dtype=torch.int8, device=dev)
    sx = torch.empty((M, groups(HIDDEN)), dtype=torch.float32, device=dev)
    qf = torch.empty((M, FFN_DIM), dtype=torch.int8, device=dev)
    sf = torch.empty((M, groups(FFN_DIM)), dtype=torch.float32, device=dev)
    mixer_out = torch.empty((M, GDN_IN), dtype=torch.float32, device=dev)
    k_out = torch.empty((M, 512), dtype=torch.float32, device=dev)
    v_out = torch.empty((M, 512), dtype=torch.float32, device=dev)
    proj_out = torch.empty((M, HIDDEN), dtype=torch.float32, device=dev)
    gate = torch.empty((M, FFN_DIM), dtype=torch.float32, device=dev)
    resid = torch.zeros((M, HIDDEN), dtype=torch.float32, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)

    def quant(x, q, s, k):
        return ("quant", lib.dq8_quantize, (ctx.handle, x.data_ptr(), M, k, q.data_ptr(), s.data_ptr(),
                                            flag.data_ptr(), sh), (M * k * 4 + M * k + M * groups(k) * 4, 0))

    def linear(w, q, s, out, ep):
        return ("linear", lib.dq8_linear, (ctx.handle, w.handle, q.data_ptr(), s.data_ptr(), M, None,
                                           out.data_ptr(), dq8.ROWS, ep, sh), (0, 2 * M * w.n * w.k))

    rank = args.lora_rank
    mids = {k: torch.empty((M, max(rank, 1)), dtype=torch.float32, device=dev) for k in ("a", "b", "c")}
    keep = []  # ctypes structs referenced by queued calls

    def lora_of(L, name):
        """The projection's rank-`rank` FP32 LoRA pair (A [rank][K], B [N][rank]), made on first use."""
        key = "lora_" + name
        if key not in L:
            w = L[name]
            a = (torch.randn((rank, w.k), generator=gen, device=dev) * 0.02).contiguous()
            b = (torch.randn((w.n, rank), generator=gen, device=dev) * 0.02).contiguous()
            L[key] = (a, b)
        return L[key]

    def mid_call(x, a, mid, k):
        return ("mid", lib.dq8_lora_mid, (ctx.handle, x.data_ptr(), M, k, a.data_ptr(), rank, mid.data_ptr(), sh),
                (0, 2 * M * k * rank))

    def mid_batch_call(entries):
        """The middle products of projections that share an input, in one dq8_lora_mid_batch call:
        entries = [(x, A, mid, k)]."""
        arr = (dq8._MidItem * len(entries))()
        for i, (x, a, mid, k) in enumerate(entries):
            arr[i] = dq8._MidItem(x.data_ptr(), M, k, a.data_ptr(), rank, mid.data_ptr())
        keep.append(arr)
        return ("mid", lib.dq8_lora_mid_batch, (ctx.handle, arr, len(entries), sh),
                (0, sum(2 * M * k * rank for _, _, _, k in entries)))

    def lora_linear(L, name, x, q, s, out, ep, mid, k, with_mid=True):
        """mid = linear(x, A) then the projection with its adapter (weights.rs:492-520)."""
        a, b = lora_of(L, name)
        w = L[name]
        lo = dq8._Lora(mid.data_ptr(), b.data_ptr(), rank, 2.0)
        keep.append(lo)
        return ([mid_call(x, a, mid, k)] if with_mid else []) + \
               [("linear", lib.dq8_linear_lora, (ctx.handle, w.handle, q.data_ptr(), s.data_ptr(), M, None,
                                                  ctypes.byref(lo), out.data_ptr(), dq8.ROWS, ep, sh),
                 (0, 2 * M * w.n * w.k))]

    def build(with_lora):
        calls = []

        def proj(L, name, x, q, s, out, ep, mid, k, with_mid=True):
            if with_lora:
                calls.extend(lora_linear(L, name, x, q, s, out, ep, mid, k, with_mid))
            else:
                calls.append(linear(L[name], q, s, out, ep))

        for L in layers:
            calls.append(quant(L["x"], qx, sx, HIDDEN))
            if L["kind"] == "gdn":
                proj(L, "in", L["x"], qx, sx, mixer_out, dq8.WRITE, mids["a"], HIDDEN)
            else:
                items = (dq8._Item * 3)()
                outs = (mixer_out, k_out, v_out)
                shared = []  # q, k and v share their input: one grouped launch of their middle products
                for i, name in enumerate(("q", "k", "v")):
                    lp = None
                    if with_lora:
                        a, b = lora_of(L, name)
                        mid = torch.empty((M, rank), dtype=torch.float32, device=dev)
                        keep.append(mid)
                        shared.append((L["x"], a, mid, HIDDEN))
                        lo = dq8._Lora(mid.data_ptr(), b.data_ptr(), rank, 2.0)
                        keep.append(lo)
                        lp = ctypes.pointer(lo)
                    items[i] = dq8._Item(L[name].handle, qx.data_ptr(), sx.data_ptr(), M, None, outs[i].data_ptr(),
                                         dq8.ROWS, dq8.WRITE, lp)
                keep.append(items)
                if shared:
                    calls.append(mid_batch_call(shared))
                flops = sum(2 * M * L[n].n * L[n].k for n in ("q", "k", "v"))
                calls.append(("linear", lib.dq8_linear_batch, (ctx.handle, items, 3, sh), (0, flops)))
            calls.append(quant(L["mix"], qx, sx, HIDDEN))
            proj(L, "out" if L["kind"] == "gdn" else "o", L["mix"], qx, sx, proj_out, dq8.WRITE, mids["a"], HIDDEN)
            calls.append(quant(L["ffn"], qx, sx, HIDDEN))
            if with_lora:  # gate and up share their input: one grouped launch of their middle products
                calls.append(mid_batch_call([(L["ffn"], lora_of(L, "gate")[0], mids["b"], HIDDEN),
                                             (L["ffn"], lora_of(L, "up")[0], mids["c"], HIDDEN)]))
            proj(L, "gate", L["ffn"], qx, sx, gate, dq8.WRITE, mids["b"], HIDDEN, with_mid=False)
            proj(L, "up", L["ffn"], qx, sx, gate, dq8.SWIGLU, mids["c"], HIDDEN, with_mid=False)
            calls.append(quant(gate, qf, sf, FFN_DIM))
            proj(L, "down", gate, qf, sf, resid, dq8.ADD, mids["a"], FFN_DIM)
        return calls

    calls = build(False)
    step_ops = sum(c[3][1] for c in calls)

    def run_step(events=None, calls=calls):
        for i, (kind, fn, a, _) in enumerate(calls):
            if events is not None:
                events[i][0].record(stream)
            st = fn(*a)
            if st != 0:
                raise dq8.Dq8Error(st, fn.__name__)
            if events is not None:
                events[i][1].record(stream)

    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()
    if int(flag.item()) != 0:
        raise RuntimeError("synthetic activations were reported non-finite")
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)

    def timed(fn):
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(args.steps):
            fn()
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / args.steps

    # eager: every call submitted from the host in turn
    ms_eager = timed(run_step)
    # graph: the same calls captured once and replayed (no per-launch host work)
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            run_step()
        for _ in range(args.warmup):
            graph.replay()
        ms_graph = timed(graph.replay)
    ms_step = ms_graph if graph is not None else ms_eager
    # per-launch durations: HIP events around each call, on the launch stream,
    # over as many eager steps again (events in the timed steps would slow the
    # host's submission and add gaps to the step time)
    ev_steps = args.steps
    ev = [[[torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)] for _ in calls]
          for _ in range(ev_steps)]
    for s in range(ev_steps):
        run_step(ev[s])
    torch.cuda.synchronize()
    lin_ms = quant_ms = 0.0
    lin_n = quant_n = 0
    quant_bytes = sum(c[3][0] for c in calls if c[0] == "quant")
    for s in range(ev_steps):
        for i, c in enumerate(calls):
            d = ev[s][i][0].elapsed_time(ev[s][i][1])
            if c[0] == "linear":
                lin_ms += d
                lin_n += 1
            else:
                quant_ms += d
                quant_n += 1
    lin_ops_per_launch = sum(c[3][1] for c in calls if c[0] == "linear") / sum(1 for c in calls if c[0] == "linear")
    lin_avg_ms = lin_ms / lin_n
    achieved = lin_ops_per_launch / (lin_avg_ms * 1e-3) / 1e12
    value = step_ops / (ms_step * 1e-3) / 1e12
    lora = run_lora_stack(args, torch, stream, build, run_step, step_ops, ms_step) if rank > 0 else None

    # release the stack before the skinny workload
    for L in layers:
        for key in ("in", "out", "q", "k", "v", "o", "gate", "up", "down"):
            if key in L:
                L[key].free()
    del layers, calls, ev
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    stacked, skinny = run_skinny(args, torch, dq8, ctx, lib, dev, stream, gen)
    load = run_load(args, torch, dq8, ctx, gen)
    cpu = None if args.no_cpu_baseline else run_cpu_baseline(args, torch, dq8, ctx, dev, gen)
    traffic = load_traffic("linear_wide_stack2048")
    out = {
        "metric": "int8 prefill-projection TOPS (% of i8 MFMA peak); skinny-M HBM GB/s",
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic (seeded; weights N(0,0.02^2) per-row group-64 int8, activations Student-t(3))",
        "config": {
            "workload": "24-layer projection stack, one 2048-token prefill (18 GDN + 6 GQA, each + 2048<->6144 "
                        "SwiGLU FFN), input quantization included",
            "tokens": M,
            "hidden": HIDDEN,
            "ops_per_step": step_ops,
            "frac_of_int8_peak": round(value / PEAK_INT8_TOPS, 4),
            "submission": "hip graph replay of the captured step" if graph is not None else "eager",
            "eager_ms_per_step": round(ms_eager, 4),
            "quantize_ms_per_step": round(quant_ms / ev_steps, 4),
            "quantize_gbs": round(quant_bytes * ev_steps / (quant_ms * 1e-3) / 1e9, 1),
            "projection_ms_per_step": round(lin_ms / ev_steps, 4),
        },
        "roofline": {
            "kernel": "k_linear_wide",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_INT8_TOPS,
            "unit": "TOP/s",
            "frac": round(achieved / PEAK_INT8_TOPS, 4),
            "traffic": traffic,
            "ops_per_launch": lin_ops_per_launch,
            "avg_launch_ms": round(lin_avg_ms, 5),
        },
        "skinny": skinny,
        "questions_stacked": stacked,
        "load": load,
        "lora": lora,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


def run_lora_stack(args, torch, stream, build, run_step, step_ops, base_ms):
    """The same stack with a rank-r FP32 LoRA pair on every projection, as the
    reference's checkpoints carry (weights.rs:420-424): per projection the middle
    product mid = x.A^T (dq8_lora_mid; one dq8_lora_mid_batch launch for the projections
    that share an input, q/k/v and gate/up) and the projection with its adapter."""
    calls = build(True)
    for _ in range(2):
        run_step(calls=calls)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # submitted the same way as the base step it is compared with
    step = lambda: run_step(calls=calls)
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            run_step(calls=calls)
        graph.replay()
        step = graph.replay
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    ev_steps = 3
    ev = [[[torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)] for _ in calls]
          for _ in range(ev_steps)]
    for s in range(ev_steps):
        run_step(ev[s], calls=calls)
    torch.cuda.synchronize()
    mid_ms = sum(ev[s][i][0].elapsed_time(ev[s][i][1]) for s in range(ev_steps)
                 for i, c in enumerate(calls) if c[0] == "mid") / ev_steps
    lin_ms = sum(ev[s][i][0].elapsed_time(ev[s][i][1]) for s in range(ev_steps)
                 for i, c in enumerate(calls) if c[0] == "linear") / ev_steps
    return {
        "workload": f"the stack above with a rank-{args.lora_rank} FP32 LoRA pair on every projection",
        "rank": args.lora_rank,
        "ms_per_step": round(ms_step, 4),
        "tops_base_ops": round(step_ops / (ms_step * 1e-3) / 1e12, 2),
        "overhead_vs_base": round(ms_step / base_ms - 1.0, 4),
        "mid_ms_per_step": round(mid_ms, 4),
        "projection_ms_per_step": round(lin_ms, 4),
    }


def run_skinny_lora(args, torch, dq8, ctx, lib, dev, stream, gen, shapes, copies, acts, launches):
    """The questions of the skinny leg with a rank-r FP32 LoRA pair on every projection: per question the 9
    middle products (one dq8_lora_mid_batch launch, few-rows kernel) and the grouped launch with adapters.  The plain and the
    adapter questions are both captured in a HIP graph and replayed, so host submission of the extra calls is
    not timed."""
    M, rank = args.question_tokens, args.lora_rank
    pairs = [((torch.randn((rank, k), generator=gen, device=dev) * 0.02).contiguous(),
              (torch.randn((n, rank), generator=gen, device=dev) * 0.02).contiguous()) for _, n, k in shapes]
    mids = [[torch.empty((M, rank), dtype=torch.float32, device=dev) for _ in shapes] for _ in acts]
    keep, lora_launches, mid_items = [], [], []
    for qi in range(args.questions):
        ws = copies[qi % len(copies)]
        items = (dq8._Item * len(shapes))()
        mi = (dq8._MidItem * len(shapes))()
        for j, (q, s, o, x) in enumerate(acts[qi]):
            lr = dq8._Lora(mids[qi][j].data_ptr(), pairs[j][1].data_ptr(), rank, 0.5)
            keep.append(lr)
            items[j] = dq8._Item(ws[j].handle, q.data_ptr(), s.data_ptr(), M, None, o.data_ptr(), dq8.ROWS,
                                 dq8.WRITE, ctypes.pointer(lr))
            mi[j] = dq8._MidItem(x.data_ptr(), M, shapes[j][2], pairs[j][0].data_ptr(), rank, mids[qi][j].data_ptr())
        lora_launches.append(items)
        mid_items.append(mi)
    sh = stream.cuda_stream

    def call(st, what):
        if st != 0:
            raise dq8.Dq8Error(st, what)

    def plain():
        for items in launches:
            call(lib.dq8_linear_batch(ctx.handle, items, len(shapes), sh), "dq8_linear_batch")

    def adapters():
        for qi, items in enumerate(lora_launches):
            # the question's 9 middle products in one grouped launch, then the projections
            call(lib.dq8_lora_mid_batch(ctx.handle, mid_items[qi], len(shapes), sh), "dq8_lora_mid_batch")
            call(lib.dq8_linear_batch(ctx.handle, items, len(shapes), sh), "dq8_linear_batch")

    def graph_ms(fn):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        g.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(args.skinny_reps):
            g.replay()
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / (args.skinny_reps * args.questions)

    plain_ms, lora_ms = graph_ms(plain), graph_ms(adapters)
    return {
        "workload": f"the same questions with a rank-{rank} FP32 LoRA pair on every projection (one grouped launch "
                    f"of the 9 middle products + the grouped launch with adapters per question; HIP graph replay)",
        "ms_per_question": round(lora_ms, 5),
        "plain_ms_per_question": round(plain_ms, 5),
        "overhead_vs_plain": round(lora_ms / plain_ms - 1.0, 4),
    }


def run_skinny(args, torch, dq8, ctx, lib, dev, stream, gen):
    """16 questions x M tokens, one grouped launch per question over a layer's projections."""
    M = args.question_tokens
    shapes = [("q", HIDDEN, HIDDEN), ("k", 512, HIDDEN), ("v", 512, HIDDEN), ("o", HIDDEN, HIDDEN),
              ("gdn_in", GDN_IN, HIDDEN), ("gdn_out", HIDDEN, HIDDEN), ("gate", FFN_DIM, HIDDEN),
              ("up", FFN_DIM, HIDDEN), ("down", HIDDEN, FFN_DIM)]
    wbytes = sum(n * k + 4 * n * ((k + 63) // 64) for _, n, k in shapes)
    copies = []
    for _ in range(args.weight_copies):
        copies.append([ctx.weights_from_f32((torch.randn((n, k), generator=gen, device=dev) * 0.02).contiguous())
                       for _, n, k in shapes])
    acts = []
    for _ in range(args.questions):
        per = []
        for _, n, k in shapes:
            x = torch.randn((M, k), generator=gen, device=dev)
            q, s = ctx.quantize(x)
            per.append((q, s, torch.empty((M, n), dtype=torch.float32, device=dev), x))
        acts.append(per)
    launches = []
    for qi in range(args.questions):
        ws = copies[qi % len(copies)]
        items = (dq8._Item * len(shapes))()
        for j, (q, s, o, _) in enumerate(acts[qi]):
            items[j] = dq8._Item(ws[j].handle, q.data_ptr(), s.data_ptr(), M, None, o.data_ptr(), dq8.ROWS,
                                 dq8.WRITE)
        launches.append(items)
    sh = stream.cuda_stream

    def go(evs=None, warm_copy=False):
        for qi, items in enumerate(launches):
            use = launches[0] if warm_copy else items
            if evs is not None:
                evs[qi][0].record(stream)
            st = lib.dq8_linear_batch(ctx.handle, use, len(shapes), sh)
            if st != 0:
                raise dq8.Dq8Error(st, "dq8_linear_batch")
            if evs is not None:
                evs[qi][1].record(stream)

    for _ in range(2):
        go()
    torch.cuda.synchronize()
    reps = args.skinny_reps
    evs = [[[torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)] for _ in launches]
           for _ in range(reps)]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for r in range(reps):
        go(evs[r])
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    launch_ms = sum(evs[r][i][0].elapsed_time(evs[r][i][1]) for r in range(reps) for i in range(len(launches)))
    avg_launch = launch_ms / (reps * len(launches))
    # MALL-resident comparison: the same launch (one weight copy) repeated
    t0.record(stream)
    for _ in range(reps):
        go(warm_copy=True)
    t1.record(stream)
    torch.cuda.synchronize()
    warm_ms = t0.elapsed_time(t1)
    gbs = wbytes * args.questions * reps / (total_ms * 1e-3) / 1e9
    kernel_gbs = wbytes / (avg_launch * 1e-3) / 1e9
    # per question with the launches captured in a HIP graph, like the main step (no host submission between
    # questions); the eager rate above is reported beside it
    lora = run_skinny_lora(args, torch, dq8, ctx, lib, dev, stream, gen, shapes, copies, acts, launches)
    graph_q_ms = lora["plain_ms_per_question"]
    stacked = run_stacked(args, torch, dq8, ctx, lib, dev, stream, gen, shapes, copies, wbytes, graph_q_ms)
    for ws in copies:
        for h in ws:
            h.free()
    return stacked, {
        "workload": f"{args.questions} questions x {M} tokens, one grouped launch per question over q,k,v,o,"
                    f"GDN in/out, FFN gate/up/down ({args.weight_copies} rotating weight copies)",
        "value": round(wbytes / (graph_q_ms * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "submission": "hip graph replay of the question launches",
        "weight_bytes_per_question": wbytes,
        "ms_per_question": graph_q_ms,
        "eager_gbs": round(gbs, 1),
        "eager_ms_per_question": round(total_ms / (reps * args.questions), 5),
        "mall_resident_gbs": round(wbytes * args.questions * reps / (warm_ms * 1e-3) / 1e9, 1),
        "roofline": {
            "kernel": "k_linear_skinny",
            "bound": "hbm",
            "achieved": round(kernel_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / PEAK_HBM_GBS, 4),
            "traffic": load_traffic("linear_skinny_questions24"),
            "bytes_per_launch": wbytes,
            "avg_launch_ms": round(avg_launch, 5),
        },
        "lora": lora,
    }


def run_stacked(args, torch, dq8, ctx, lib, dev, stream, gen, shapes, copies, wbytes, per_question_ms):
    """The same questions continued layer by layer: every question's token rows
    stacked into one projection launch per layer set (M = questions x tokens),
    so a layer's weights are read once for all questions.  Weight copies rotate
    per launch as in the per-question schedule."""
    M = args.questions * args.question_tokens
    sets = []
    keep = []
    for ws in copies:
        items = (dq8._Item * len(shapes))()
        for j, (_, n, k) in enumerate(shapes):
            q, s = ctx.quantize(torch.randn((M, k), generator=gen, device=dev))
            o = torch.empty((M, n), dtype=torch.float32, device=dev)
            keep += [q, s, o]
            items[j] = dq8._Item(ws[j].handle, q.data_ptr(), s.data_ptr(), M, None, o.data_ptr(), dq8.ROWS,
                                 dq8.WRITE)
        sets.append(items)
    sh = stream.cuda_stream

    def go(i):
        st = lib.dq8_linear_batch(ctx.handle, sets[i % len(sets)], len(shapes), sh)
        if st != 0:
            raise dq8.Dq8Error(st, "dq8_linear_batch")

    for i in range(len(sets)):
        go(i)
    torch.cuda.synchronize()
    reps = 10 * len(sets)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(reps):
        go(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    ops = sum(2 * M * n * k for _, n, k in shapes)
    del keep
    return {
        "workload": f"{args.questions} questions x {args.question_tokens} tokens stacked into one {M}-row launch per "
                    f"layer set (q,k,v,o, GDN in/out, FFN gate/up/down; {len(copies)} rotating weight copies)",
        "ms_per_layer_set": round(ms, 5),
        "ms_per_question": round(ms / args.questions, 5),
        "tops": round(ops / (ms * 1e-3) / 1e12, 1),
        "weight_gbs": round(wbytes / (ms * 1e-3) / 1e9, 1),
        "speedup_vs_per_question_launches": round(per_question_ms / (ms / args.questions), 2),
    }


def run_load(args, torch, dq8, ctx, gen):
    """Weight load path: one layer set's projections (the skinny leg's shapes) as
    BF16 tensors of one safetensors file, read by dq8_st_load_weights into
    quantized, repacked device weights (file -> pinned staging -> device decode,
    check, quantize, repack).  The file is written first, so it is read from
    the page cache: this is the host-memory-to-weights rate, not a disk rate."""
    import json as _json
    import struct as _struct
    import tempfile

    shapes = [("q", HIDDEN, HIDDEN), ("k", 512, HIDDEN), ("v", 512, HIDDEN), ("o", HIDDEN, HIDDEN),
              ("gdn_in", GDN_IN, HIDDEN), ("gdn_out", HIDDEN, HIDDEN), ("gate", FFN_DIM, HIDDEN),
              ("up", FFN_DIM, HIDDEN), ("down", HIDDEN, FFN_DIM)]
    header, blobs, off = {}, [], 0
    for name, n, k in shapes:
        t = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).to(torch.bfloat16).cpu()
        b = t.view(torch.int16).numpy().tobytes()
        header[f"layers.0.{name}_proj.weight"] = {"dtype": "BF16", "shape": [n, k], "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    text = _json.dumps(header).encode()
    fd, path = tempfile.mkstemp(suffix=".safetensors")
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(_struct.pack("<Q", len(text)) + text + b"".join(blobs))
        del blobs
        times = []
        for _ in range(3):
            with dq8.SafeTensors(path) as st:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                ws = [st.load_weights(ctx, name) for name in st.names]
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
                for w in ws:
                    w.free()
    finally:
        os.unlink(path)
    best = min(times)
    return {
        "workload": "one layer set's 9 projection weights (q,k,v,o, GDN in/out, FFN gate/up/down) as BF16 in one "
                    "safetensors file (page cache) -> quantized device weights",
        "file_bytes": off,
        "ms": round(best * 1e3, 2),
        "gbs": round(off / best / 1e9, 2),
    }


def run_cpu_baseline(args, torch, dq8, ctx, dev, gen):
    """The oracle (C restatement of the reference's x86 int8 path: per-projection
    input quantization + per-column scalar group dots, threads over columns)
    on the first GDN layer + its FFN for a bounded number of token rows."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import dq8o

    threads = max(1, min(16, os.cpu_count() or 1))
    rng = np.random.default_rng(5)
    shapes = [("gdn_in", GDN_IN, HIDDEN), ("gdn_out", HIDDEN, HIDDEN), ("gate", FFN_DIM, HIDDEN),
              ("up", FFN_DIM, HIDDEN), ("down", HIDDEN, FFN_DIM)]
    ws = {}
    for name, n, k in shapes:
        h = ctx.weights_from_f32((torch.randn((n, k), generator=gen, device=dev) * 0.02).contiguous())
        v, s = h.export()
        torch.cuda.synchronize()
        ws[name] = (v.cpu().numpy(), s.cpu().numpy())
        h.free()

    def layer(rows):
        x = rng.standard_normal((rows, HIDDEN)).astype(np.float32)
        t = time.perf_counter()
        dq8o.linear(x, *ws["gdn_in"], threads=threads)
        dq8o.linear(x, *ws["gdn_out"], threads=threads)
        g = dq8o.linear(x, *ws["gate"], threads=threads)
        g = dq8o.linear(x, *ws["up"], result=g, epilogue=2, threads=threads)
        dq8o.linear(g, *ws["down"], result=x, epilogue=1, threads=threads)
        return time.perf_counter() - t

    ops_per_row = 2 * sum(n * k for _, n, k in shapes)
    rows = 16
    secs = layer(rows)
    # size the sample to about cpu_seconds of work (per-row cost measured on the previous sample)
    while secs < 0.5 * args.cpu_seconds and rows < 2048:
        rows = int(max(rows + 1, min(2048, rows * args.cpu_seconds / max(secs, 1e-6))))
        secs = layer(rows)
    # a whole 2048-token layer shorter than the target: time that many layers back to back
    n_layers = 1
    if secs < 0.5 * args.cpu_seconds:
        n_layers = max(1, int(round(args.cpu_seconds / secs)))
        secs = sum(layer(rows) for _ in range(n_layers))
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(ops_per_row * rows * n_layers / secs / 1e12, 5),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"{n_layers} x (GDN layer + FFN projections: in 2048->8224, out, gate/up SwiGlu, re-quantized "
                  f"down) for {rows} of the 2048 tokens, quantization included; {secs:.1f} s on {cpu_model}",
    }


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic_<name>.json), or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


if __name__ == "__main__":
    main()
