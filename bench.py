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
the launch stream (launches queued behind a GPU lead, so that the events time
the kernels rather than their submission from the host).

Further legs, each timed on its own: "config1" (one 128 x 2048 -> 2048 linear,
seed 0), "config2" (the 512-token SwiGLU FFN block through dq8_ffn), "config3"
(one layer's projections at 4096 tokens with 1% of the channels x20),
"reference_benchmarks" (the reference's own timed benchmarks, tensor.rs:553-603
and weights.rs:580-631, on their formula inputs, next to its published times)
and "host_round_trip" (pinned host buffers in and out around the device work,
as a caller with host-resident activations pays).

"cpu_baseline" times the oracle (the C restatement of the reference's x86
path) on a bounded sample of the stack's workload, with all usable host cores
(at most 16) and with one, median of 5 runs.  The same leg recomputes sampled
rows of every timed GPU workload above with the oracle and compares them bit
for bit ("checks"); a mismatch fails the run.  With --no-cpu-baseline neither
runs.
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
HIDDEN, FFN_DIM, GDN_IN, KV_DIM = 2048, 6144, 4 * 2048 + 2 * 16, 4 * 128
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
    p.add_argument("--only", choices=["stack", "skinny"],
                   help="run one leg only (no CPU baseline) and print its figures: for kernel profiles")
    p.add_argument("--no-graph", action="store_true", help="time eager submission only (no HIP graph replay)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--lora-rank", type=int, default=16,
                   help="rank of the LoRA adapters of the stack's second pass (0: skip it)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device copy (for rocprof counter calibration)")
    return p.parse_args()


_SLEEP_CYCLES_PER_MS = None


def gpu_lead(torch, stream, ms):
    """Queue about ms of GPU work (torch's spin kernel) on the stream ahead of evented launches: the host's
    submissions then run ahead of the GPU, so each event pair brackets a kernel that was already queued, not
    the host's submission of it (which shows for kernels of a few tens of microseconds)."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 16)
        a.record(stream)
        torch.cuda._sleep(1 << 22)
        b.record(stream)
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = (1 << 22) / max(a.elapsed_time(b), 1e-3)
    torch.cuda._sleep(int(ms * _SLEEP_CYCLES_PER_MS))


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
    # a second stream (default priority) for the LoRA leg's middle products that run beside a quantize
    stream2 = torch.cuda.Stream(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    if args.only == "skinny":
        args.no_cpu_baseline = True
        stacked, skinny = run_skinny(args, torch, dq8, ctx, lib, dev, stream, gen)
        print(json.dumps({"skinny": skinny, "questions_stacked": stacked}))
        return

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
            L["k"] = weights(KV_DIM, HIDDEN)
            L["v"] = weights(KV_DIM, HIDDEN)
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
    bufs = {"mixer": mixer_out, "k": k_out, "v": v_out, "proj": proj_out, "gate": gate, "resid": resid}

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

    def mid_call(x, a, mid, k, side=False):
        return ("mid2" if side else "mid", lib.dq8_lora_mid,
                (ctx.handle, x.data_ptr(), M, k, a.data_ptr(), rank, mid.data_ptr(),
                 stream2.cuda_stream if side else sh), (0, 2 * M * k * rank))

    def mid_batch_call(entries, side=False):
        """The middle products of projections that share an input, in one dq8_lora_mid_batch call:
        entries = [(x, A, mid, k)]."""
        arr = (dq8._MidItem * len(entries))()
        for i, (x, a, mid, k) in enumerate(entries):
            arr[i] = dq8._MidItem(x.data_ptr(), M, k, a.data_ptr(), rank, mid.data_ptr())
        keep.append(arr)
        return ("mid2" if side else "mid", lib.dq8_lora_mid_batch,
                (ctx.handle, arr, len(entries), stream2.cuda_stream if side else sh),
                (0, sum(2 * M * k * rank for _, _, _, k in entries)))

    def fork():
        """stream2 waits for everything queued on the main stream so far."""
        ev = torch.cuda.Event()

        def f():
            ev.record(stream)
            stream2.wait_event(ev)
            return 0
        return ("sync", f, (), (0, 0))

    def join():
        """The main stream waits for everything queued on stream2 so far."""
        ev = torch.cuda.Event()

        def f():
            ev.record(stream2)
            stream.wait_event(ev)
            return 0
        return ("sync", f, (), (0, 0))

    def beside_quant(mid, q):
        """A middle product of x on stream2 while the main stream quantizes x: both only read x."""
        return [fork(), mid, q, join()]

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

    layer_bounds = []  # [start, end) of each layer's calls in the last build

    def build(with_lora):
        calls = []
        layer_bounds.clear()

        def proj(L, name, x, q, s, out, ep, mid, k, with_mid=True):
            if with_lora:
                calls.extend(lora_linear(L, name, x, q, s, out, ep, mid, k, with_mid))
            else:
                calls.append(linear(L[name], q, s, out, ep))

        for L in layers:
            layer_bounds.append(len(calls))
            if with_lora and L["kind"] == "gdn":
                calls.extend(beside_quant(mid_call(L["x"], lora_of(L, "in")[0], mids["a"], HIDDEN, side=True),
                                          quant(L["x"], qx, sx, HIDDEN)))
                proj(L, "in", L["x"], qx, sx, mixer_out, dq8.WRITE, mids["a"], HIDDEN, with_mid=False)
            elif L["kind"] == "gdn":
                calls.append(quant(L["x"], qx, sx, HIDDEN))
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
                if shared:  # q, k and v share their input: one grouped launch of their middle products
                    calls.extend(beside_quant(mid_batch_call(shared, side=True), quant(L["x"], qx, sx, HIDDEN)))
                else:
                    calls.append(quant(L["x"], qx, sx, HIDDEN))
                flops = sum(2 * M * L[n].n * L[n].k for n in ("q", "k", "v"))
                calls.append(("linear", lib.dq8_linear_batch, (ctx.handle, items, 3, sh), (0, flops)))
            mixer = "out" if L["kind"] == "gdn" else "o"
            if with_lora:
                calls.extend(beside_quant(mid_call(L["mix"], lora_of(L, mixer)[0], mids["a"], HIDDEN, side=True),
                                          quant(L["mix"], qx, sx, HIDDEN)))
            else:
                calls.append(quant(L["mix"], qx, sx, HIDDEN))
            proj(L, mixer, L["mix"], qx, sx, proj_out, dq8.WRITE, mids["a"], HIDDEN, with_mid=False)
            # gate and up in one launch storing h and its quantization for down (qwen.rs:489-491),
            # each with its adapter when the leg has them, then down Add
            ops = sum(2 * M * L[n].n * L[n].k for n in ("gate", "up"))
            lg = lu = None
            if not with_lora:
                calls.append(quant(L["ffn"], qx, sx, HIDDEN))
            else:  # gate and up share their input: one grouped launch of their middle products
                calls.extend(beside_quant(mid_batch_call([(L["ffn"], lora_of(L, "gate")[0], mids["b"], HIDDEN),
                                                          (L["ffn"], lora_of(L, "up")[0], mids["c"], HIDDEN)],
                                                         side=True),
                                          quant(L["ffn"], qx, sx, HIDDEN)))
                lg = dq8._Lora(mids["b"].data_ptr(), lora_of(L, "gate")[1].data_ptr(), rank, 2.0)
                lu = dq8._Lora(mids["c"].data_ptr(), lora_of(L, "up")[1].data_ptr(), rank, 2.0)
                keep.extend((lg, lu))
                lg, lu = ctypes.byref(lg), ctypes.byref(lu)
            calls.append(("linear", lib.dq8_ffn_gate_up_lora, (ctx.handle, L["gate"].handle, L["up"].handle,
                                                               qx.data_ptr(), sx.data_ptr(), M, None, None, lg, lu,
                                                               gate.data_ptr(), qf.data_ptr(), sf.data_ptr(),
                                                               flag.data_ptr(), sh), (0, ops)))
            proj(L, "down", gate, qf, sf, resid, dq8.ADD, mids["a"], FFN_DIM)
        layer_bounds.append(len(calls))
        return calls

    calls = build(False)
    bounds = list(layer_bounds)
    step_ops = sum(c[3][1] for c in calls)

    def run_step(events=None, calls=calls):
        for i, (kind, fn, a, _) in enumerate(calls):
            on = stream2 if kind == "mid2" else stream
            if events is not None:
                events[i][0].record(on)
            st = fn(*a)
            if st != 0:
                raise dq8.Dq8Error(st, fn.__name__)
            if events is not None:
                events[i][1].record(on)

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
    gpu_lead(torch, stream, 5.0)
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
    # the step's quantize calls alone, captured in one graph and replayed as the step is: their share of the
    # replayed step (the evented figures above include each eager call's launch gap)
    quant_graph_ms = None
    if graph is not None:
        qcalls = [c for c in calls if c[0] == "quant"]
        qgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(qgraph, stream=stream):
            run_step(calls=qcalls)
        for _ in range(args.warmup):
            qgraph.replay()
        quant_graph_ms = timed(qgraph.replay)
    # the same inputs through one of torch's own elementwise kernels that reads each input once and writes a
    # quarter of its size (the quantizer's traffic, less the scales), replayed the same way: what a launch that
    # moves these bytes reaches
    quant_torch_ms = None
    if graph is not None:
        qins = [L[key] for L in layers for key in ("x", "mix", "ffn")]
        sink = torch.empty((M, HIDDEN // 4), dtype=torch.float32, device=dev)
        tgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(tgraph, stream=stream):
            for x in qins:
                torch.mul(x[:, ::4], 1.0, out=sink)
        for _ in range(args.warmup):
            tgraph.replay()
        quant_torch_ms = timed(tgraph.replay)
        quant_torch_bytes = sum(x.numel() * 4 + sink.numel() * 4 for x in qins)
    lin_ops_per_launch = sum(c[3][1] for c in calls if c[0] == "linear") / sum(1 for c in calls if c[0] == "linear")
    lin_avg_ms = lin_ms / lin_n
    achieved = lin_ops_per_launch / (lin_avg_ms * 1e-3) / 1e12
    value = step_ops / (ms_step * 1e-3) / 1e12
    if args.only == "stack":
        args.no_cpu_baseline = True
    lora = run_lora_stack(args, torch, stream, build, run_step, step_ops, ms_step) \
        if rank > 0 and args.only is None else None
    # outputs of the first (GDN) and last (GQA) layer of the timed step, run once more on their own from a zero
    # residual, kept for the oracle check of the cpu_baseline leg
    stack_checks = [capture_layer(torch, dq8, layers, calls[bounds[i]:bounds[i + 1]], i, M, bufs)
                    for i in (0, len(layers) - 1)] \
        if not args.no_cpu_baseline else []

    # release the stack before the skinny workload
    for L in layers:
        for key in ("in", "out", "q", "k", "v", "o", "gate", "up", "down"):
            if key in L:
                L[key].free()
    del layers, calls, ev
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    stacked = skinny = load = config1 = config2 = config3 = reference = round_trip = None
    if args.only is None:
        stacked, skinny = run_skinny(args, torch, dq8, ctx, lib, dev, stream, gen)
        load = run_load(args, torch, dq8, ctx, gen)
        keep_checks = not args.no_cpu_baseline
        config1 = run_config1(args, torch, dq8, ctx, lib, dev, stream, keep_checks)
        config2 = run_config2(args, torch, dq8, ctx, lib, dev, stream, keep_checks)
        config3 = run_config3(args, torch, dq8, ctx, lib, dev, stream, keep_checks)
        reference = run_reference_benchmarks(args, torch, dq8, ctx, lib, dev, stream, keep_checks)
        round_trip = run_host_round_trip(args, torch, dq8, ctx, lib, dev, stream)
    cpu = None
    if not args.no_cpu_baseline:
        checks = {"stack_layer_0": stack_checks[0], "stack_layer_23": stack_checks[1],
                  "config1": config1.pop("_check"), "config2": config2.pop("_check"),
                  "config3": config3.pop("_check")}
        for leg in reference.values():
            for key in list(leg):
                if key.startswith("_check"):
                    checks[key[len("_check_"):]] = leg.pop(key)
        cpu = run_cpu_baseline(args, torch, dq8, ctx, dev, gen, checks)
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
            "quantize_ms_per_step": round(quant_graph_ms if quant_graph_ms else quant_ms / ev_steps, 4),
            "quantize_gbs": round(quant_bytes / ((quant_graph_ms if quant_graph_ms else quant_ms / ev_steps) * 1e-3)
                                  / 1e9, 1),
            "quantize_timing": "the step's quantize calls replayed alone in a HIP graph" if quant_graph_ms else
                               "HIP events around each eager call",
            "quantize_ms_per_step_events": round(quant_ms / ev_steps, 4),
            "quantize_torch_same_bytes_gbs": round(quant_torch_bytes / (quant_torch_ms * 1e-3) / 1e9, 1)
            if quant_torch_ms else None,
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
        "config1": config1,
        "config2": config2,
        "config3": config3,
        "reference_benchmarks": reference,
        "host_round_trip": round_trip,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    if cpu is not None and not cpu["checks_passed"]:
        print("bench: a sampled oracle check of the timed workloads failed: " +
              json.dumps({k: v for k, v in cpu["checks"].items() if v != "bit-exact"}), file=sys.stderr)
        sys.exit(1)


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
                 for i, c in enumerate(calls) if c[0] in ("mid", "mid2")) / ev_steps
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
    shapes = [("q", HIDDEN, HIDDEN), ("k", KV_DIM, HIDDEN), ("v", KV_DIM, HIDDEN), ("o", HIDDEN, HIDDEN),
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

    def go(warm_copy=False):
        for items in launches:
            st = lib.dq8_linear_batch(ctx.handle, launches[0] if warm_copy else items, len(shapes), sh)
            if st != 0:
                raise dq8.Dq8Error(st, "dq8_linear_batch")

    for _ in range(2):
        go()
    torch.cuda.synchronize()
    reps = args.skinny_reps
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for r in range(reps):
        go()
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    # per-launch duration: the same launches again, queued behind a GPU lead so that they run back to back
    # (the eager rate above includes the host's submission of each), between one pair of events: every call
    # is one k_linear_skinny launch, so the region's time over the launch count is the kernel's mean duration.
    # (An event pair around each launch adds ~2.7 us of event processing to a ~20 us launch.)
    gpu_lead(torch, stream, 10.0)
    t0.record(stream)
    for r in range(reps):
        go()
    t1.record(stream)
    torch.cuda.synchronize()
    avg_launch = t0.elapsed_time(t1) / (reps * len(launches))
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
    # two questions in flight: the questions are independent (each continues from the shared prefix), so the
    # graph alternates their launches over two streams; one launch's ramp and tail overlap the other's stream
    side = torch.cuda.Stream(dev)

    def go_two():
        ev = torch.cuda.Event()
        ev.record(stream)
        side.wait_event(ev)
        for qi, items in enumerate(launches):
            st = lib.dq8_linear_batch(ctx.handle, items, len(shapes), (side if qi % 2 else stream).cuda_stream)
            if st != 0:
                raise dq8.Dq8Error(st, "dq8_linear_batch")
        back = torch.cuda.Event()
        back.record(side)
        stream.wait_event(back)

    go_two()
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=stream):
        go_two()
    g2.replay()
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(reps):
        g2.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    two_q_ms = t0.elapsed_time(t1) / (reps * args.questions)
    # the same projections as a model issues them, one launch per input: x (q, k, v, GDN in), the mixer outputs
    # (o, GDN out), the FFN input (gate, up), h (down); graph-replayed like the grouped launch
    parts = [[0, 1, 2, 4], [3, 5], [6, 7], [8]]
    split = []
    for items in launches:
        for idx in parts:
            sub = (dq8._Item * len(idx))()
            for j, i in enumerate(idx):
                sub[j] = items[i]
            split.append(sub)

    def go_split():
        for sub in split:
            st = lib.dq8_linear_batch(ctx.handle, sub, len(sub), sh)
            if st != 0:
                raise dq8.Dq8Error(st, "dq8_linear_batch")

    go_split()
    torch.cuda.synchronize()
    sg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(sg, stream=stream):
        go_split()
    sg.replay()
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(reps):
        sg.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    split_q_ms = t0.elapsed_time(t1) / (reps * args.questions)
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
        "two_in_flight": {
            "workload": "the same question launches alternating over two streams of one HIP graph (two questions "
                        "in flight; the 5 rotating weight copies keep their bytes distinct)",
            "ms_per_question": round(two_q_ms, 5),
            "gbs": round(wbytes / (two_q_ms * 1e-3) / 1e9, 1),
            "frac": round(wbytes / (two_q_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        },
        "layer_order_launches": {
            "workload": "the same questions, each as 4 launches in a layer's order: q,k,v + GDN in (x), o + GDN out "
                        "(mixer outputs), gate + up (FFN input), down (h); HIP graph replay",
            "ms_per_question": round(split_q_ms, 5),
            "gbs": round(wbytes / (split_q_ms * 1e-3) / 1e9, 1),
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

    shapes = [("q", HIDDEN, HIDDEN), ("k", KV_DIM, HIDDEN), ("v", KV_DIM, HIDDEN), ("o", HIDDEN, HIDDEN),
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


def sample_rows(m, count, seed):
    """count sorted distinct row indices of [0, m), always holding the first and the last row."""
    import numpy as np

    rows = np.random.default_rng(seed).choice(m, size=min(count, m), replace=False)
    rows[0], rows[-1] = 0, m - 1
    return np.unique(rows)


def host_rows(torch, t, rows):
    torch.cuda.synchronize()
    return t[torch.as_tensor(rows, device=t.device)].cpu().numpy()


def exported(torch, w):
    v, s = w.export()
    torch.cuda.synchronize()
    return v.cpu().numpy(), s.cpu().numpy()


def timed_calls(torch, stream, fn, reps):
    """Device time per call of fn() over reps back-to-back calls on stream (events around the batch), in ms."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(reps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def ok(st, what):
    if st != 0:
        import dq8

        raise dq8.Dq8Error(st, what)


def capture_layer(torch, dq8, layers, calls, i, M, bufs):
    """Layer i of the stack (its calls of the timed step: quantize, in / q,k,v, quantize, out / o, quantize,
    the FFN chain: gate and up (SwiGlu) storing h and its quantization, down (Add)) run once more from a zero
    residual; sampled rows of its inputs, outputs and weights are kept for the oracle."""
    L = layers[i]
    bufs["resid"].zero_()
    for _, fn, a, _ in calls:
        ok(fn(*a), fn.__name__)
    torch.cuda.synchronize()
    rows = sample_rows(M, 16, 100 + i)
    x, mix, ffn = (host_rows(torch, L[key], rows) for key in ("x", "mix", "ffn"))
    items = []
    if L["kind"] == "gdn":
        items.append(("linear", x, *exported(torch, L["in"]), None, 0, host_rows(torch, bufs["mixer"], rows)))
        items.append(("linear", mix, *exported(torch, L["out"]), None, 0, host_rows(torch, bufs["proj"], rows)))
    else:
        q_view = bufs["mixer"].view(-1)[:M * HIDDEN].view(M, HIDDEN)
        for name, buf in (("q", q_view), ("k", bufs["k"]), ("v", bufs["v"])):
            items.append(("linear", x, *exported(torch, L[name]), None, 0, host_rows(torch, buf, rows)))
        items.append(("linear", mix, *exported(torch, L["o"]), None, 0, host_rows(torch, bufs["proj"], rows)))
    h = host_rows(torch, bufs["gate"], rows)
    items.append(("ffn_h", ffn, exported(torch, L["gate"]), exported(torch, L["up"]), h))
    items.append(("linear", h, *exported(torch, L["down"]), np_zeros(len(rows), HIDDEN), 1,
                  host_rows(torch, bufs["resid"], rows)))
    return {"what": f"layer {i} ({L['kind']}) of the timed step, {len(rows)} sampled rows", "items": items}


def np_zeros(*shape):
    import numpy as np

    return np.zeros(shape, np.float32)


def run_config1(args, torch, dq8, ctx, lib, dev, stream, keep):
    """Single linear M=128, K=N=2048, weights N(0, 0.02^2), activations N(0, 1), seed 0: quantize + project."""
    import numpy as np

    M, K, N = 128, HIDDEN, HIDDEN
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    h = ctx.weights_from_f32(torch.from_numpy(w).to(dev))
    xd = torch.from_numpy(x).to(dev)
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    s = torch.empty((M, K // 64), dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    sh = stream.cuda_stream
    quant = lambda: ok(lib.dq8_quantize(ctx.handle, xd.data_ptr(), M, K, q.data_ptr(), s.data_ptr(), flag.data_ptr(),
                                        sh), "dq8_quantize")
    lin = lambda: ok(lib.dq8_linear(ctx.handle, h.handle, q.data_ptr(), s.data_ptr(), M, None, out.data_ptr(),
                                    dq8.ROWS, dq8.WRITE, sh), "dq8_linear")
    ms = timed_calls(torch, stream, lambda: (quant(), lin()), 50)
    ms_lin = timed_calls(torch, stream, lin, 50)
    ops = 2 * M * N * K
    gemm_bytes = N * K + 4 * N * (K // 64) + M * K + 4 * M * (K // 64) + 4 * M * N
    res = {
        "workload": "single int8 linear, 128 tokens x 2048 -> 2048, seed 0 (weights N(0,0.02^2), x N(0,1)); "
                    "quantize + project, back-to-back calls",
        "ms": round(ms, 5), "tops": round(ops / (ms * 1e-3) / 1e12, 2),
        "projection_ms": round(ms_lin, 5), "projection_tops": round(ops / (ms_lin * 1e-3) / 1e12, 2),
        "projection_gbs": round(gemm_bytes / (ms_lin * 1e-3) / 1e9, 1),
    }
    res["_check"] = {"what": "all 128 rows", "items": [("linear_w", x, w, None, 0, host_rows(torch, out, np.arange(M)))]} \
        if keep else None
    h.free()
    return res


def run_config2(args, torch, dq8, ctx, lib, dev, stream, keep):
    """SwiGLU FFN block for a 512-token prompt (dq8_ffn: gate Write, up SwiGlu, h re-quantized, down Add)."""
    import numpy as np

    M = 512
    rng = np.random.default_rng(2)
    ws = {nm: (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
          for nm, n, k in (("gate", FFN_DIM, HIDDEN), ("up", FFN_DIM, HIDDEN), ("down", HIDDEN, FFN_DIM))}
    x = rng.standard_normal((M, HIDDEN)).astype(np.float32)
    W = {nm: ctx.weights_from_f32(torch.from_numpy(w).to(dev)) for nm, w in ws.items()}
    xd = torch.from_numpy(x).to(dev)
    q = torch.empty((M, HIDDEN), dtype=torch.int8, device=dev)
    s = torch.empty((M, HIDDEN // 64), dtype=torch.float32, device=dev)
    hbuf = torch.empty((M, FFN_DIM), dtype=torch.float32, device=dev)
    resid = torch.zeros((M, HIDDEN), dtype=torch.float32, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)

    def step():
        ok(lib.dq8_quantize(ctx.handle, xd.data_ptr(), M, HIDDEN, q.data_ptr(), s.data_ptr(), flag.data_ptr(),
                            stream.cuda_stream), "dq8_quantize")
        ctx.ffn(W["gate"], W["up"], W["down"], q, s, resid, h=hbuf, nonfinite=flag)

    ms = timed_calls(torch, stream, step, 30)
    ops = 2 * M * (2 * FFN_DIM * HIDDEN + HIDDEN * FFN_DIM)
    res = {
        "workload": "SwiGLU FFN block, 512 tokens: gate/up 2048->6144, silu(gate)*up, re-quantized, down 6144->2048 "
                    "Add; seed 2; input quantization included (dq8_quantize + dq8_ffn)",
        "ms": round(ms, 5), "tops": round(ops / (ms * 1e-3) / 1e12, 2),
        "weight_gbs": round(3 * FFN_DIM * HIDDEN * (1 + 4 / 64) / (ms * 1e-3) / 1e9, 1),
    }
    check = None
    if keep:
        resid.zero_()
        step()
        rows = sample_rows(M, 32, 2)
        h = host_rows(torch, hbuf, rows)
        check = {"what": f"{len(rows)} sampled rows of h and the residual", "items": [
            ("ffn_h_w", x[rows], ws["gate"], ws["up"], h),
            ("linear_w", h, ws["down"], np_zeros(len(rows), HIDDEN), 1, host_rows(torch, resid, rows))]}
    res["_check"] = check
    for w in W.values():
        w.free()
    return res


def run_config3(args, torch, dq8, ctx, lib, dev, stream, keep):
    """One layer's projection set at the 4096-token window with 1% of the channels x20: GQA q/k/v (one grouped
    launch) and o, Gated DeltaNet in (q,k,v,z + b,a) and out, each input quantized."""
    import numpy as np

    M = 4096
    rng = np.random.default_rng(3)

    def outliers():
        a = rng.standard_normal((M, HIDDEN)).astype(np.float32)
        a[:, rng.choice(HIDDEN, size=HIDDEN // 100, replace=False)] *= np.float32(20.0)
        return a

    shapes = [("q", HIDDEN), ("k", 512), ("v", 512), ("o", HIDDEN), ("gdn_in", GDN_IN), ("gdn_out", HIDDEN)]
    ws = {nm: (rng.standard_normal((n, HIDDEN)) * 0.02).astype(np.float32) for nm, n in shapes}
    xs = {"x": outliers(), "attn": outliers(), "rec": outliers()}
    src = {"q": "x", "k": "x", "v": "x", "gdn_in": "x", "o": "attn", "gdn_out": "rec"}
    W = {nm: ctx.weights_from_f32(torch.from_numpy(w).to(dev)) for nm, w in ws.items()}
    X = {k: torch.from_numpy(v).to(dev) for k, v in xs.items()}
    Q = {k: (torch.empty((M, HIDDEN), dtype=torch.int8, device=dev),
             torch.empty((M, HIDDEN // 64), dtype=torch.float32, device=dev)) for k in xs}
    out = {nm: torch.empty((M, n), dtype=torch.float32, device=dev) for nm, n in shapes}
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    sh = stream.cuda_stream
    qkv = (dq8._Item * 3)()
    for i, nm in enumerate(("q", "k", "v")):
        qkv[i] = dq8._Item(W[nm].handle, Q["x"][0].data_ptr(), Q["x"][1].data_ptr(), M, None, out[nm].data_ptr(),
                           dq8.ROWS, dq8.WRITE)

    def step():
        for k in xs:
            ok(lib.dq8_quantize(ctx.handle, X[k].data_ptr(), M, HIDDEN, Q[k][0].data_ptr(), Q[k][1].data_ptr(),
                                flag.data_ptr(), sh), "dq8_quantize")
            if k == "x":
                ok(lib.dq8_linear_batch(ctx.handle, qkv, 3, sh), "dq8_linear_batch")
                nms = ("gdn_in",)
            else:
                nms = ("o",) if k == "attn" else ("gdn_out",)
            for nm in nms:
                ok(lib.dq8_linear(ctx.handle, W[nm].handle, Q[k][0].data_ptr(), Q[k][1].data_ptr(), M, None,
                                  out[nm].data_ptr(), dq8.ROWS, dq8.WRITE, sh), "dq8_linear")

    ms = timed_calls(torch, stream, step, 20)
    ops = sum(2 * M * n * HIDDEN for _, n in shapes)
    res = {
        "workload": "one layer's projections at the 4096-token window: GQA q 2048->2048, k/v 2048->512 (grouped), "
                    "o 2048->2048; Gated DeltaNet in 2048->8224, out 2048->2048; inputs N(0,1) with 1% of the "
                    "channels x20; seed 3; the 3 input quantizations included",
        "ms": round(ms, 5), "tops": round(ops / (ms * 1e-3) / 1e12, 2),
        "frac_of_int8_peak": round(ops / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
    }
    check = None
    if keep:
        torch.cuda.synchronize()
        rows = sample_rows(M, 16, 3)
        check = {"what": f"{len(rows)} sampled rows of each projection", "items": [
            ("linear_w", xs[src[nm]][rows], ws[nm], None, 0, host_rows(torch, out[nm], rows)) for nm, _ in shapes]}
    res["_check"] = check
    for w in W.values():
        w.free()
    return res


def run_reference_benchmarks(args, torch, dq8, ctx, lib, dev, stream, keep):
    """The reference's own timed benchmarks on their formula inputs, through dq8_apply (quantization included,
    as in their timed region), next to the numbers the reference publishes for them (ARM64 CI runner, NEON SDOT,
    4 workers, mean of 3; docs/lambda.md)."""
    import numpy as np

    sh = stream.cuda_stream
    res = {}
    # tensor.rs:553-603 benchmark_int8_projections: 2048x2048, values ((i*71 % 255) - 127) as u8, scales 1/127,
    # x = ((i*43 % 255) - 127)/127, rows 1 / 32 / 128, int8 compute
    K = N = 2048
    values = ((np.arange(N * K, dtype=np.int64) * 71 % 255).astype(np.int16) - 127).astype(np.uint8).reshape(N, K)
    scales = np.full((N, K // 64), np.float32(1.0) / np.float32(127.0), np.float32)
    h = ctx.weights_from_quantized(torch.from_numpy(values).to(dev), torch.from_numpy(scales).to(dev))
    published = {1: 0.097, 32: 1.866, 128: 7.220}
    leg = {"workload": "tensor.rs:553-603 benchmark_int8_projections: 2048x2048 int8 compute, formula inputs, "
                       "quantization included (dq8_apply), back-to-back calls", "rows": {}}
    for rows in (1, 32, 128):
        x = ((np.arange(rows * K, dtype=np.int64) * 43 % 255).astype(np.float32) - np.float32(127.0)) / \
            np.float32(127.0)
        xd = torch.from_numpy(x.reshape(rows, K)).to(dev)
        out = torch.empty((rows, N), dtype=torch.float32, device=dev)
        ms = timed_calls(torch, stream, lambda: ok(lib.dq8_apply(ctx.handle, h.handle, xd.data_ptr(), rows, None, None,
                                                                 out.data_ptr(), dq8.ROWS, dq8.WRITE, sh),
                                                   "dq8_apply"), 50)
        leg["rows"][str(rows)] = {"ms": round(ms, 5), "gops": round(2 * rows * N * K / (ms * 1e-3) / 1e9, 1),
                                  "published_arm_ms": published[rows],
                                  "speedup_vs_published": round(published[rows] / ms, 1)}
        if keep:
            leg[f"_check_int8_projections_rows{rows}"] = {"what": f"{rows} rows, all outputs", "items": [
                ("linear", x.reshape(rows, K), values, scales, None, 0, host_rows(torch, out, np.arange(rows)))]}
    h.free()
    res["int8_projections"] = leg
    # weights.rs:580-631 benchmark_fused_projection: 2048 -> 6144 int8 compute + rank-16 LoRA (scale 0.5) +
    # SwiGlu store into gate, BF16-valued matrices ((i*17 % 89) - 44)/64, x = ((i*43 % 113) - 56)/127,
    # gate = ((i*53 % 127) - 63)/32, rows 32 / 128, fused
    K, N, R = HIDDEN, FFN_DIM, 16
    packed = lambda n: ((np.arange(n, dtype=np.int64) * 17 % 89).astype(np.float32) - np.float32(44.0)) / \
        np.float32(64.0)
    w = packed(N * K).reshape(N, K)
    a = packed(R * K).reshape(R, K)
    b = packed(N * R).reshape(N, R)
    h = ctx.weights_from_f32(torch.from_numpy(w).to(dev))
    ad, bd = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    published = {32: 7.573, 128: 29.630}
    leg = {"workload": "weights.rs:580-631 benchmark_fused_projection: 2048->6144 int8 compute + rank-16 LoRA "
                       "(scale 0.5) + SwiGlu store, formula inputs; per call: gate restored, middle product "
                       "(dq8_lora_mid), projection with adapter and fused SwiGlu (dq8_apply); back-to-back calls",
           "rows": {}}
    for rows in (32, 128):
        x = ((np.arange(rows * K, dtype=np.int64) * 43 % 113).astype(np.float32) - np.float32(56.0)) / \
            np.float32(127.0)
        g0 = ((np.arange(rows * N, dtype=np.int64) * 53 % 127).astype(np.float32) - np.float32(63.0)) / \
            np.float32(32.0)
        xd = torch.from_numpy(x.reshape(rows, K)).to(dev)
        gd0 = torch.from_numpy(g0.reshape(rows, N)).to(dev)
        gate = gd0.clone()
        mid = torch.empty((rows, R), dtype=torch.float32, device=dev)
        lo = dq8._Lora(mid.data_ptr(), bd.data_ptr(), R, 0.5)

        def call():
            gate.copy_(gd0)
            ok(lib.dq8_lora_mid(ctx.handle, xd.data_ptr(), rows, K, ad.data_ptr(), R, mid.data_ptr(), sh),
               "dq8_lora_mid")
            ok(lib.dq8_apply(ctx.handle, h.handle, xd.data_ptr(), rows, None, ctypes.byref(lo), gate.data_ptr(),
                             dq8.ROWS, dq8.SWIGLU, sh), "dq8_apply")

        ms = timed_calls(torch, stream, call, 50)
        leg["rows"][str(rows)] = {"ms": round(ms, 5), "base_gops": round(2 * rows * N * K / (ms * 1e-3) / 1e9, 1),
                                  "published_arm_ms": published[rows],
                                  "speedup_vs_published": round(published[rows] / ms, 1)}
        if keep:
            call()
            leg[f"_check_fused_projection_rows{rows}"] = {"what": f"{rows} rows, all outputs", "items": [
                ("linear_lora_w", x.reshape(rows, K), w, a, b, 0.5, g0.reshape(rows, N), 2,
                 host_rows(torch, gate, np.arange(rows)))]}
    h.free()
    res["fused_projection"] = leg
    return res


def run_host_round_trip(args, torch, dq8, ctx, lib, dev, stream):
    """What a caller whose activations live in host memory pays (the crate's projections take host slices,
    tensor.rs:379-383): pinned host input -> device, the projection, result -> pinned host, synchronized; wall
    time per call on the host, against the device-only time of the same work.  Shapes of the multi-question
    continuation: 24 tokens."""
    import numpy as np

    M = args.question_tokens
    sh = stream.cuda_stream
    res = {"workload": f"{M} tokens: one 2048->2048 projection (dq8_apply), and one question's layer set (3 inputs "
                       f"quantized, one grouped launch of the 9 projections); pinned H2D, device work, pinned D2H, "
                       f"stream synchronize; host wall time, median of 50"}
    w = ctx.weights_from_f32((torch.randn((HIDDEN, HIDDEN), device=dev) * 0.02).contiguous())
    xh = torch.randn((M, HIDDEN)).pin_memory()
    oh = torch.empty((M, HIDDEN)).pin_memory()
    xd = torch.empty((M, HIDDEN), device=dev)
    od = torch.empty((M, HIDDEN), device=dev)
    proj = lambda: ok(lib.dq8_apply(ctx.handle, w.handle, xd.data_ptr(), M, None, None, od.data_ptr(), dq8.ROWS,
                                    dq8.WRITE, sh), "dq8_apply")

    def wall(fn, reps=50):
        for _ in range(5):
            fn()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return sorted(ts)[reps // 2] * 1e3

    def trip():
        xd.copy_(xh, non_blocking=True)
        proj()
        oh.copy_(od, non_blocking=True)
        stream.synchronize()

    def dev_only():
        proj()
        stream.synchronize()

    res["projection"] = {"round_trip_ms": round(wall(trip), 4), "device_sync_ms": round(wall(dev_only), 4),
                         "device_ms": round(timed_calls(torch, stream, proj, 50), 5),
                         "h2d_bytes": M * HIDDEN * 4, "d2h_bytes": M * HIDDEN * 4}
    w.free()
    shapes = [("q", HIDDEN, HIDDEN), ("k", KV_DIM, HIDDEN), ("v", KV_DIM, HIDDEN), ("o", HIDDEN, HIDDEN),
              ("gdn_in", GDN_IN, HIDDEN), ("gdn_out", HIDDEN, HIDDEN), ("gate", FFN_DIM, HIDDEN),
              ("up", FFN_DIM, HIDDEN), ("down", HIDDEN, FFN_DIM)]
    src = {"q": 0, "k": 0, "v": 0, "gdn_in": 0, "gate": 0, "up": 0, "o": 1, "gdn_out": 1, "down": 2}
    widths = [HIDDEN, HIDDEN, FFN_DIM]
    W = [ctx.weights_from_f32((torch.randn((n, k), device=dev) * 0.02).contiguous()) for _, n, k in shapes]
    ins_h = [torch.randn((M, k)).pin_memory() for k in widths]
    ins_d = [torch.empty((M, k), device=dev) for k in widths]
    qs = [(torch.empty((M, k), dtype=torch.int8, device=dev),
           torch.empty((M, (k + 63) // 64), dtype=torch.float32, device=dev)) for k in widths]
    outs_d = [torch.empty((M, n), device=dev) for _, n, _ in shapes]
    outs_h = [torch.empty((M, n)).pin_memory() for _, n, _ in shapes]
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    items = (dq8._Item * len(shapes))()
    for j, (nm, n, k) in enumerate(shapes):
        q, s = qs[src[nm]]
        items[j] = dq8._Item(W[j].handle, q.data_ptr(), s.data_ptr(), M, None, outs_d[j].data_ptr(), dq8.ROWS,
                             dq8.WRITE)

    def layer_dev():
        for i, k in enumerate(widths):
            ok(lib.dq8_quantize(ctx.handle, ins_d[i].data_ptr(), M, k, qs[i][0].data_ptr(), qs[i][1].data_ptr(),
                                flag.data_ptr(), sh), "dq8_quantize")
        ok(lib.dq8_linear_batch(ctx.handle, items, len(shapes), sh), "dq8_linear_batch")

    def layer_trip():
        for i in range(len(widths)):
            ins_d[i].copy_(ins_h[i], non_blocking=True)
        layer_dev()
        for o_h, o_d in zip(outs_h, outs_d):
            o_h.copy_(o_d, non_blocking=True)
        stream.synchronize()

    def layer_sync():
        layer_dev()
        stream.synchronize()

    res["question_layer_set"] = {
        "round_trip_ms": round(wall(layer_trip, 30), 4), "device_sync_ms": round(wall(layer_sync, 30), 4),
        "device_ms": round(timed_calls(torch, stream, layer_dev, 30), 5),
        "h2d_bytes": sum(M * k * 4 for k in widths), "d2h_bytes": sum(M * n * 4 for _, n, _ in shapes)}
    for x in W:
        x.free()
    return res


def run_checks(dq8o, checks, threads):
    """Each check item recomputed by the oracle on the host and compared bit for bit with the GPU's bits."""
    import numpy as np

    def same(a, b):
        a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
        return a.shape == b.shape and a.tobytes() == b.tobytes()

    out = {}
    for name, chk in checks.items():
        if chk is None:
            continue
        bad = []
        for j, it in enumerate(chk["items"]):
            kind = it[0]
            if kind in ("linear", "linear_w"):
                if kind == "linear":
                    _, x, wv, ws, result, ep, got = it
                else:
                    _, x, wf, result, ep, got = it
                    wv, ws = dq8o.quantize_weights(wf)
                want = dq8o.linear(x, wv, ws, result=result, epilogue=ep, threads=threads)
            elif kind in ("ffn_h", "ffn_h_w"):
                _, x, g, u, got = it
                if kind == "ffn_h_w":
                    g, u = dq8o.quantize_weights(g), dq8o.quantize_weights(u)
                gate = dq8o.linear(x, *g, threads=threads)
                want = dq8o.linear(x, *u, result=gate, epilogue=2, threads=threads)
            elif kind == "linear_lora_w":
                _, x, wf, a, b, scale, result, ep, got = it
                wv, ws = dq8o.quantize_weights(wf)
                want = dq8o.linear_lora(x, wv, ws, a, b, scale, result=result, epilogue=ep, threads=threads)
            else:
                raise ValueError(kind)
            if not same(got, want):
                bad.append(j)
        out[name] = "bit-exact" if not bad else f"MISMATCH in items {bad} ({chk['what']})"
    return out


def run_cpu_baseline(args, torch, dq8, ctx, dev, gen, checks):
    """The oracle (C restatement of the reference's x86 int8 path: per-projection input quantization +
    per-column scalar group dots, threads over output columns as rayon does, tensor.rs:442-448) on a sample of
    the stack's workload: one period of its 3:1 layer order (three GDN layers and one GQA layer, each with its
    FFN) for a bounded number of token rows.  One warm-up, then the median of 5 timed runs, with all usable host
    cores and with one.  Then the sampled oracle checks of the timed GPU workloads."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import dq8o

    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    # at most 16 threads: one GPU's share of the host
    threads = max(1, min(16, nproc, int(os.environ.get("OMP_NUM_THREADS", "16") or 16)))
    rng = np.random.default_rng(5)
    gdn = [("gdn_in", GDN_IN, HIDDEN), ("gdn_out", HIDDEN, HIDDEN)]
    gqa = [("q", HIDDEN, HIDDEN), ("k", KV_DIM, HIDDEN), ("v", KV_DIM, HIDDEN), ("o", HIDDEN, HIDDEN)]
    ffn = [("gate", FFN_DIM, HIDDEN), ("up", FFN_DIM, HIDDEN), ("down", HIDDEN, FFN_DIM)]
    ws = {}
    for name, n, k in gdn + gqa + ffn:
        h = ctx.weights_from_f32((torch.randn((n, k), generator=gen, device=dev) * 0.02).contiguous())
        ws[name] = exported(torch, h)
        h.free()

    def block(x, t):
        # three GDN layers, then a GQA layer (the stack's 3:1 order), each followed by its FFN; every
        # projection quantizes its own input, as the crate's linear does
        s = time.perf_counter()
        for mixer in ("gdn", "gdn", "gdn", "gqa"):
            names = ("gdn_in", "gdn_out") if mixer == "gdn" else ("q", "k", "v", "o")
            for name in names:
                dq8o.linear(x, *ws[name], threads=t)
            g = dq8o.linear(x, *ws["gate"], threads=t)
            g = dq8o.linear(x, *ws["up"], result=g, epilogue=2, threads=t)
            dq8o.linear(g, *ws["down"], result=x, epilogue=1, threads=t)
        return time.perf_counter() - s

    ops_per_row = 2 * (3 * sum(n * k for _, n, k in gdn) + sum(n * k for _, n, k in gqa) +
                       4 * sum(n * k for _, n, k in ffn))
    # size the sample so that one single-thread run takes about cpu_seconds / 10
    probe = rng.standard_normal((4, HIDDEN)).astype(np.float32)
    per_row = block(probe, 1) / 4
    rows = int(max(8, min(512, args.cpu_seconds / 10 / per_row)))
    x = rng.standard_normal((rows, HIDDEN)).astype(np.float32)

    def median_tops(t):
        block(x, t)
        secs = sorted(block(x, t) for _ in range(5))[2]
        return ops_per_row * rows / secs / 1e12, secs

    tops, secs = median_tops(threads)
    tops1, secs1 = median_tops(1)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    results = run_checks(dq8o, checks, threads)
    return {
        "value": round(tops, 5),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"one period of the stack's 3:1 layer order (3 GDN layers: in 2048->8224, out; 1 GQA layer: q, k, "
                  f"v, o; each with its FFN: gate/up SwiGlu, re-quantized down) for {rows} of the stack's 2048 "
                  f"tokens, quantization included; median of 5 runs after 1 warm-up "
                  f"({secs:.2f} s each at {threads} threads, {secs1:.2f} s at 1) on {cpu_model}",
        "value_1_thread": round(tops1, 5),
        "nproc": nproc,
        "cpu_model": cpu_model,
        "checks": results,
        "checks_passed": all(v == "bit-exact" for v in results.values()),
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
