"""Benchmark of the fused int4 frozen-base LoRA linear on one MI355X.

Workload (the north-star configuration): int4 group-64 frozen Linear 3072 -> 12288 with
LoRA r=32, alpha=32, M=4096 tokens, forward + backward (y, t, dx, dA, dB)
per step. Inputs are synthetic, seeded (numpy PCG64: W=0, X=1, A=2, B=3,
dY=4), resident in HBM before timing starts.

Prints ONE JSON line. `value` is whole-step algorithmic TFLOP/s,
F = 4MNK + 6Mr(K+N) per step.

`--workload skinny` measures the few-token forward instead (M=16, same
layer, forward only, HBM-bound): `value` is algorithmic GB/s,
W_B + 2MK + 2MN + 4r(K+N) bytes per forward, with the packed weight rotated
over more than 256 MB of distinct copies so the Infinity Cache cannot serve
it, and the forwards replayed from a HIP graph so host launch overhead is
not in the timed region. `roofline` is for the dominant kernel: its
algorithmic work per launch over its launch time. That time is the
kernel's in-step cost: HIP graphs of 10 steps, with and without one more
launch of the step's own launch of that kernel per step
(lrq_profile_relaunch, same arguments and outputs), replayed in
alternation; for the one-launch few-token forward it is the
graph-replayed forward itself. `kernels_us` holds every kernel of the
step measured that way, `kernels_us_isolated` each kernel repeated alone
back to back (a sustained repeat runs a few percent slower under the
power limit), and `kernels_us_events` the library's per-launch event
brackets (each adds a few microseconds of markers). `ceiling` holds what the box
delivers: torch.matmul's bf16 GEMM (hipBLASLt) at the layer's forward
and input-gradient shapes, and a streaming read of the packed weight.
`cpu_baseline` times the reference's CPU algorithm (the oracle's f32
dequant + f32 GEMMs) on a bounded token sample of the same layer.

The default line also carries `c1` (the 3072 -> 3072 r16 layer at
M=1024, the same measurement) and `c5` (the Qwen3-style decoder's 196
linears at M=16 and M=256, one step replayed from a HIP graph), and
`mmdit` (the C4 training step).

`--workload ns8` is the north-star layer over an int8 (Q8S) group-64 base,
`--workload c2` over a per-channel fp8 base: the same step and metric.

`--workload requant` measures the on-device load path: an fp8 checkpoint
tensor of the same layer (e4m3fn bytes and per-row f32 scales, [12288,
3072]) re-quantized to int4-g64 by one kernel; `value` is GB/s of fp8 bytes
and scales in plus packed int4 and group scales out per call.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

WORKLOADS = {
    # name: (M, K, N, r, alpha, fmt, group)
    "ns": (4096, 3072, 12288, 32, 32.0, "int4", 64),
    "c1": (1024, 3072, 3072, 16, 16.0, "int4", 64),
    "c2": (4096, 3072, 12288, 32, 32.0, "fp8", 0),
    "ns8": (4096, 3072, 12288, 32, 32.0, "int8", 64),  # the north-star layer over an int8 (Q8S) base
    "skinny": (16, 3072, 12288, 32, 32.0, "int4", 64),  # forward only, HBM-bound
    "skinny8": (16, 3072, 12288, 32, 32.0, "int8", 64),  # the same over an int8 (Q8S) base
    "requant": (0, 3072, 12288, 0, 0.0, "fp8", 64),  # fp8 checkpoint tensor -> int4, load time
    "c3": None,  # one synthetic MMDiT double-stream block's linear set (C3_SITES), image + text stream
    "c5": None,  # a Qwen3-style 28-layer decoder's linears (C5_LAYER), M swept over C5_M
    "mmdit": None,  # C4: the block-checkpointed synthetic MMDiT training step (loractl_amd.mmdit)
    "fewfit": None,  # few-token (M=16) forward and backward time against weight bytes over FEWFIT_SHAPES
}
MMDIT_TOKENS = (4096, 512)  # image tokens (64x64 latent, 2x2 patches), text tokens
# C3: (d_in, d_out) of QKV, attn-out, MLP up, MLP down, adaLN-mod; int4 g64, r=32, alpha=32
C3_SITES = [(3072, 9216), (3072, 3072), (3072, 12288), (12288, 3072), (3072, 18432)]
C3_STREAMS = (("image", 4096), ("text", 512))
# C5: q, k, v, o, gate, up, down of one layer; 28 layers; int4 g64, r=16, alpha=16
C5_LAYER = [(2560, 4096), (2560, 1024), (2560, 1024), (4096, 2560), (2560, 9728), (2560, 9728), (9728, 2560)]
C5_LAYERS = 28
C5_M = (1, 16, 256, 2048)
INFINITY_CACHE_BYTES = 256 << 20
GPU_SPIN_CYCLES = 100_000_000  # ~50 ms: longer than the host needs to enqueue a profiled loop


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--workload", default="ns", choices=sorted(WORKLOADS))
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-skinny", action="store_true", help="leave the skinny-M sub-object out of the ns line")
    p.add_argument("--no-mmdit", action="store_true", help="leave the MMDiT step sub-object out of the ns line")
    p.add_argument("--no-extra", action="store_true", help="leave the C1 and C5 sub-objects out of the ns line")
    p.add_argument("--profile-run", action="store_true",
                   help="no timing: run --steps steps of the workload (c5: at M=16 and 256) after one warm step, "
                        "plus one 256 MiB streaming-read probe (a known byte count for the traffic counters), for "
                        "rocprofv3 --pmc; prints one JSON line naming what ran")
    p.add_argument("--no-mmdit-kept", action="store_true",
                   help="MMDiT step: leave out the second measurement, with the capture's attention output kept "
                        "for the replay")
    return p.parse_args()


def flops_step(M, K, N, r):
    return 4.0 * M * N * K + 6.0 * M * r * (K + N)


def make_inputs(M, K, N, r):
    import numpy as np

    g = lambda seed: np.random.Generator(np.random.PCG64(seed))  # noqa: E731
    w = (g(0).standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    x = g(1).standard_normal((M, K), dtype=np.float32)
    bound = 1.0 / np.sqrt(K)
    a = g(2).uniform(-bound, bound, (K, r)).astype(np.float32)
    b = (g(3).standard_normal((r, N), dtype=np.float32) * np.float32(1e-3))
    dy = g(4).standard_normal((M, N), dtype=np.float32)
    return w, x, a, b, dy


def load_traffic(kernel, workload):
    """HBM bytes per launch from committed rocprofv3 --pmc summaries, if any."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        v = d.get(workload, {}).get(kernel)
        return None if v is None else float(v)
    except (OSError, ValueError):
        return None


WARM_MIN_MS = 200.0     # warm for at least this much GPU time, whatever --warmup says
WARM_MAX_MS = 20000.0   # and give up waiting for two agreeing windows after this much
WARM_AGREE = 0.03       # consecutive windows agreeing within 3% = steady state
X2_WINDOW = (1.7, 2.3)  # crates/loractl-bench/src/lib.rs:39-115: 2x the iterations takes 2x the time
X2_TRIES = 4


def event_timer(run, n):
    """GPU milliseconds of ``run(n)`` bracketed by events on the current
    stream, with a device synchronize on both sides."""
    import torch

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    run(n)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def warm_and_time(run, steps, warmup):
    """The timing protocol: ``warmup`` untimed iterations, then more until
    the GPU is in steady state (at least WARM_MIN_MS of work and two
    consecutive ``steps``-iteration windows within WARM_AGREE), then ``steps``
    timed iterations and ``2 * steps`` for the sanity ratio, re-timed until
    the ratio lands in X2_WINDOW. Returns (ms for ``steps``, ratio, warm ms)."""
    run(warmup)
    warm_ms, prev = 0.0, None
    while True:
        cur = event_timer(run, steps)
        warm_ms += cur
        if warm_ms >= WARM_MIN_MS and prev is not None and abs(cur - prev) <= WARM_AGREE * prev:
            break
        if warm_ms >= WARM_MAX_MS:
            break
        prev = cur
    for _ in range(X2_TRIES):
        ms = event_timer(run, steps)
        ratio = event_timer(run, 2 * steps) / ms
        if X2_WINDOW[0] <= ratio <= X2_WINDOW[1]:
            return ms, ratio, warm_ms
    raise RuntimeError(f"timing never settled: 2x-iteration ratio {ratio:.3f} outside {X2_WINDOW} "
                       f"after {X2_TRIES} tries")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box of this build has one MI355X and the path is "
              f"single-device; --gpus {args.gpus} is not supported (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)
    import torch

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    if args.profile_run:
        return profile_run(args, dev)
    if args.workload in ("skinny", "skinny8"):
        return bench_skinny(args, dev)
    if args.workload == "requant":
        return bench_requant(args, dev)
    if args.workload == "c3":
        return bench_c3(args, dev)
    if args.workload == "c5":
        return bench_c5(args, dev)
    if args.workload == "mmdit":
        return bench_mmdit(args, dev)
    if args.workload == "fewfit":
        print(json.dumps(few_token_fit(dev)), flush=True)
        return None
    out, ceilings_for = site_measure(args, dev, args.workload, with_cpu=not args.no_cpu_baseline,
                                     ceilings=args.workload in ("ns", "c1"))
    if args.workload == "ns" and not args.no_skinny:
        # the north star's second bar, the few-token forward of the same layer
        out["skinny"] = skinny_measure(args, dev, with_cpu=not args.no_cpu_baseline)
        read = out.get("ceiling", {}).get("stream_read_packed_weight")
        if read:
            r = out["skinny"]["roofline"]
            r["measured_ceiling"] = read["gbs"]
            r["frac_of_measured"] = round(r["achieved"] / read["gbs"], 4)
    if args.workload == "ns" and not args.no_extra:
        # the mid-size configurations, timed by the driver too: C1, and C5
        # at the few-token and mid token counts
        torch.cuda.empty_cache()
        out["c1"] = site_measure(args, dev, "c1", with_cpu=False, ceilings=True)[0]
        torch.cuda.empty_cache()
        out["c5"] = c5_measure(args, dev, (16, 256), with_cpu=False)
        torch.cuda.empty_cache()
        out["few_token_fit"] = few_token_fit(dev)
    if args.workload == "ns" and not args.no_mmdit:
        # the metric's second half: MMDiT train steps/s (C4)
        torch.cuda.empty_cache()
        out["mmdit"] = mmdit_measure(args, dev, steps=min(args.steps, 5), warmup=min(args.warmup, 2),
                                     with_cpu=not args.no_cpu_baseline)
    print(json.dumps(out), flush=True)


# (K, N, r) of the few-token fit: C5's projections and the north-star layer
FEWFIT_SHAPES = ((2560, 1024, 16), (2560, 4096, 16), (4096, 2560, 16), (2560, 9728, 16), (9728, 2560, 16),
                 (3072, 12288, 32))


def few_token_fit(dev, M=16, reps=60):
    """Graph-replay time of one few-token (M=16, int4 g64) forward (y, t) and
    one backward (dx, dA, dB: one launch each) per shape, with the packed
    weight rotated past the Infinity Cache, against the bytes the launch
    must move; then the least-squares line time = intercept + slope * MB
    over the shapes. The intercept is the per-launch cost that does not
    depend on the weight (launch, the t / u publication, the epilogue
    hand-off); 1 / slope is the marginal streaming rate."""
    import math

    import numpy as np
    import torch

    from loractl_amd import _lib as L
    from loractl_amd import device as D

    rows = []
    for K, N, r in FEWFIT_SHAPES:
        g = np.random.Generator(np.random.PCG64(K * 7 + N))
        wq = D.quantize_int4(torch.from_numpy((g.standard_normal((N, K)) * 0.02).astype(np.float32)).to(dev), 64)
        wb = D.compute_weight(wq)
        del wq
        NB, KB = (N + 63) // 64, (K + 63) // 64
        data_b, scale_b = N * K // 2, 4 * NB * KB * 64  # one section of the blocked layout and its scales
        ncopy = max(2, math.ceil(1.15 * INFINITY_CACHE_BYTES / (data_b + scale_b)))
        copies = [wb] + [D.PackedWeight(wb.fmt, wb.n, wb.k, wb.data.clone(), wb.scales.clone(), wb.group,
                                        wb.per_channel, None, L.LRQ_LAYOUT_BLOCKED) for _ in range(ncopy - 1)]
        x = torch.from_numpy(g.standard_normal((M, K)).astype(np.float32)).to(dev).to(torch.bfloat16)
        dy = torch.from_numpy(g.standard_normal((M, N)).astype(np.float32)).to(dev).to(torch.bfloat16)
        a = torch.from_numpy(g.uniform(-1 / math.sqrt(K), 1 / math.sqrt(K), (K, r)).astype(np.float32)).to(dev).to(
            torch.bfloat16)
        b = torch.from_numpy((g.standard_normal((r, N)) * 1e-3).astype(np.float32)).to(dev).to(torch.bfloat16)
        s = 1.0
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        out = {}
        with torch.cuda.stream(stream):
            D.reserve(M, N, K, r)
            y, t = D.lora_fwd(x, wb, a, b, s)
            dx, da, db = D.lora_bwd(x, dy, wb, a, b, s, t)
            torch.cuda.synchronize()
            for name, call in (("fwd", lambda i: D.lora_fwd(x, copies[i % ncopy], a, b, s, y=y, t=t)),
                               ("bwd", lambda i: D.lora_bwd(x, dy, copies[i % ncopy], a, b, s, t,
                                                            out=(dx, da, db)))):
                call(0)
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for i in range(reps):
                        call(i)
                graph.replay()
                torch.cuda.synchronize()
                best = float("inf")
                for _ in range(5):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    graph.replay()
                    e1.record(stream)
                    torch.cuda.synchronize()
                    best = min(best, e0.elapsed_time(e1) * 1000.0 / reps)
                out[name] = best
                del graph
        # bytes a launch must move: the weight section and its scales, the
        # activations and factors read, the outputs written
        fwd_b = data_b + scale_b + 2 * M * K + 2 * K * r + 2 * r * N + 2 * M * N + 2 * M * r
        bwd_b = data_b + scale_b + 2 * M * N + 2 * r * N + 2 * K * r + 2 * M * K + 2 * M * r + 2 * M * K \
            + 4 * K * r + 4 * r * N
        rows.append({"K": K, "N": N, "r": r, "fwd_us": round(out["fwd"], 2), "bwd_us": round(out["bwd"], 2),
                     "fwd_mb": round(fwd_b / 1e6, 3), "bwd_mb": round(bwd_b / 1e6, 3)})
        del copies, wb
        torch.cuda.empty_cache()

    def fit(xs, ys):
        A = np.stack([np.ones(len(xs)), np.asarray(xs)], axis=1)
        (c0, c1), *_ = np.linalg.lstsq(A, np.asarray(ys), rcond=None)
        return {"intercept_us": round(float(c0), 2), "us_per_mb": round(float(c1), 4),
                "marginal_tbs": round(1.0 / float(c1), 2) if c1 > 0 else None}

    return {"workload": f"few-token int4-g64 LoRA linear, M={M}, one launch per pass (forward y, t; backward "
                        "dx, dA, dB), packed weight rotated past the Infinity Cache, graph replay",
            "shapes": rows,
            "fwd_fit": fit([r_["fwd_mb"] for r_ in rows], [r_["fwd_us"] for r_ in rows]),
            "bwd_fit": fit([r_["bwd_mb"] for r_ in rows], [r_["bwd_us"] for r_ in rows])}


PROBE_BYTES = 256 << 20


def profile_run(args, dev):
    """The kernels of one workload for a counter run, untimed: one warm step,
    then ``--steps`` steps (the site workloads: host-launched fwd + bwd; c5:
    every site at M = 16, then at M = 256; c3: every site of both streams;
    mmdit: the checkpointed training step with its optimizer step; skinny:
    the few-token forward over the rotated weight copies), then one
    streaming read of PROBE_BYTES by lrq_probe_stream_read, whose byte count
    calibrates FETCH_SIZE."""
    import math

    import torch

    from loractl_amd import _lib as L
    from loractl_amd import device as D

    w = args.workload
    if w in ("ns", "ns8", "c1", "c2", "skinny", "skinny8"):
        M, K, N, r, alpha, fmt, group = WORKLOADS[w]
        s = alpha / r
        wf, x, a, b, dy = make_inputs(M, K, N, r)
        wt = torch.from_numpy(wf).to(dev)
        wq = {"int4": lambda: D.quantize_int4(wt, group), "int8": lambda: D.quantize_int8(wt, group),
              "fp8": lambda: D.quantize_fp8(wt, True)}[fmt]()
        del wt
        wq = D.compute_weight(wq)
        xb, ab, bb, dyb = (torch.from_numpy(v).to(dev).to(torch.bfloat16) for v in (x, a, b, dy))
        D.reserve(M, N, K, r)
        if w.startswith("skinny"):
            row_bytes = wq.data.numel() // 2
            ncopy = max(2, math.ceil(1.15 * INFINITY_CACHE_BYTES / row_bytes))
            copies = [wq] + [D.PackedWeight(wq.fmt, wq.n, wq.k, wq.data.clone(), wq.scales.clone(), wq.group,
                                            wq.per_channel, None, L.LRQ_LAYOUT_BLOCKED) for _ in range(ncopy - 1)]

            def step(i):
                D.lora_fwd(xb, copies[i % ncopy], ab, bb, s)
        else:
            def step(i):
                _, t = D.lora_fwd(xb, wq, ab, bb, s)
                D.lora_bwd(xb, dyb, wq, ab, bb, s, t)
        for i in range(1 + args.steps):
            step(i)
        torch.cuda.synchronize()
        ran = f"{w}: {1 + args.steps} steps"
    elif w == "c5":
        ran = []
        for M in (16, 256):
            sites = [(M, K, N, 16, 16.0) for _layer in range(C5_LAYERS) for (K, N) in C5_LAYER]
            ls = LinearSet(dev, sites, seed=5)
            ls.run(1 + args.steps)
            torch.cuda.synchronize()
            ran.append(f"c5 M={M}: {1 + args.steps} steps")
            del ls
            torch.cuda.empty_cache()
        ran = "; ".join(ran)
    elif w == "c3":
        sites = [(M, K, N, 32, 32.0) for (_name, M) in C3_STREAMS for (K, N) in C3_SITES]
        ls = LinearSet(dev, sites, seed=3)
        ls.run(1 + args.steps)
        torch.cuda.synchronize()
        ran = f"c3: {1 + args.steps} steps"
    elif w == "mmdit":
        from loractl_amd.mmdit import Mmdit, MmditConfig, build_mmdit_adapters, checkpointed_step, flow_batch

        cfg = MmditConfig()
        model = Mmdit(cfg, dev, seed=0)
        ad = build_mmdit_adapters(cfg, dev, seed=1)
        batch = flow_batch(cfg, *MMDIT_TOKENS, dev, seed=2)
        opt = torch.optim.AdamW([p for d in ad.deltas for p in (d.lora_a, d.lora_b)], lr=1e-4, eps=1e-5,
                                weight_decay=0.0, fused=True)
        for i in range(1 + args.steps):
            opt.zero_grad(set_to_none=True)
            checkpointed_step(model, ad, batch)
            opt.step()
        torch.cuda.synchronize()
        ran = f"mmdit: {1 + args.steps} steps"
    else:
        raise SystemExit(f"--profile-run covers ns, ns8, c1, c2, c3, c5, mmdit, skinny, skinny8, not {w}")
    buf = torch.empty(PROBE_BYTES, dtype=torch.uint8, device=dev)
    D.probe_stream_read(buf)
    torch.cuda.synchronize()
    print(json.dumps({"profile_run": ran, "probe_stream_read_bytes": PROBE_BYTES}), flush=True)


RELAUNCH_REPS = 20  # back-to-back repeats of one kernel per graph
RELAUNCH_ROUNDS = 5


def isolated_kernel_us(kernels, reps=RELAUNCH_REPS, rounds=RELAUNCH_ROUNDS):
    """GPU microseconds per launch of each of ``kernels`` (profiler names)
    alone: the library repeats its last launch of that kernel with the same
    arguments (lrq_profile_relaunch), ``reps`` times back to back in one HIP
    graph, which is replayed ``rounds`` times between events on the replay
    stream. No per-launch markers sit between the repeats."""
    import torch

    from loractl_amd import device as D

    ctx = D.context()
    side = torch.cuda.Stream()
    out = {}
    for k in kernels:
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            D.profile_relaunch(k, reps, ctx=ctx, on_stream=side)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(rounds):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        out[k] = e0.elapsed_time(e1) * 1e3 / (rounds * reps)
        del graph
    return out


FWD_KERNELS = ("lora_t", "fwd_main")


def in_step_kernel_us(fwd, bwd, kernels, reserve, n_steps=10, rounds=10):
    """Each kernel's cost inside the step, in microseconds per launch: HIP
    graphs of ``n_steps`` steps (``fwd`` then ``bwd``), one plain and one per
    kernel in which that kernel's step launch is repeated once more right
    after its pass (lrq_profile_relaunch: same arguments, same outputs),
    replayed in alternation ``rounds`` times; the extra time per step is the
    kernel's duration among the step's other kernels (so under the step's
    power state, not a sustained repeat's). Returns (per kernel, step us)."""
    import torch

    from loractl_amd import device as D

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graphs = {}
    with torch.cuda.stream(side):
        reserve()
        fwd()
        bwd()
        torch.cuda.synchronize()
        for k in [None] + list(kernels):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for _ in range(n_steps):
                    fwd()
                    if k in FWD_KERNELS:
                        D.profile_relaunch(k, 1)
                    bwd()
                    if k is not None and k not in FWD_KERNELS:
                        D.profile_relaunch(k, 1)
            graphs[k] = g
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for g in graphs.values():
        g.replay()
    torch.cuda.synchronize()
    total = {k: 0.0 for k in graphs}
    for _ in range(rounds):
        for k, g in graphs.items():
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            total[k] += e0.elapsed_time(e1)
    per = {k: 1e3 * v / (rounds * n_steps) for k, v in total.items()}
    del graphs
    return {k: per[k] - per[None] for k in kernels}, per[None]


GEMM_CEILING_HOW = ("50 calls per HIP graph, replayed (best of three); the faster of W^T as a transposed view and "
                    "as a contiguous copy for the forward, of W and of a transposed view of the copy for dx")


def gemm_pair_us(x, w, wt, dy):
    """The vendor library's bf16 GEMM time for x . W^T and dy . W (w [N, K],
    wt its contiguous transpose), graph-replayed, the faster operand layout
    of each."""
    import torch

    fwd = min(graph_us(lambda: torch.matmul(x, w.t())), graph_us(lambda: torch.matmul(x, wt)))
    dx = min(graph_us(lambda: torch.matmul(dy, w)), graph_us(lambda: torch.matmul(dy, wt.t())))
    return fwd, dx


def measure_ceilings(M, K, N, weights, row_bytes):
    """What the part delivers on this box, for the fractions of the bench
    line: the bf16 GEMM of the vendor library (torch.matmul, hipBLASLt) at
    the forward shape x[M,K] . W^T and the input-gradient shape dy[M,N] . W,
    no dequantization; and a streaming read of the packed weight's row
    section (``row_bytes`` of each of ``weights``, rotated past the Infinity
    Cache) by the library's probe (16-byte loads, every byte once)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(9)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    wt = w.t().contiguous()
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)

    def timed(fn, n=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        best = float("inf")
        for _ in range(3):
            e0.record()
            for _ in range(n):
                fn()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3 / n)
        return best

    fwd_us, dx_us = gemm_pair_us(x, w, wt, dy)
    del w, wt, x, dy
    from loractl_amd import device as D

    views = [wb.data[:row_bytes] for wb in weights]
    n = len(views)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    reads = 100
    with torch.cuda.stream(side):
        D.probe_stream_read(views[0])
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for i in range(reads):
                D.probe_stream_read(views[i % n])
    torch.cuda.synchronize()
    read_us = timed(lambda: graph.replay(), n=4) / reads
    fl = 2.0 * M * N * K
    return {
        "gemm_bf16_hipblaslt": {"fwd_us": round(fwd_us, 2), "fwd_tflops": round(fl / (fwd_us * 1e-6) / 1e12, 1),
                                "dx_us": round(dx_us, 2), "dx_tflops": round(fl / (dx_us * 1e-6) / 1e12, 1),
                                "shape": f"x[{M},{K}] . W^T[{K},{N}] and dy[{M},{N}] . W[{N},{K}], bf16, torch.matmul",
                                "how": GEMM_CEILING_HOW},
        "stream_read_packed_weight": {"us": round(read_us, 3), "bytes": row_bytes,
                                      "gbs": round(row_bytes / (read_us * 1e-6) / 1e9, 1),
                                      "how": f"lrq_probe_stream_read over the blocked weight's row section, "
                                             f"rotated over {n} copies, {reads} reads replayed from a HIP graph"},
    }


def site_measure(args, dev, workload, with_cpu=True, ceilings=False):
    """One fused site of ``workload`` (ns, ns8, c1, c2): the step y, t =
    fwd(x); dx, dA, dB = bwd(dy) timed over host-launched steps; every
    kernel's in-step cost from graph differentials (``kernels_us``), its
    time alone (``kernels_us_isolated``) and its event brackets
    (``kernels_us_events``); the roofline of the dominant kernel from its
    in-step cost; measured ceilings when asked. Returns (line, None)."""
    import math

    import torch

    from loractl_amd import _lib as L
    from loractl_amd import device as D

    M, K, N, r, alpha, fmt, group = WORKLOADS[workload]
    s = alpha / r
    w, x, a, b, dy = make_inputs(M, K, N, r)
    wt = torch.from_numpy(w).to(dev)
    wq = {"int4": lambda: D.quantize_int4(wt, group), "int8": lambda: D.quantize_int8(wt, group),
          "fp8": lambda: D.quantize_fp8(wt, True)}[fmt]()
    del wt
    # the interchange (row) layout, for the CPU baseline: the first fused
    # call re-lays the weight into the blocked layout in place
    wq_rows = (wq.data.cpu().numpy(), wq.scales.cpu().numpy()) if with_cpu else None
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    ab = torch.from_numpy(a).to(dev).to(torch.bfloat16)
    bb = torch.from_numpy(b).to(dev).to(torch.bfloat16)
    dyb = torch.from_numpy(dy).to(dev).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    t = torch.empty((M, r), dtype=torch.bfloat16, device=dev)
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    da = torch.empty((K, r), dtype=torch.float32, device=dev)
    db = torch.empty((r, N), dtype=torch.float32, device=dev)
    D.reserve(M, N, K, r)

    def step():
        D.lora_fwd(xb, wq, ab, bb, s, y=y, t=t)
        D.lora_bwd(xb, dyb, wq, ab, bb, s, t, out=(dx, da, db))

    def run(n):
        for _ in range(n):
            step()

    run(1)
    torch.cuda.synchronize()
    for v in (y, dx, da, db):
        if not torch.isfinite(v).all() or not v.abs().max() > 0:
            raise RuntimeError("implausible output (all-zero or non-finite)")

    ms_total, ratio, warm_ms = warm_and_time(run, args.steps, args.warmup)
    ms_step = ms_total / args.steps
    F = flops_step(M, K, N, r)
    value = F / (ms_step * 1e-3) / 1e12

    # which kernels a step launches, and their event-bracketed times (the GPU
    # first spins so that every profiled launch is queued behind it)
    prof = profile_kernels(run, args.steps)
    events = {k: 1e3 * ms / n for k, (ms, n) in prof.items()}
    # each kernel's cost inside the step (graph differential), and alone
    # (back-to-back repeats of its step launch)
    in_step, graph_step_us = in_step_kernel_us(lambda: D.lora_fwd(xb, wq, ab, bb, s, y=y, t=t),
                                               lambda: D.lora_bwd(xb, dyb, wq, ab, bb, s, t, out=(dx, da, db)),
                                               list(prof), lambda: D.reserve(M, N, K, r))
    step()
    torch.cuda.synchronize()
    iso = isolated_kernel_us(list(prof))
    per_kernel_flops = {"fwd_main": 2.0 * M * N * (K + r), "bwd_dx": 2.0 * M * K * (N + r)}
    dom = max(("fwd_main", "bwd_dx"), key=lambda k: in_step[k])
    achieved = per_kernel_flops[dom] / (in_step[dom] * 1e-6) / 1e12
    roofline = {
        "kernel": dom,
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "traffic": load_traffic(dom, workload),
        "flops_per_launch": per_kernel_flops[dom],
        "avg_launch_us": round(in_step[dom], 2),
        "launch_time_from": "in-step cost: HIP graphs of 10 steps with and without one more launch of the "
                            "step's own " + dom + " per step, replayed in alternation",
        "isolated_us": round(iso[dom], 2),
        "achieved_isolated": round(per_kernel_flops[dom] / (iso[dom] * 1e-6) / 1e12, 2),
    }
    out = {
        "metric": f"{fmt}-base LoRA linear fwd+bwd TFLOP/s",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded PCG64; W~N(0,0.02) quantized on device, X,dY~N(0,1), A~U(+-1/sqrt(K)), B~N(0,1e-3))",
        "config": {
            "workload": f"{fmt}{'-per-channel' if fmt == 'fp8' else '-g' + str(group)} frozen Linear {K}->{N} "
                        f"+ LoRA r={r} alpha={alpha:g}, M={M} tokens, forward+backward (y, dx, dA, dB)",
            "M": M, "K": K, "N": N, "rank": r, "group": group, "format": fmt,
            "parallelism": "single-gpu",
        },
        "pct_of_mfma_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "flops_per_step": F,
        "sanity_x2_ratio": round(ratio, 3),
        "warm_ms": round(warm_ms, 1),
        "kernels_us": {k: round(v, 2) for k, v in in_step.items()},
        "kernels_us_sum": round(sum(in_step.values()), 2),
        "graph_step_us": round(graph_step_us, 2),
        "kernels_us_isolated": {k: round(v, 2) for k, v in iso.items()},
        "kernels_us_events": {k: round(v, 2) for k, v in events.items()},
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if ceilings:
        NB, KB = (N + 63) // 64, (K + 63) // 64
        row_bytes = wq.data.numel() // 2
        ncopy = max(2, math.ceil(1.15 * INFINITY_CACHE_BYTES / row_bytes))
        copies = [wq] + [D.PackedWeight(wq.fmt, wq.n, wq.k, wq.data.clone(), wq.scales, wq.group, wq.per_channel,
                                        None, L.LRQ_LAYOUT_BLOCKED) for _ in range(ncopy - 1)]
        ceil_ = measure_ceilings(M, K, N, copies, row_bytes)
        del copies
        out["ceiling"] = ceil_
        key = "fwd_tflops" if dom == "fwd_main" else "dx_tflops"
        roofline["measured_ceiling"] = ceil_["gemm_bf16_hipblaslt"][key]
        roofline["frac_of_measured"] = round(achieved / ceil_["gemm_bf16_hipblaslt"][key], 4)
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(wq_rows, x, a, b, dy, M, K, N, r, s, group, fmt, args.cpu_seconds)
    del wq, xb, ab, bb, dyb, y, t, dx, da, db
    return out, None


def skinny_measure(args, dev, with_cpu=True, steps=100, workload="skinny"):
    """The few-token forward of the north-star layer (M=16): GB/s with the
    packed weight rotated past the Infinity Cache and ``steps`` forwards
    replayed from a HIP graph; per-kernel times from the library's events;
    the roofline of the dominant kernel; the CPU baseline when asked."""
    import math

    import torch

    from loractl_amd import _lib as L
    from loractl_amd import device as D

    M, K, N, r, alpha, fmt, group = WORKLOADS[workload]
    s = alpha / r
    w, x, a, b, _ = make_inputs(M, K, N, r)
    wt = torch.from_numpy(w).to(dev)
    wq = D.quantize_int8(wt, group) if fmt == "int8" else D.quantize_int4(wt, group)
    del wt
    wq_rows = (wq.data.cpu().numpy(), wq.scales.cpu().numpy()) if with_cpu else None
    wb = D.compute_weight(wq)
    # the row section of the blocked layout, the part the few-token kernel
    # reads: half the data (the transposed section follows) and the first
    # [NB][Gp][64] scales
    NB, KB = (N + 63) // 64, (K + 63) // 64
    wbytes = wb.data.numel() // 2 + 4 * NB * (KB * 64 // group) * 64
    ncopy = max(2, math.ceil(1.15 * INFINITY_CACHE_BYTES / wbytes))
    copies = [wb] + [D.PackedWeight(wb.fmt, wb.n, wb.k, wb.data.clone(), wb.scales.clone(), wb.group,
                                    wb.per_channel, None, L.LRQ_LAYOUT_BLOCKED) for _ in range(ncopy - 1)]
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    ab = torch.from_numpy(a).to(dev).to(torch.bfloat16)
    bb = torch.from_numpy(b).to(dev).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    t = torch.empty((M, r), dtype=torch.bfloat16, device=dev)
    D.reserve(M, N, K, r)

    def fwd(i):
        D.lora_fwd(xb, copies[i % ncopy], ab, bb, s, y=y, t=t)

    for i in range(ncopy):
        fwd(i)
    torch.cuda.synchronize()
    if not torch.isfinite(y).all() or not y.abs().max() > 0:
        raise RuntimeError("implausible output (all-zero or non-finite)")
    # one graph of `steps` forwards over the rotating copies, captured on a
    # side stream whose context was sized before the capture
    n_graph = steps
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        D.reserve(M, N, K, r)
        fwd(0)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(n_graph):
                fwd(i)
    torch.cuda.synchronize()

    def run(reps):
        for _ in range(reps):
            graph.replay()

    ms_total, ratio, warm_ms = warm_and_time(run, 4, 2)
    ms_fwd = ms_total / (4 * n_graph)
    wb_alg = N * K * (1 if fmt == "int8" else 0.5) + 4 * N * K / group  # W_B (packed q + f32 group scales)
    bytes_fwd = wb_alg + 2 * M * K + 2 * M * N + 4 * r * (K + N)
    value = bytes_fwd / (ms_fwd * 1e-3) / 1e9

    D.profile_reset()
    D.profile_enable(True)
    torch.cuda._sleep(GPU_SPIN_CYCLES)
    for i in range(steps):
        fwd(i)
    torch.cuda.synchronize()
    prof = D.profile_read()
    D.profile_enable(False)
    kernels = {k: 1e3 * ms / n for k, (ms, n) in prof.items() if n}
    launches = {k: n for k, (ms, n) in prof.items() if n}
    rp = (r + 15) // 16 * 16
    # the few-token kernel's own traffic: packed weight as stored (blocked
    # data + scales), x, y, B and the padded t
    k_bytes = wbytes + 2 * M * K + 2 * M * N + 2 * r * N + 2 * M * rp
    # When the forward is that one launch, its duration is the timed graph
    # replay per forward (events on the replay stream, back-to-back launches);
    # the per-launch event brackets add their own markers, a quarter of a
    # 14 us kernel.
    one_launch = list(launches) == ["fwd_main"] and launches["fwd_main"] == steps
    launch_us = ms_fwd * 1e3 if one_launch else kernels["fwd_main"]
    achieved = k_bytes / (launch_us * 1e-6) / 1e9
    roofline = {
        "kernel": "fwd_main",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": load_traffic("fwd_main", workload),
        "bytes_per_launch": k_bytes,
        "avg_launch_us": round(launch_us, 3),
        "launch_time_from": "graph replay per forward (one launch)" if one_launch else "per-launch events",
    }
    cpu = None
    if with_cpu:
        cpu = cpu_baseline_fwd(wq_rows, x, a, b, M, K, N, r, s, group, args.cpu_seconds, bytes_fwd, fmt)
    return {
        "metric": f"{fmt}-base LoRA linear skinny-M forward GB/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "us_per_forward": round(ms_fwd * 1e3, 3),
        "pct_of_hbm_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
        "bytes_per_forward": bytes_fwd,
        "sanity_x2_ratio": round(ratio, 3),
        "workload": f"{fmt}-g{group} frozen Linear {K}->{N} + LoRA r={r} alpha={alpha:g}, M={M} tokens, "
                    f"forward (y, t); packed weight rotated over {ncopy} copies "
                    f"({ncopy * wbytes / 2**20:.0f} MiB), {n_graph} forwards replayed from a HIP graph",
        "kernels_us": {k: round(v, 3) for k, v in kernels.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }


def bench_skinny(args, dev):
    M, K, N, r, alpha, fmt, group = WORKLOADS[args.workload]
    m = skinny_measure(args, dev, with_cpu=not args.no_cpu_baseline, steps=args.steps, workload=args.workload)
    out = {
        "metric": m["metric"],
        "value": m["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["us_per_forward"] * 1e-3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded PCG64; W~N(0,0.02) quantized on device, X~N(0,1), A~U(+-1/sqrt(K)), B~N(0,1e-3))",
        "config": {"workload": m["workload"], "M": M, "K": K, "N": N, "rank": r, "group": group, "format": fmt,
                   "parallelism": "single-gpu"},
        "pct_of_hbm_peak": m["pct_of_hbm_peak"],
        "bytes_per_step": m["bytes_per_forward"],
        "sanity_x2_ratio": m["sanity_x2_ratio"],
        "kernels_us": m["kernels_us"],
        "roofline": m["roofline"],
        "cpu_baseline": m["cpu_baseline"],
    }
    print(json.dumps(out), flush=True)


def bench_requant(args, dev):
    """fp8 e4m3fn [N, K] + per-row scales -> int4 (Q4S, g64) on the device,
    timed over `steps` calls with inputs resident; the CPU baseline is the
    reference's host path (f32 decode, then the Q4S quantizer) on a row
    sample."""
    import numpy as np
    import torch

    from loractl_amd import device as D
    from loractl_amd import fp8 as F

    _, K, N, _, _, _, group = WORKLOADS["requant"]
    w, _, _, _, _ = make_inputs(1, K, N, 1)
    w8 = D.quantize_fp8(torch.from_numpy(w).to(dev), True)
    w8 = F.fp8_weight("w", w8.data, w8.scales)
    for _ in range(args.warmup):
        D.requantize_fp8_int4(w8, group)
    torch.cuda.synchronize()
    out = D.requantize_fp8_int4(w8, group)
    if not out.scales.abs().max() > 0:
        raise RuntimeError("implausible output (all-zero scales)")

    def timed(n):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            D.requantize_fp8_int4(w8, group)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    ms = timed(args.steps) / args.steps
    ratio = timed(2 * args.steps) / (ms * args.steps)
    nbytes = N * K + 4 * N + N * K // 2 + 4 * N * (K // group)
    value = nbytes / (ms * 1e-3) / 1e9
    D.profile_reset()
    D.profile_enable(True)
    torch.cuda._sleep(GPU_SPIN_CYCLES)
    for _ in range(args.steps):
        D.requantize_fp8_int4(w8, group)
    torch.cuda.synchronize()
    prof = D.profile_read()
    D.profile_enable(False)
    kernels = {k: 1e3 * t / n for k, (t, n) in prof.items() if n}
    achieved = nbytes / (kernels["quantize_int4"] * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        import oracle as O

        rows = 256
        b8, s8 = w8.data[:rows].cpu().numpy(), w8.scales[:rows].cpu().numpy()
        O.quantize_int4_packed(O.fp8_dequant(b8, s8), group)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0):
            O.quantize_int4_packed(O.fp8_dequant(b8, s8), group)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        cpu = {"value": round(nbytes * rows / N / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{rows} of {N} rows, {reps} reps of {dt:.4f} s (f32 decode, then Q4S quantize)"}
    print(json.dumps({
        "metric": "fp8 checkpoint tensor -> int4 on-device requantization GB/s",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic (seeded PCG64 W~N(0,0.02), fp8 per-row repack on device)",
        "config": {"workload": f"fp8 e4m3fn [{N}, {K}] + per-row f32 scales -> int4-g{group} (packed + scales)",
                   "N": N, "K": K, "group": group, "parallelism": "single-gpu"},
        "sanity_x2_ratio": round(ratio, 3),
        "kernels_us": {k: round(v, 3) for k, v in kernels.items()},
        "roofline": {"kernel": "quantize_int4", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": load_traffic("quantize_int4", "requant"), "bytes_per_launch": nbytes,
                     "avg_launch_us": round(kernels["quantize_int4"], 3)},
        "cpu_baseline": cpu,
    }), flush=True)


class LinearSet:
    """A set of fused int4 LoRA linear sites sharing one step: each site has
    its own frozen weight (quantized on the device from seeded
    W ~ N(0, 0.02), then blocked), LoRA factors and bf16 activations;
    ``acts`` maps an activation key to x [M, K] / dy [M, N] buffers that
    sites of the same shape may share. A step runs every site's forward
    (y, t) then backward (dx, dA, dB)."""

    def __init__(self, dev, sites, group=64, seed=0, keep_rows=0):
        import torch

        from loractl_amd import device as D

        self.D = D
        self.sites = []
        self.rows = []
        g = torch.Generator(device=dev).manual_seed(seed)
        acts = {}
        for i, (M, K, N, r, alpha) in enumerate(sites):
            w = torch.randn(N, K, device=dev, generator=g) * 0.02
            wq = D.quantize_int4(w, group)
            if i < keep_rows:
                self.rows.append((wq.data.cpu().numpy(), wq.scales.cpu().numpy()))
            del w
            D.compute_weight(wq)
            key = (M, K, N)
            if key not in acts:
                x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
                dy = torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16)
                out = (torch.empty((M, N), dtype=torch.bfloat16, device=dev),
                       torch.empty((M, r), dtype=torch.bfloat16, device=dev),
                       torch.empty((M, K), dtype=torch.bfloat16, device=dev),
                       torch.empty((K, r), dtype=torch.float32, device=dev),
                       torch.empty((r, N), dtype=torch.float32, device=dev))
                acts[key] = (x, dy, out)
            a = ((torch.rand(K, r, device=dev, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
            b = (torch.randn(r, N, device=dev, generator=g) * 1e-3).to(torch.bfloat16)
            self.sites.append((M, K, N, r, alpha / r, wq, a, b) + acts[key])
        for (M, K, N, r, *_rest) in sites:
            D.reserve(M, N, K, r)

    def step(self):
        D = self.D
        for (M, K, N, r, s, wq, a, b, x, dy, (y, t, dx, da, db)) in self.sites:
            D.lora_fwd(x, wq, a, b, s, y=y, t=t)
            D.lora_bwd(x, dy, wq, a, b, s, t, out=(dx, da, db))

    def run(self, n):
        for _ in range(n):
            self.step()

    def capture(self):
        """Capture one step into a HIP graph on a side stream (its context's
        workspace reserved first: the library refuses to grow it while
        capturing); ``replay(n)`` then runs n steps with no host launch cost."""
        import torch

        D = self.D
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            for (M, K, N, r, *_r) in self.sites:
                D.reserve(M, N, K, r)
            self.step()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                self.step()
        torch.cuda.synchronize()
        self.graph = graph

    def replay(self, n):
        for _ in range(n):
            self.graph.replay()

    def flops(self):
        return sum(flops_step(M, K, N, r) for (M, K, N, r, *_r) in self.sites)

    def kernel_flops(self):
        """Algorithmic flops of the two fused GEMM kernels per step."""
        f = sum(2.0 * M * N * (K + r) for (M, K, N, r, *_r) in self.sites)
        b = sum(2.0 * M * K * (N + r) for (M, K, N, r, *_r) in self.sites)
        return {"fwd_main": f, "bwd_dx": b}

    def bytes(self, group=64):
        """Algorithmic HBM bytes per step: packed int4 weight and its group
        scales, activations and factors, forward plus backward."""
        tot = 0.0
        for (M, K, N, r, *_r) in self.sites:
            wb = N * K / 2 + 4 * N * K / group
            tot += wb + 2 * M * K + 2 * M * N + 4 * r * (K + N)
            tot += wb + 2 * M * N + 4 * M * K + 8 * r * (K + N)
        return tot

    def check(self):
        import torch

        for (M, K, N, r, s, wq, a, b, x, dy, outs) in self.sites:
            for v in outs:
                if not torch.isfinite(v).all() or not v.abs().max() > 0:
                    raise RuntimeError("implausible output (all-zero or non-finite)")


def profile_kernels(run, n):
    """Per-kernel GPU time of ``run(n)`` from the library's HIP events:
    {kernel: (total ms, launches)} for the kernels that ran."""
    import torch

    from loractl_amd import device as D

    D.profile_reset()
    D.profile_enable(True)
    torch.cuda._sleep(GPU_SPIN_CYCLES)
    run(n)
    torch.cuda.synchronize()
    prof = D.profile_read()
    D.profile_enable(False)
    return {k: v for k, v in prof.items() if v[1]}


def mfma_roofline(prof, kflops, steps, workload):
    """The roofline object of the dominant fused GEMM kernel: its algorithmic
    flops over the profiled steps / its total launch time; `traffic` its
    committed HBM bytes per launch (averaged over the workload's launches of
    it), if profiled."""
    dom = max((k for k in kflops if k in prof), key=lambda k: prof[k][0])
    ms, n = prof[dom]
    achieved = kflops[dom] * steps / (ms * 1e-3) / 1e12
    return {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": load_traffic(dom, workload),
            "flops_per_launch": kflops[dom] * steps / n, "avg_launch_us": round(1e3 * ms / n, 2),
            "launch_time_from": "per-launch HIP event brackets averaged over every site's launches (each "
                                "bracket adds a few microseconds of markers)"}


def cpu_baseline_set(rows, sites, group, budget_s, scale=1.0, what=""):
    """The reference's CPU step (f32 dequant per pass + f32 GEMMs, as
    ``cpu_baseline``) over ``sites`` [(M, K, N, r, alpha)] with their packed
    row-layout weights ``rows``; ``scale`` multiplies the sampled flops to
    the whole workload when the sample is a part of it."""
    import numpy as np

    import oracle as O

    steps = []
    for i, ((M, K, N, r, alpha), (p, sc)) in enumerate(zip(sites, rows)):
        rng = np.random.Generator(np.random.PCG64(100 + i))
        x = rng.standard_normal((M, K), dtype=np.float32)
        dy = rng.standard_normal((M, N), dtype=np.float32)
        a = rng.uniform(-1 / np.sqrt(K), 1 / np.sqrt(K), (K, r)).astype(np.float32)
        b = (rng.standard_normal((r, N), dtype=np.float32) * np.float32(1e-3))
        steps.append(O.CpuStepInt4(p, sc, group, x, a, b, alpha / r, dy))
    for st in steps:
        st.run()
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < budget_s:
        for st in steps:
            st.run()
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    F = sum(flops_step(M, K, N, r) for (M, K, N, r, _a) in sites)
    return {"value": round(F / dt / 1e12, 5), "unit": "TFLOP/s", "cores": O.blas_threads(), "kind": "port",
            "sample": f"{what}{reps} steps of {dt:.3f} s: f32 dequant of each full weight per forward and per "
                      f"backward (OpenMP), then f32 GEMMs in {O.blas_info()}",
            "_seconds_per_step": dt * scale}


def bench_c3(args, dev):
    """C3: one synthetic MMDiT double-stream block's linear set, every site an
    int4 g64 frozen base with LoRA r=32, on the image stream (M=4096) and the
    text stream (M=512, its own weights), forward + backward per step."""
    sites = [(M, K, N, 32, 32.0) for (_name, M) in C3_STREAMS for (K, N) in C3_SITES]
    keep = 0 if args.no_cpu_baseline else len(sites)
    ls = LinearSet(dev, sites, seed=3, keep_rows=keep)
    ls.run(1)
    import torch

    torch.cuda.synchronize()
    ls.check()
    ls.capture()
    ms, ratio, warm_ms = warm_and_time(ls.replay, args.steps, args.warmup)
    ms_step = ms / args.steps
    F = ls.flops()
    value = F / (ms_step * 1e-3) / 1e12
    prof = profile_kernels(ls.run, args.steps)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_set(ls.rows, sites, 64, args.cpu_seconds, what="the whole step (both streams), ")
        cpu.pop("_seconds_per_step")
    print(json.dumps({
        "metric": "int4-base LoRA linear set fwd+bwd TFLOP/s (C3: MMDiT double-stream block)",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (torch seeded; W~N(0,0.02) quantized on device, X,dY~N(0,1), "
                                 "A~U(+-1/sqrt(K)), B~N(0,1e-3))",
        "config": {"workload": "C3: QKV 3072->9216, attn-out 3072->3072, MLP 3072->12288->3072, adaLN "
                               "3072->18432, int4-g64 + LoRA r=32 on each; image stream M=4096 and text stream "
                               "M=512 (own weights), forward+backward; one step replayed from a HIP graph",
                   "parallelism": "single-gpu"},
        "pct_of_mfma_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2), "flops_per_step": F,
        "sanity_x2_ratio": round(ratio, 3), "warm_ms": round(warm_ms, 1),
        "kernels_us": {k: round(1e3 * v[0] / v[1], 2) for k, v in prof.items()},
        "kernel_share": {k: round(v[0] / sum(x[0] for x in prof.values()), 4) for k, v in prof.items()},
        "roofline": mfma_roofline(prof, ls.kernel_flops(), args.steps, "c3"),
        "cpu_baseline": cpu,
    }), flush=True)


def graph_us(fn, reps=50):
    """Microseconds per call of `fn` (GPU work only): `reps` calls captured
    in a HIP graph on a side stream, replayed; the best of three replays."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(reps):
                fn()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / reps)
    return best


def c5_gemm_ceiling(M):
    """The vendor library's bf16 GEMMs (torch.matmul, hipBLASLt) at every C5
    site's forward and input-gradient shapes for M tokens, no dequantization
    and no LoRA: their sum over one step (28 layers), the time a step of the
    plain products would take."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(11)
    per, total = {}, 0.0
    for (K, N) in dict.fromkeys(C5_LAYER):
        w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        wt = w.t().contiguous()
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        dy = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
        f, b = gemm_pair_us(x, w, wt, dy)
        per[f"{K}->{N}"] = {"fwd_us": round(f, 2), "dx_us": round(b, 2)}
        total += (f + b) * C5_LAYER.count((K, N)) * C5_LAYERS
        del w, wt, x, dy
    return total / 1e3, per


def c5_measure(args, dev, Ms, with_cpu=True):
    """C5 at each token count of ``Ms``: the linears of a Qwen3-style 28-layer
    decoder (q/k/v/o/gate/up/down, int4 g64, LoRA r=16), forward + backward
    of every site per step, one step replayed from a HIP graph. Every layer
    has its own weights (3.2 GB blocked, past the Infinity Cache), so the
    few-token end streams HBM. The roofline object is the whole step's (196
    sites, both passes, many kernels): algorithmic flops (m >= 256, MFMA
    bound) or bytes (m <= 16, HBM bound) per step over the step time; the
    per-kernel figures are event-bracketed launch averages over all sites."""
    import torch

    sweep = {}
    for M in Ms:
        sites = [(M, K, N, 16, 16.0) for _layer in range(C5_LAYERS) for (K, N) in C5_LAYER]
        keep = len(C5_LAYER) if with_cpu else 0
        ls = LinearSet(dev, sites, seed=5, keep_rows=keep)
        ls.run(1)
        torch.cuda.synchronize()
        ls.check()
        ls.capture()
        steps = args.steps if M >= 256 else max(args.steps, 20)
        ms, ratio, warm_ms = warm_and_time(ls.replay, steps, args.warmup)
        ms_step = ms / steps
        F = ls.flops()
        B = ls.bytes()
        prof = profile_kernels(ls.run, steps)
        entry = {"ms_per_step": round(ms_step, 4), "tflops": round(F / (ms_step * 1e-3) / 1e12, 2),
                 "gbs": round(B / (ms_step * 1e-3) / 1e9, 1), "flops_per_step": F, "bytes_per_step": B,
                 "sanity_x2_ratio": round(ratio, 3),
                 "kernels_us_events": {k: round(1e3 * v[0] / v[1], 2) for k, v in prof.items()},
                 "launches_per_step": {k: round(v[1] / steps, 2) for k, v in prof.items()}}
        if M >= 256:
            achieved = F / (ms_step * 1e-3) / 1e12
            entry["roofline"] = {"kernel": "whole step (196 sites, forward and backward)", "bound": "mfma",
                                 "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                                 "traffic": load_traffic(f"step_M{M}", "c5"),
                                 "flops_per_step": F, "time_from": "graph replay of the whole step"}
            # the measured ceiling: the same step's plain bf16 GEMMs in the
            # vendor library (the rate at which this step's work would run
            # at their speed, and this step's time as a fraction of theirs)
            ceil_ms, per = c5_gemm_ceiling(M)
            entry["ceiling"] = {"gemm_bf16_hipblaslt": {
                "step_ms": round(ceil_ms, 4), "per_site_us": per,
                "how": "torch.matmul of x[M,K] . W^T and dy[M,N] . W in bf16 at every site's shape, no "
                       "dequantization and no LoRA, summed over the step's 196 sites; " + GEMM_CEILING_HOW}}
            entry["roofline"]["measured_ceiling"] = round(F / (ceil_ms * 1e-3) / 1e12, 2)
            entry["roofline"]["frac_of_measured"] = round(ceil_ms / ms_step, 4)
        else:
            achieved = B / (ms_step * 1e-3) / 1e9
            entry["roofline"] = {"kernel": "whole step (196 weights streamed by both passes)", "bound": "hbm",
                                 "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                 "frac": round(achieved / PEAK_HBM_GBS, 4),
                                 "traffic": load_traffic(f"step_M{M}", "c5"),
                                 "bytes_per_step": B, "time_from": "graph replay of the whole step"}
        if with_cpu:
            c = cpu_baseline_set(ls.rows, sites[:len(C5_LAYER)], 64, args.cpu_seconds / len(Ms),
                                 scale=C5_LAYERS, what=f"1 of {C5_LAYERS} layers at M={M}, ")
            entry["cpu_baseline"] = {k: v for k, v in c.items() if k != "_seconds_per_step"}
        sweep[str(M)] = entry
        del ls
        torch.cuda.empty_cache()
    return sweep


def bench_c5(args, dev):
    sweep = c5_measure(args, dev, C5_M, with_cpu=not args.no_cpu_baseline)
    head = sweep[str(C5_M[-1])]
    print(json.dumps({
        "metric": "int4-base LoRA linear set fwd+bwd TFLOP/s (C5: Qwen3-style decoder linears, M sweep)",
        "value": head["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (torch seeded; W~N(0,0.02) quantized on device, X,dY~N(0,1), "
                                 "A~U(+-1/sqrt(K)), B~N(0,1e-3))",
        "config": {"workload": f"C5: {C5_LAYERS} layers x q/k/v/o/gate/up/down (2560 hidden, 9728 MLP, GQA "
                               f"32q/8kv x 128), int4-g64 + LoRA r=16, forward+backward, one step replayed "
                               f"from a HIP graph; value at M={C5_M[-1]}",
                   "M_sweep": list(C5_M), "parallelism": "single-gpu"},
        "pct_of_mfma_peak": round(100.0 * head["tflops"] / PEAK_BF16_TFLOPS, 2),
        "sweep": sweep, "roofline": head["roofline"], "cpu_baseline": head.get("cpu_baseline"),
    }), flush=True)


def mmdit_measure(args, dev, steps, warmup, with_cpu=True):
    """C4: steps/s of the block-checkpointed synthetic MMDiT LoRA training
    step (loractl_amd.mmdit.checkpointed_step + AdamW on the adapters), one
    step = capture forward, head loss, per-block replay with backward, the
    optimizer step; the loss is read back every step (the reference's
    per-step fence)."""
    import torch

    from loractl_amd import device as D
    from loractl_amd.mmdit import (Mmdit, MmditConfig, build_mmdit_adapters, checkpointed_step, flow_batch,
                                   mmdit_step_flops)

    cfg = MmditConfig()
    img_tokens, txt_tokens = MMDIT_TOKENS
    t0 = time.perf_counter()
    model = Mmdit(cfg, dev, seed=0)
    ad = build_mmdit_adapters(cfg, dev, seed=1)
    setup_s = time.perf_counter() - t0
    batch = flow_batch(cfg, img_tokens, txt_tokens, dev, seed=2)
    params = [p for d in ad.deltas for p in (d.lora_a, d.lora_b)]
    # burn's AdamWConfig defaults (beta 0.9/0.999, eps 1e-5); the trainer's weight decay default 0
    opt = torch.optim.AdamW(params, lr=1e-4, eps=1e-5, weight_decay=0.0, fused=True)
    for (M, (K, N)) in [(m, kn) for m in MMDIT_TOKENS for kn in cfg.site_shapes().values()]:
        D.reserve(M, N, K, cfg.rank)
    losses = []

    keep = [False]  # the config's policy: every block replayed whole

    def step():
        opt.zero_grad(set_to_none=True)
        losses.append(checkpointed_step(model, ad, batch, keep_attention=keep[0]))
        opt.step()

    def run(n):
        for _ in range(n):
            step()

    run(1)
    torch.cuda.synchronize()
    if not all(map(lambda v: v == v and v > 0, losses)):
        raise RuntimeError(f"implausible loss {losses}")
    ms, ratio, warm_ms = warm_and_time(run, steps, warmup)
    ms_step = ms / steps
    fl = mmdit_step_flops(cfg, img_tokens, txt_tokens)
    prof = profile_kernels(run, 1)
    kept = None
    if not getattr(args, "no_mmdit_kept", False):
        # the same model and step with each block's attention output and
        # log-sum-exp kept from the capture (the replay skips that forward)
        keep[0] = True
        kms, kratio, _ = warm_and_time(run, steps, warmup)
        keep[0] = False
        kept = {"value": round(1e3 * steps / kms, 4), "unit": "steps/s", "ms_per_step": round(kms / steps, 2),
                "sanity_x2_ratio": round(kratio, 3),
                "checkpointing": "per block; the capture's attention output and log-sum-exp kept for the replay"}
    fused = {k: v for k, v in prof.items()}
    fused_ms = sum(v[0] for v in fused.values())
    # the fused GEMMs' algorithmic flops per step: two forwards (capture and
    # replay) and one input gradient of every site, LoRA step included
    kflops = {"fwd_main": 0.0, "bwd_dx": 0.0}
    for M in MMDIT_TOKENS:
        for n, (K, N) in cfg.site_shapes().items():
            rows = 1 if n == "mod" else M
            kflops["fwd_main"] += 2 * 2.0 * rows * N * (K + cfg.rank) * cfg.layers
            kflops["bwd_dx"] += 2.0 * rows * K * (N + cfg.rank) * cfg.layers
    out = {
        "metric": "MMDiT train steps/s (C4: 24 double-stream blocks, block checkpointing)",
        "value": round(1e3 / ms_step, 4),
        "unit": "steps/s",
        "ms_per_step": round(ms_step, 2),
        "tflops": round(fl["total"] / (ms_step * 1e-3) / 1e12, 2),
        "flop_model": {k: fl[k] for k in ("proj", "attn", "lora", "total")},
        # the same step's work if the modulation linears ran at the stream's
        # token count, as a work model that treats them like the other
        # projections counts them (not what this step executes)
        "flop_model_mod_at_stream": {
            k: v for k, v in mmdit_step_flops(cfg, img_tokens, txt_tokens, mod_at_stream=True).items()
            if k in ("proj", "total")},
        "flop_model_note": "the modulation (adaLN) linears run on the one conditioning row per batch element, "
                           "as in a FLUX-style double-stream block; a work model that counts them at the "
                           "stream's token count (flop_model_mod_at_stream) adds work this step does not do",
        "checkpointing": "per block, whole-block replay (re-forward in backward)",
        "attention_kept": kept,
        "sanity_x2_ratio": round(ratio, 3),
        "warm_ms": round(warm_ms, 1),
        "setup_s": round(setup_s, 1),
        "loss_first_last": [round(losses[0], 5), round(losses[-1], 5)],
        "fused_kernels_ms_per_step": round(fused_ms, 2),
        "fused_share_of_step": round(fused_ms / ms_step, 4),
        "kernels_ms_per_step": {k: round(v[0], 3) for k, v in fused.items()},
        "roofline": mfma_roofline(prof, kflops, 1, "mmdit"),
        "workload": f"batch 1 of {img_tokens} image + {txt_tokens} text tokens, hidden {cfg.hidden}, {cfg.heads} "
                    f"heads, {cfg.layers} double-stream blocks, MLP x{cfg.mlp_ratio}, int4-g{cfg.group} frozen "
                    f"base and LoRA r={cfg.rank} on all {len(cfg.site_paths())} block linears (modulation on the "
                    f"conditioning vector), AdamW on the adapters, flow-matching MSE with t~U(0,1)",
        "cpu_baseline": None,
    }
    del model, ad, opt, params
    torch.cuda.empty_cache()
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline_mmdit(cfg, img_tokens, txt_tokens, args.cpu_seconds)
    return out


def cpu_baseline_mmdit(cfg, img_tokens, txt_tokens, budget_s):
    """The reference's CPU algorithm for one block of the step, scaled to the
    trunk: the block's ten linears through the f32 dequant + f32 GEMM step
    (dequant per pass: two forwards and one backward under block
    checkpointing) and the attention matmuls (QK^T and PV twice forward,
    their four gradients once) in numpy's SGEMM; norms and elementwise work
    are left out, so the time is an under-count."""
    import numpy as np

    import oracle as O

    rng = np.random.Generator(np.random.PCG64(9))
    sites = []
    for M in (img_tokens, txt_tokens):
        for n, (K, N) in cfg.site_shapes().items():
            rows = 1 if n == "mod" else M
            w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
            p, sc = O.quantize_int4_packed(w, cfg.group)
            x = rng.standard_normal((rows, K), dtype=np.float32)
            dy = rng.standard_normal((rows, N), dtype=np.float32)
            a = rng.uniform(-1 / np.sqrt(K), 1 / np.sqrt(K), (K, cfg.rank)).astype(np.float32)
            b = (rng.standard_normal((cfg.rank, N), dtype=np.float32) * np.float32(1e-3))
            sites.append(O.CpuStepInt4(p, sc, cfg.group, x, a, b, cfg.alpha / cfg.rank, dy))
    L, nh, hd = img_tokens + txt_tokens, cfg.heads, cfg.head_dim
    q, k, v, do = (rng.standard_normal((nh, L, hd), dtype=np.float32) for _ in range(4))

    def attention():
        for _ in range(2):  # capture forward and replay forward
            s_ = q @ k.transpose(0, 2, 1)
            s_ -= s_.max(-1, keepdims=True)
            p_ = np.exp(s_)
            p_ /= p_.sum(-1, keepdims=True)
            o = p_ @ v
        dv = p_.transpose(0, 2, 1) @ do
        dp = do @ v.transpose(0, 2, 1)
        ds = p_ * (dp - (dp * p_).sum(-1, keepdims=True))
        dq = ds @ k
        dk = ds.transpose(0, 2, 1) @ q
        return o, dv, dq, dk

    def block():
        for st in sites:
            st.run()      # forward + backward, each with its own f32 dequant
            st.forward()  # the replay forward of block checkpointing
        attention()

    block()
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < budget_s:
        block()
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    step_s = dt * cfg.layers
    return {"value": round(1.0 / step_s, 6), "unit": "steps/s", "cores": O.blas_threads(), "kind": "port",
            "sample": f"1 of {cfg.layers} blocks ({reps} reps of {dt:.2f} s, times {cfg.layers}): its 10 linears "
                      f"as f32 dequant per pass + f32 GEMMs (2 forwards, 1 backward) and the attention matmuls, "
                      f"in {O.blas_info()}; norms and elementwise work left out"}


def bench_mmdit(args, dev):
    m = mmdit_measure(args, dev, steps=args.steps, warmup=args.warmup, with_cpu=not args.no_cpu_baseline)
    out = {"metric": m.pop("metric"), "value": m.pop("value"), "unit": "steps/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": m.pop("ms_per_step"), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (torch seeded; random-init weights, latents and text embeddings ~N(0,1))",
           "config": {"workload": m.pop("workload"), "parallelism": "single-gpu"}}
    out.update(m)
    print(json.dumps(out), flush=True)


def cpu_baseline_fwd(wq_rows, x, a, b, M, K, N, r, s, group, budget_s, bytes_fwd, fmt="int4"):
    """The reference's CPU forward (f32 dequant of the whole weight, f32
    GEMMs) on the whole few-token workload, on this host's cores;
    ``wq_rows`` is the (packed or int8 q, scales) row layout."""
    import numpy as np

    import oracle as O

    if fmt == "int8":
        st = O.CpuStepInt8(wq_rows[0], wq_rows[1], group, x, a, b, s, np.zeros((M, N), np.float32))
        st.run = st.forward  # forward only
    else:
        st = O.CpuFwdInt4(wq_rows[0], wq_rows[1], group, x, a, b, s)
    t0 = time.perf_counter()
    threads = st.run()
    first = time.perf_counter() - t0
    reps = max(1, int(budget_s / max(first, 1e-3)))
    t0 = time.perf_counter()
    for _ in range(reps):
        st.run()
    dt = (time.perf_counter() - t0) / reps
    return {
        "value": round(bytes_fwd / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"the whole workload (M={M}, {K}->{N} r={r} {fmt}-g{group}), forward, {reps} reps of {dt:.4f} s "
                  f"(f32 dequant of the full weight + f32 GEMMs, OpenMP)",
    }


def cpu_baseline(wq_rows, x, a, b, dy, M, K, N, r, s, group, fmt, budget_s):
    """The reference's CPU algorithm (burn-ndarray, f32) on the whole step of
    the same layer, on this host's cores: int4 dequantizes the whole weight
    to f32 on every forward and every backward (quant.rs:232, :250), fp8 is
    an f32 weight decoded once at load (fp8.rs:306-318, kept Plain); then
    the f32 GEMMs of the forward and backward in numpy's cache-blocked SGEMM.
    Steps are repeated for about ``budget_s`` seconds."""
    import oracle as O

    if fmt == "int4":
        st = O.CpuStepInt4(wq_rows[0], wq_rows[1], group, x, a, b, s, dy)
        what = "f32 dequant of the full weight per forward and per backward (OpenMP), then f32 GEMMs"
    elif fmt == "int8":
        st = O.CpuStepInt8(wq_rows[0], wq_rows[1], group, x, a, b, s, dy)
        what = "f32 dequant of the full int8 weight per forward and per backward (OpenMP), then f32 GEMMs"
    else:
        st = O.CpuStepF32(O.fp8_dequant(wq_rows[0], wq_rows[1]), x, a, b, s, dy)
        what = "f32 weight decoded once at load, f32 GEMMs"
    st.run()  # first touch of the work buffers
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < budget_s:
        st.run()
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    F = flops_step(M, K, N, r)
    return {
        "value": round(F / dt / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": O.blas_threads(),
        "kind": "port",
        "sample": f"the whole step (M={M}, {K}->{N} r={r} {fmt}{'' if fmt == 'fp8' else '-g' + str(group)}), fwd+bwd, "
                  f"{reps} steps of {dt:.3f} s: {what} in {O.blas_info()}",
    }


if __name__ == "__main__":
    main()
