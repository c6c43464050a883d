#!/usr/bin/env python3
"""Benchmark of the MI355X attention + W4 linear hot path (one GPU).

Headline: DiT self-attention at S=4096 (1x64x64 patch grid), B=1, H=16, D=128,
fp16 in/out, per-head RMSNorm on Q/K and 3-D RoPE fused in — TFLOP/s and the
fraction of the fp16 dense MFMA peak — plus ms per full DiT block (hidden 2048,
S=4096, 512-token context, all ten linears W4 group-64).

One "step" = one attention call on fresh synthetic inputs already resident in
HBM (8 rotating input sets, 512 MiB, twice the 256 MB Infinity Cache, so it does not
hold a step's inputs).  Prints ONE JSON line.  The CPU baseline is the repository's
torch-CPU fp32 oracle timed on the same workload on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "DiT self-attn TFLOP/s + % fp16 MFMA peak at S=4096; ms per DiT block (1 GPU)"
FP16_PEAK_TFLOPS = 2516.6   # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
HBM_PEAK_GBS = 8000.0
B, H, D, S = 1, 16, 128, 4096
SIDE = 64


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--block-steps", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-table", action="store_true",
                    help="also time the oracle on all five workloads (C1-C5, incl. ms per DiT block) at all threads "
                         "and at 4 threads, median of 5 after 1 warm-up (several minutes of CPU work)")
    ap.add_argument("--no-block", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the per-workload table")
    ap.add_argument("--profile-block", action="store_true",
                    help="only run the S=4096 DiT block (--block-steps times), for a rocprofv3 kernel trace")
    ap.add_argument("--profile-step", action="store_true",
                    help="only the 1024px sampler step (for a kernel trace of the whole step)")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only launch the dominant flash kernel (--warmup + --steps times) and a 256 MiB "
                         "calibration copy, for rocprofv3 counter passes; prints no JSON")
    ap.add_argument("--profile-gemm", metavar="M,N,K",
                    help="only launch the W4 GEMM of this shape over rotating weight sets (> 600 MB), settle + "
                         "--warmup + --steps times, then the calibration copies; for rocprofv3 counter passes")
    ap.add_argument("--profile-vae", action="store_true",
                    help="only the VAE mid-block attention (1 head, head_dim 384, 4096 positions), settle + "
                         "--warmup + --steps calls; for a rocprofv3 kernel trace")
    ap.add_argument("--profile-c1", action="store_true",
                    help="only workload 1 (S=1024 self-attention, key splits + merge), settle + --warmup + --steps "
                         "calls, then the calibration copies; for rocprofv3")
    ap.add_argument("--profile-c3", action="store_true",
                    help="only workload 3 (B4 masked cross attention), settle + --warmup + --steps calls, then the "
                         "calibration copies; for rocprofv3")
    ap.add_argument("--counter-summary", metavar="CSV",
                    help="no GPU: per-dispatch means of a rocprofv3 --pmc counter_collection.csv, per kernel "
                         "(last --trace-last dispatches of each) and exit")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="no GPU: summarise a rocprofv3 kernel_trace.csv (per kernel: dispatches, mean/median/p10/p90 "
                         "of the last --trace-last dispatches) and exit")
    ap.add_argument("--trace-last", type=int, default=0, help="with --trace-summary: only the last N dispatches of "
                    "each kernel (the timed ones; 0 = all)")
    ap.add_argument("--trace-order", type=int, default=0,
                    help="with --trace-summary: list the last N dispatches of the whole trace in launch order instead")
    return ap.parse_args()


def counter_summary(path, last):
    """Per kernel: mean / min / max over its last ``last`` dispatches of every counter in a
    rocprofv3 --pmc counter_collection.csv (one row per dispatch and counter, the value
    already summed over the counter's instances)."""
    import csv
    import numpy as np
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            k = per.setdefault(r["Kernel_Name"], {})
            k.setdefault(r["Counter_Name"], []).append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    print("| kernel | counter | dispatches | summarised | mean per dispatch | min | max |")
    print("|---|---|---|---|---|---|---|")
    for name, counters in per.items():
        for cname, v in sorted(counters.items()):
            v.sort()
            d = np.array([x[1] for x in (v[-last:] if last else v)])
            print(f"| `{name[:70]}` | {cname} | {len(v)} | {len(d)} | {d.mean():.1f} | {d.min():.1f} | {d.max():.1f} |")


def trace_summary(path, last, order=0):
    """Per-kernel durations from a rocprofv3 --kernel-trace CSV (Kernel_Name,
    Start_Timestamp, End_Timestamp in ns); with ``order`` the last ``order`` dispatches
    in launch order (start offset from the first of them, duration, grid, kernel)."""
    import csv
    import numpy as np
    if order:
        with open(path) as f:
            rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))[-order:]
        t0 = int(rows[0]["Start_Timestamp"])
        print("| start us | duration us | grid (threads) | kernel |")
        print("|---|---|---|---|")
        for r in rows:
            st, en = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            grid = r.get("Grid_Size_X") or r.get("Grid_Size") or "?"
            print(f"| {(st - t0) / 1e3:.1f} | {(en - st) / 1e3:.2f} | {grid} | `{r['Kernel_Name'][:80]}` |")
        last_end = max(int(r["End_Timestamp"]) for r in rows)
        print(f"\nspan {(last_end - t0) / 1e3:.1f} us, kernel time {sum(int(r['End_Timestamp']) - int(r['Start_Timestamp']) for r in rows) / 1e3:.1f} us")
        return
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            per.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]),
                                                         int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    rows = []
    for name, v in per.items():
        v.sort()
        d = np.array([x[1] for x in (v[-last:] if last else v)], dtype=np.float64) / 1e3
        rows.append((d.sum(), name, len(v), len(d), d.mean(), np.median(d), np.percentile(d, 10), np.percentile(d, 90)))
    rows.sort(reverse=True)
    print("| kernel | dispatches | summarised | mean us | median us | p10 us | p90 us |")
    print("|---|---|---|---|---|---|---|")
    for _, name, n, k, mean, med, p10, p90 in rows:
        print(f"| `{name[:90]}` | {n} | {k} | {mean:.2f} | {med:.2f} | {p10:.2f} | {p90:.2f} |")


def attn_flops(Sq, Sk, heads=H, batch=B, d=D):
    return 4.0 * batch * heads * Sq * Sk * d


def gen_attention_inputs(torch, sets, seed=1002):
    """Workload: Q/K/V ~N(0,1) fp16 [1,4096,16,128], norm weights ~U(0.8,1.2)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    out = []
    for _ in range(sets):
        q = torch.randn(B, S, H, D, device="cuda", generator=g).half()
        k = torch.randn(B, S, H, D, device="cuda", generator=g).half()
        v = torch.randn(B, S, H, D, device="cuda", generator=g).half()
        o = torch.empty(B, S, H, D, device="cuda", dtype=torch.float16)
        out.append((q, k, v, o))
    qw = (0.8 + 0.4 * torch.rand(D, device="cuda", generator=g)).half()
    kw = (0.8 + 0.4 * torch.rand(D, device="cuda", generator=g)).half()
    return out, qw, kw


def settle_clock(torch, fn, seconds=0.03, rest=0.3):
    """Untimed: give every timed region the same starting state.  The part first rests for
    `rest` seconds (after tens of milliseconds of back-to-back launches its clock steps
    down), then runs fn back to back for about `seconds` (the first region after idle
    otherwise runs ~10 % slower while the clock ramps up)."""
    import time
    torch.cuda.synchronize()
    time.sleep(rest)
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(16):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def time_region(torch, stream, fn, steps, warmup, settle=True):
    if settle:
        settle_clock(torch, fn)
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def time_calls(torch, stream, fn, calls, warmup, settle=True):
    """Two timed passes of ``calls`` back-to-back calls after one settle + warm-up:
    one event pair around the whole pass (the mean, nothing between the calls), then
    an event after every call (per-call durations: median, p10, p90).  Returns a dict
    in ms."""
    import numpy as np
    mean = time_region(torch, stream, fn, calls, warmup, settle)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(calls + 1)]
    evs[0].record(stream)
    for i in range(calls):
        fn(i)
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(calls)])
    return {"mean_ms": round(mean, 5), "median_ms": round(float(np.median(per)), 5),
            "p10_ms": round(float(np.percentile(per, 10)), 5), "p90_ms": round(float(np.percentile(per, 90)), 5),
            "calls": calls}


def time_graph(torch, ctx, fn, calls, reps=5):
    """ms per call of ``calls`` back-to-back encodes captured once into a HIP graph and
    replayed ``reps`` times (events on the replay stream)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ctx.set_stream(side)
        for i in range(calls):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.set_stream(torch.cuda.current_stream())
        for i in range(calls):
            fn(i)
    main_stream = torch.cuda.current_stream()
    ctx.set_stream(main_stream)
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(main_stream)
    for _ in range(reps):
        g.replay()
    end.record(main_stream)
    torch.cuda.synchronize()
    del g
    return start.elapsed_time(end) / (reps * calls)


def main():
    args = parse()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.trace_last, args.trace_order)
        return
    if args.counter_summary:
        counter_summary(args.counter_summary, args.trace_last)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the attention/W4 hot path is "
              "benchmarked per GPU and multi-GPU sharding is a design note, not a measured mode.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import animaxs_amd as A

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.init()
    dev_name = torch.cuda.get_device_name(0)
    stream = torch.cuda.current_stream()
    ctx = A.Context(0, stream)
    print(f"# device {dev_name}", file=sys.stderr, flush=True)

    if args.profile_block:
        blk = time_block(torch, A, ctx, stream, args)
        print(f"# profile-block: DiT block S4096 {blk['ms']:.3f} ms ({blk['timing']})", file=sys.stderr)
        return
    if args.profile_gemm:
        profile_gemm(torch, A, ctx, stream, args, *(int(x) for x in args.profile_gemm.split(",")))
        return
    if args.profile_vae:
        ms = time_region(torch, stream, vae_attention_call(torch, A, ctx), args.steps, args.warmup)
        print(f"# profile-vae: {ms * 1e3:.2f} us per call (HIP events, {args.steps} timed calls)", file=sys.stderr)
        return
    if args.profile_c1 or args.profile_c3:
        fn = c1_call(torch, A, ctx) if args.profile_c1 else c3_call(torch, A, ctx)[0]
        ms = time_region(torch, stream, fn, args.steps, args.warmup)
        calibration_copies(torch)
        print(f"# profile-{'c1' if args.profile_c1 else 'c3'}: {ms * 1e3:.2f} us per call (HIP events, {args.steps} "
              "timed calls), then 3 x 256 MiB copies", file=sys.stderr)
        return
    if args.profile_step:
        st_ms, first_ms, fwd_ms, finite, streamed = time_sampler_step(torch, A, ctx, stream, args)
        print(f"# profile-step: sampler step 1024px {st_ms:.3f} ms (first {first_ms:.3f} ms, 28-block forward "
              f"{fwd_ms:.3f} ms, velocity finite {finite}); streamed forward {streamed}", file=sys.stderr)
        return

    # ---------------- headline: S=4096 self-attention with fused norm+RoPE ----------------
    sets, qw, kw = gen_attention_inputs(torch, 8)
    rope = torch.from_numpy(A.DitRoPE.generate(1, SIDE, SIDE)).cuda()
    pro = A.QKPrologue(qw, kw, 1e-6, rope, S, True, True)
    ex = A.AttentionExecutor(ctx, layout=("tokenMajor", H * D), backend="flash")

    def step(i):
        q, k, v, o = sets[i % len(sets)]
        ex.encode(query=q, key=k, value=v, output=o, heads=H, query_count=S, key_count=S, head_dim=D, prologue=pro)

    flops = attn_flops(S, S)
    if not args.profile_kernel:
        step_t = time_calls(torch, stream, step, args.steps, args.warmup)
        ms = step_t["mean_ms"]
        tflops = flops / (ms * 1e-3) / 1e12
        print(f"# self-attn S4096 (norm+rope, incl. K prologue): {step_t}  {tflops:.1f} TFLOP/s", file=sys.stderr,
              flush=True)

    # Dominant kernel alone: the flash kernel with Q norm+RoPE fused and K given already
    # normalised (torch maths on device, input preparation only), so each encode is
    # exactly one flash launch and the event pair brackets back-to-back launches.
    pro_q = A.QKPrologue(qw, None, 1e-6, rope, S, True, False)
    knorm = []
    c_ = rope[:, :, 0, 0][None, :, None, :]
    s_ = rope[:, :, 1, 0][None, :, None, :]
    for (q, k, v, o) in sets:
        kf = k.float()
        kf = kf * torch.rsqrt(kf.pow(2).mean(-1, keepdim=True) + 1e-6) * kw.float()
        a, bb = kf[..., :64], kf[..., 64:]
        knorm.append(torch.cat([c_ * a - s_ * bb, s_ * a + c_ * bb], dim=-1).half().contiguous())

    def kstep(i):
        q, k, v, o = sets[i % len(sets)]
        ex.encode(query=q, key=knorm[i % len(sets)], value=v, output=o, heads=H, query_count=S, key_count=S,
                  head_dim=D, prologue=pro_q)

    if args.profile_kernel:
        # The same timed region as the normal run, so the trace's average duration of
        # these launches can be set beside the live HIP-event figure printed here.
        kms = time_region(torch, stream, kstep, args.steps, args.warmup)
        print(f"# profile-kernel: flash kernel alone {kms:.4f} ms (HIP events, {args.steps} timed launches)",
              file=sys.stderr, flush=True)
        calibration_copies(torch)
        print(f"# profile-kernel: settle launches, then {args.warmup} warmup + {args.steps} timed flash launches, "
              "3 x 256 MiB copies", file=sys.stderr)
        return

    kern_t = time_calls(torch, stream, kstep, args.steps, args.warmup)
    kms = kern_t["mean_ms"]
    k_tflops = flops / (kms * 1e-3) / 1e12
    print(f"# flash kernel alone: {kern_t}  {k_tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)

    roofline = {
        "bound": "mfma", "kernel": "flash_attention_v2_kernel<128>", "achieved": round(k_tflops, 2),
        "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(k_tflops / FP16_PEAK_TFLOPS, 4),
        "traffic": load_traffic(), "flops_per_launch": flops, "avg_launch_ms": round(kms, 5),
        "launch_timing": kern_t,
    }

    extra = {}
    if not args.no_extra:
        extra = other_workloads(torch, A, ctx, stream, args)

    block_ms = None
    if not args.no_block:
        blk = time_block(torch, A, ctx, stream, args)
        block_ms = blk["ms"]
        extra["dit_block_s4096"] = blk
        print(f"# DiT block S4096: {blk}", file=sys.stderr, flush=True)
        qwen = time_qwen_layer(torch, A, ctx, stream, args)
        extra["qwen_layer_b4_s512"] = qwen
        print(f"# Qwen layer B4 S512: {qwen}", file=sys.stderr, flush=True)
        st_ms, first_ms, fwd_ms, finite, streamed = time_sampler_step(torch, A, ctx, stream, args)
        extra["forward_28_blocks_streamed"] = streamed
        print(f"# streamed 28-block forward: {streamed}", file=sys.stderr, flush=True)
        extra["sampler_step_1024px"] = {
            "ms": round(st_ms, 3), "first_step_ms": round(first_ms, 3), "forward_28_blocks_ms": round(fwd_ms, 3),
            "ms_per_block": round(fwd_ms / 28, 4), "generation_8_steps_ms": round(first_ms + 7 * st_ms, 2),
            "velocity_finite": finite,
            "includes": "DiT preparation + 28 W4 blocks (cross K/V cached after step 1) + final layer + "
                        "flow-to-denoised + Euler; weights resident"}
        print(f"# sampler step 1024px: {extra['sampler_step_1024px']}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
        if args.cpu_table:
            cpu["table"] = cpu_table()

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "step_timing": step_t,
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "dit_self_attention_1024px", "batch": B, "heads": H, "head_dim": D, "seq_len": S,
                   "qk_rmsnorm": True, "rope": "dit3d 1x64x64", "layout": "token-major stride 2048",
                   "includes": "K RMSNorm+RoPE prologue kernel + flash kernel (Q norm+RoPE fused)"},
        "mfma_peak_frac": round(tflops / FP16_PEAK_TFLOPS, 4),
        "dit_block_ms": None if block_ms is None else round(block_ms, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "workloads": extra,
        "device": dev_name,
    }
    print(json.dumps(line), flush=True)


def vae_attention_call(torch, A, ctx, sets=4):
    """VAE decoder mid-block attention: one head, head_dim 384, 4096 positions (64x64
    latent), Q/K/V contiguous [4096, 384] fp16 (VAEDecoder.swift:396-404); rotating sets."""
    g = torch.Generator(device="cuda")
    g.manual_seed(1009)
    vsets = [tuple(torch.randn(4096, 384, device="cuda", generator=g).half() for _ in range(3)) for _ in range(sets)]
    vo = torch.empty(4096, 384, device="cuda", dtype=torch.float16)
    exv = A.AttentionExecutor(ctx, layout="headMajor", backend="flash")

    def call(i):
        q, k, v = vsets[i % sets]
        exv.encode(query=q, key=k, value=v, output=vo, heads=1, query_count=4096, key_count=4096, head_dim=384)
    return call


def calibration_copies(torch):
    """A plain device copy of known size (256 MiB read + 256 MiB written), three times:
    the reference point for the memory-traffic counters."""
    src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def read_floor_ms(torch, A, ctx, nbytes, nsets):
    """ms per call of a plain streaming read of ``nbytes`` (the library's read probe),
    rotating over ``nsets`` disjoint buffers and replayed from a HIP graph exactly like the
    small-M GEMM it is the floor of."""
    per = -(-nbytes // 256) * 256
    buf = torch.empty(per * nsets, dtype=torch.uint8, device="cuda")
    buf.random_(0, 256)
    sink = torch.empty(A.read_probe_sink_bytes(per), dtype=torch.uint8, device="cuda")
    nb = -(-nbytes // 16) * 16
    ms = time_graph(torch, ctx, lambda i: A.read_probe(ctx, buf, nb, sink, src_offset=(i % nsets) * per), nsets)
    del buf
    return ms


def gemm_weight_sets(torch, A, N, K, min_bytes=600 << 20):
    """Rotating W4 weight sets (random codes, group-64 scales, zero = -8 * scale) whose
    total exceeds the 256 MB Infinity Cache."""
    wbytes = N * K // 2
    nsets = max(1, min(512, -(-min_bytes // wbytes)))
    ws = []
    for _ in range(nsets):
        p = torch.randint(0, 256, (N, K // 2), device="cuda", dtype=torch.uint8)
        sc = (0.005 + 0.015 * torch.rand(N, K // 64, device="cuda")).half()
        z = (-8 * sc.float()).half()
        ws.append((A.QuantizedLinearWeightBuffers(0, p, sc, z, N, K, K // 2), p, sc, z))
    return ws


def profile_gemm(torch, A, ctx, stream, args, M, N, K):
    lin = A.LinearExecutor(ctx)
    ws = gemm_weight_sets(torch, A, N, K)
    x = torch.randn(M, K, device="cuda").half()
    y = torch.empty(M, N, device="cuda", dtype=torch.float16)
    ms = time_region(torch, stream, lambda i: lin.encode(x, ws[i % len(ws)][0], y, M), args.steps, args.warmup)
    print(f"# profile-gemm M{M} N{N} K{K}: {ms * 1e3:.2f} us per launch (HIP events, {args.steps} timed launches "
          f"over {len(ws)} weight sets)", file=sys.stderr, flush=True)
    calibration_copies(torch)


def load_traffic():
    """HBM bytes per flash launch from the committed rocprofv3 --pmc summary, or None."""
    p = os.path.join(ROOT, "profiles", "flash_attention_v2_s4096_traffic.md")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    return None


def c1_call(torch, A, ctx):
    """Workload 1: DiT self-attention at 512 px, B1 H16 D128 S1024, no norm / RoPE."""
    g = torch.Generator(device="cuda")
    g.manual_seed(1001)
    q, k, v = (torch.randn(1, 1024, H, D, device="cuda", generator=g).half() for _ in range(3))
    o = torch.empty_like(q)
    ex = A.AttentionExecutor(ctx, layout=("tokenMajor", H * D), backend="flash")
    return lambda i: ex.encode(query=q, key=k, value=v, output=o, heads=H, query_count=1024, key_count=1024,
                               head_dim=D)


def c3_call(torch, A, ctx):
    """Workload 3: DiT cross attention, B4, 4096 queries over 512 context keys with per-image
    key lengths, per-head Q/K RMSNorm; 4 rotating input sets.  Returns (call, lengths, norm weight)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(1003)
    sets = []
    for _ in range(4):
        q = torch.randn(4, 4096, H, D, device="cuda", generator=g).half()
        k = torch.randn(4, 512, H, D, device="cuda", generator=g).half()
        v = torch.randn(4, 512, H, D, device="cuda", generator=g).half()
        sets.append((q, k, v, torch.empty_like(q)))
    nw = (0.8 + 0.4 * torch.rand(D, device="cuda", generator=g)).half()
    lengths = torch.randint(77, 513, (4,), generator=torch.Generator().manual_seed(1003)).int().numpy()
    pro = A.QKPrologue(nw, nw, 1e-6, None, 0, False, False)
    ex3 = A.AttentionExecutor(ctx, layout=("tokenMajor", H * D), backend="flash")

    def s3(i):
        q, k, v, o = sets[i % 4]
        ex3.encode(query=q, key=k, value=v, output=o, heads=H, query_count=4096, key_count=512, head_dim=D, batch=4,
                   key_lengths=lengths, prologue=pro)
    return s3, lengths, nw


def other_workloads(torch, A, ctx, stream, args):
    """ms/call and throughput of the other attention workloads (parity configs) and the
    small-M W4 GEMMs, each against its binding roofline."""
    res = {}
    g = torch.Generator(device="cuda")
    # workload 1: S=1024 plain self-attention
    t = time_calls(torch, stream, c1_call(torch, A, ctx), args.steps, args.warmup)
    ms = t["mean_ms"]
    f = attn_flops(1024, 1024)
    res["self_attention_s1024"] = {"ms": round(ms, 5), "tflops": round(f / ms / 1e9, 2),
                                   "mfma_frac": round(f / ms / 1e9 / FP16_PEAK_TFLOPS, 4), "timing": t}
    # workload 3: cross attention B4, 4096 queries, 512 keys, masked, q/k RMSNorm
    s3, lengths, nw = c3_call(torch, A, ctx)
    t = time_calls(torch, stream, s3, args.steps, args.warmup)
    ms = t["mean_ms"]
    L = [int(x) for x in lengths]
    f = sum(4.0 * H * 4096 * l * D for l in L)
    byts = 2.0 * (4 * 4096 * H * D * 2) + sum(2.0 * l * H * D * 2 for l in L)
    res["cross_attention_b4_masked"] = {"ms": round(ms, 5), "tflops": round(f / ms / 1e9, 2),
                                        "gbs": round(byts / ms / 1e6, 1), "key_lengths": L,
                                        "hbm_frac": round(byts / ms / 1e6 / HBM_PEAK_GBS, 4),
                                        "mfma_frac": round(f / ms / 1e9 / FP16_PEAK_TFLOPS, 4), "timing": t}
    # workload 4: Qwen causal GQA B4 S512, head-major, norm + rope 1e6, right padding
    g.manual_seed(1004)
    qh = torch.randn(4, 16, 512, D, device="cuda", generator=g).half()
    kh = torch.randn(4, 8, 512, D, device="cuda", generator=g).half()
    vh = torch.randn(4, 8, 512, D, device="cuda", generator=g).half()
    oh = torch.empty_like(qh)
    rq = torch.from_numpy(A.qwen_rope(512)).cuda()
    lens = torch.randint(8, 513, (4,), generator=torch.Generator().manual_seed(1004)).int().numpy()
    pro4 = A.QKPrologue(nw, nw, 1e-6, rq, 512, True, True)
    ex4 = A.AttentionExecutor(ctx, layout="headMajor", backend="flash")
    t = time_calls(torch, stream, lambda i: ex4.encode(query=qh, key=kh, value=vh, output=oh, heads=16, query_count=512,
                                                       key_count=512, head_dim=D, key_value_heads=8, causal=True,
                                                       batch=4, key_lengths=lens, prologue=pro4),
                   args.steps, args.warmup)
    ms = t["mean_ms"]
    pairs = sum(sum(min(i + 1, int(l)) for i in range(512)) for l in lens)
    f = 4.0 * D * 16 * pairs
    byts = (4 * 16 * 512 * D * 2) * 2 + (4 * 8 * 512 * D * 2) * 2
    res["qwen_causal_gqa_b4_s512_per_layer"] = {"ms": round(ms, 5), "tflops": round(f / ms / 1e9, 2),
                                                "gbs": round(byts / ms / 1e6, 1),
                                                "hbm_frac": round(byts / ms / 1e6 / HBM_PEAK_GBS, 4),
                                                "mfma_frac": round(f / ms / 1e9 / FP16_PEAK_TFLOPS, 4),
                                                "key_lengths": [int(x) for x in lens], "timing": t}
    # VAE decoder mid-block attention: one head, head_dim 384, 4096 positions (64x64 latent),
    # Q/K/V contiguous [4096, 384] (VAEDecoder.swift:396-404); 4 rotating input sets
    t = time_calls(torch, stream, vae_attention_call(torch, A, ctx), args.steps, args.warmup)
    ms = t["mean_ms"]
    f = attn_flops(4096, 4096, heads=1, d=384)
    res["vae_attention_hd384_s4096"] = {"ms": round(ms, 5), "tflops": round(f / ms / 1e9, 2),
                                        "mfma_frac": round(f / ms / 1e9 / FP16_PEAK_TFLOPS, 4), "timing": t}
    # LLM-adapter attention: 16 heads x head_dim 64 over 512 target tokens, 512 context
    # tokens, per-head RMSNorm on both sides, separate Q / K RoPE tables (theta 1e4)
    # (LLMAdapterMetal.swift:360-405)
    g.manual_seed(1010)
    qa, ka, va = (torch.randn(1, 512, 16, 64, device="cuda", generator=g).half() for _ in range(3))
    oa = torch.empty_like(qa)
    wa = (0.8 + 0.4 * torch.rand(64, device="cuda", generator=g)).half()
    ra = torch.from_numpy(A.qwen_rope(512, head_dim=64, theta=1.0e4)).cuda()
    proa = A.QKPrologue(wa, wa, 1e-6, ra, 512, True, True, k_rope=ra, k_rope_tokens=512)
    exa = A.AttentionExecutor(ctx, layout=("tokenMajor", 1024), backend="flash")
    t = time_calls(torch, stream, lambda i: exa.encode(query=qa, key=ka, value=va, output=oa, heads=16, query_count=512,
                                                       key_count=512, head_dim=64, prologue=proa),
                   args.steps, args.warmup)
    ms = t["mean_ms"]
    f = attn_flops(512, 512, heads=16, d=64)
    res["adapter_attention_hd64_512x512"] = {"ms": round(ms, 5), "tflops": round(f / ms / 1e9, 2),
                                             "mfma_frac": round(f / ms / 1e9 / FP16_PEAK_TFLOPS, 4), "timing": t}
    # W4 GEMMs.  Small M is HBM-bound on the weight stream: each timed pass rotates
    # over weight sets totalling > 512 MB (so the 256 MB Infinity Cache cannot hold
    # them) and is replayed from a HIP graph, so the figure is the GPU's back-to-back
    # kernel throughput rather than the host's launch rate.
    lin = A.LinearExecutor(ctx)
    shapes = [(M, N, K) for M in (1, 16, 64) for (N, K) in ((2048, 2048), (8192, 2048), (2048, 8192))]
    shapes += [(4096, 2048, 2048), (4096, 8192, 2048)]
    for (M, N, K) in shapes:
        ws = gemm_weight_sets(torch, A, N, K)
        nsets = len(ws)
        x = torch.randn(M, K, device="cuda").half()
        y = torch.empty(M, N, device="cuda", dtype=torch.float16)
        call = lambda i: lin.encode(x, ws[i % nsets][0], y, M)
        if M <= 64:
            ms = time_graph(torch, ctx, call, nsets)
        else:
            ms = time_region(torch, stream, call, max(args.steps, nsets), args.warmup)
        byts = N * K / 2 + 2 * 2 * N * (K // 64) + 2 * M * K + 2 * M * N
        f = 2.0 * M * N * K
        entry = {"ms": round(ms, 5), "gbs": round(byts / ms / 1e6, 1),
                 "hbm_frac": round(byts / ms / 1e6 / HBM_PEAK_GBS, 4),
                 "tflops": round(f / ms / 1e9, 2),
                 "mfma_frac": round(f / ms / 1e9 / FP16_PEAK_TFLOPS, 4)}
        del ws
        if M <= 64:
            floor_ms = read_floor_ms(torch, A, ctx, int(byts), nsets)
            entry["copy_floor_us"] = round(floor_ms * 1e3, 3)
            entry["copy_floor_gbs"] = round(byts / floor_ms / 1e6, 1)
            entry["vs_copy_floor"] = round(ms / floor_ms, 3)
        res[f"w4_gemm_m{M}_n{N}_k{K}"] = entry
    for k_, v_ in res.items():
        print(f"# {k_}: {v_}", file=sys.stderr, flush=True)
    return res


def time_block(torch, A, ctx, stream, args):
    """ms per DiT block at S=4096 (all linears W4 symmetric int4, group 64)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(1005)
    dim, hidden, T, C = 2048, 8192, 512, 1024
    keep = []

    def w4(n, k):
        p = torch.randint(0, 256, (n, k // 2), device="cuda", generator=g, dtype=torch.uint8)
        sc = (0.005 + 0.015 * torch.rand(n, k // 64, device="cuda", generator=g)).half()
        z = (-8 * sc.float()).half()
        keep.extend([p, sc, z])
        return A.QuantizedLinearWeightBuffers(0, p, sc, z, n, k, k // 2)

    def f16(n, k):
        w = (0.02 * torch.randn(n, k, device="cuda", generator=g)).half()
        keep.append(w)
        return A.QuantizedLinearWeightBuffers(2, w, w, w, n, k, k)

    shapes = {"self_q": (dim, dim), "self_k": (dim, dim), "self_v": (dim, dim), "self_o": (dim, dim),
              "cross_q": (dim, dim), "cross_k": (dim, C), "cross_v": (dim, C), "cross_o": (dim, dim),
              "mlp1": (hidden, dim), "mlp2": (dim, hidden)}

    def block_weights():
        weights = {n: w4(*s) for n, s in shapes.items()}
        for br in ("self", "cross", "mlp"):
            weights[f"mod_{br}_w1"] = f16(256, dim)
            weights[f"mod_{br}_w2"] = f16(3 * dim, 256)
        return weights

    # Eight weight sets (about 8 x 38 MB, more than the 256 MB Infinity Cache) taken in turn,
    # as consecutive blocks of the forward read different weights from HBM.
    wsets = [block_weights() for _ in range(8)]
    norms = {n: (0.8 + 0.4 * torch.rand(128, device="cuda", generator=g)).half()
             for n in ("self_q_norm", "self_k_norm", "cross_q_norm", "cross_k_norm")}
    residual = torch.randn(S, dim, device="cuda", generator=g)
    emb = torch.randn(dim, device="cuda", generator=g)
    adaln = torch.randn(3 * dim, device="cuda", generator=g)
    ctxt = torch.randn(T, C, device="cuda", generator=g).half()
    rope = torch.from_numpy(A.DitRoPE.generate(1, SIDE, SIDE)).cuda()
    blk = A.DiTBlockExecutor(ctx)

    def step(i):
        blk.encode(wsets[i % len(wsets)], norms, residual, emb, adaln, ctxt, rope, tokens=S)

    t = time_calls(torch, stream, step, max(args.block_steps, 16), 2)
    f = block_flops()
    return {"ms": t["mean_ms"], "tflops": round(f / t["mean_ms"] / 1e9, 2),
            "mfma_frac": round(f / t["mean_ms"] / 1e9 / FP16_PEAK_TFLOPS, 4), "gflop": round(f / 1e9, 2),
            "weight_sets": len(wsets), "timing": t}


def block_flops(S_=4096, T=512, dim=2048, C=1024, hidden=8192, heads=16, hd=128):
    """Algorithmic FLOPs of one DiT block: the ten linears plus self and cross attention."""
    lin = 2 * S_ * dim * dim * 6 + 2 * T * dim * C * 2 + 2 * S_ * dim * hidden * 2
    att = 4 * heads * hd * S_ * S_ + 4 * heads * hd * S_ * T
    return float(lin + att)


def time_sampler_step(torch, A, ctx, stream, args, blocks=28):
    """One denoising step of the 1024px configuration (DiffusionSampler.swift:212-250):
    DiTPreparation on the [16, 128, 128] latent (4096 tokens) -> 28 DiT blocks (all ten
    linears W4, cross-attention K/V from the cache) -> final layer -> flow-to-denoised ->
    Euler.  Returns (ms per step with the cache filled, ms of the first step that fills
    it, ms of the 28-block forward alone, velocity finite)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(1008)
    dim, hidden, T, C, side = 2048, 8192, 512, 1024, 128
    keep = []

    def w4(n, k):
        st, gr = (k + 1) // 2, (k + 63) // 64
        p = torch.randint(0, 256, (n, st), device="cuda", generator=g, dtype=torch.uint8)
        sc = (0.005 + 0.015 * torch.rand(n, gr, device="cuda", generator=g)).half()
        z = (-8 * sc.float()).half()
        keep.extend([p, sc, z])
        return A.QuantizedLinearWeightBuffers(0, p, sc, z, n, k, st)

    def f16(n, k):
        w = (0.02 * torch.randn(n, k, device="cuda", generator=g)).half()
        keep.append(w)
        return A.QuantizedLinearWeightBuffers(2, w, w, w, n, k, k)

    shapes = {"self_q": (dim, dim), "self_k": (dim, dim), "self_v": (dim, dim), "self_o": (dim, dim),
              "cross_q": (dim, dim), "cross_k": (dim, C), "cross_v": (dim, C), "cross_o": (dim, dim),
              "mlp1": (hidden, dim), "mlp2": (dim, hidden)}
    block_list = []
    for _ in range(blocks):
        weights = {n: w4(*sh) for n, sh in shapes.items()}
        for br in ("self", "cross", "mlp"):
            weights[f"mod_{br}_w1"] = f16(256, dim)
            weights[f"mod_{br}_w2"] = f16(3 * dim, 256)
        norms = {n: (0.8 + 0.4 * torch.rand(128, device="cuda", generator=g)).half()
                 for n in ("self_q_norm", "self_k_norm", "cross_q_norm", "cross_k_norm")}
        block_list.append((weights, norms))
    pw = {"x_embed": w4(dim, 68), "t_embed1": w4(dim, dim), "t_embed2": w4(3 * dim, dim),
          "t_norm": (0.8 + 0.4 * torch.rand(dim, device="cuda", generator=g)).half()}
    fw = {"mod_w1": w4(256, dim), "mod_w2": w4(2 * dim, 256), "proj": w4(64, dim)}
    latent = torch.randn(16, side, side, device="cuda", generator=g)
    ctxt = torch.randn(T, C, device="cuda", generator=g).half()
    rope = torch.from_numpy(A.DitRoPE.generate(1, SIDE, SIDE)).cuda()
    residual = torch.empty(S, dim, device="cuda")
    emb = torch.empty(dim, device="cuda")
    adaln = torch.empty(3 * dim, device="cuda")
    vel = torch.empty(16, side, side, device="cuda")
    den, nxt = torch.empty_like(vel), torch.empty_like(vel)
    prep, fin, blk = A.DiTPreparationExecutor(ctx), A.DiTFinalLayerExecutor(ctx), A.DiTBlockExecutor(ctx)
    ops, eu = A.LatentOps(ctx), A.EulerSampler(ctx)
    cache = A.CrossKVCache(ctx, blocks)
    sig = A.EulerSampler.SIGMAS
    n = vel.numel()

    def step(i):
        s, ns = sig[i % 8], sig[i % 8 + 1]
        prep.execute(pw, latent, s, residual, emb, adaln, height=side, width=side)
        blk.forward(block_list, residual, emb, adaln, ctxt, rope, tokens=S, cache=cache)
        fin.execute(fw, residual, emb, adaln, vel, height=side, width=side)
        ops.flow_velocity_to_denoised(latent, vel, den, s, n)
        eu.encode_step(latent, den, nxt, s, ns, n)

    def forward_only(i):
        blk.forward(block_list, residual, emb, adaln, ctxt, rope, tokens=S, cache=cache)

    # the first step projects every block's context K/V into the cache
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    step(0)
    e1.record(stream)
    torch.cuda.synchronize()
    first_ms = e0.elapsed_time(e1)
    finite = bool(torch.isfinite(vel).all())
    ms = time_region(torch, stream, step, args.block_steps, 1)
    fwd = time_region(torch, stream, forward_only, args.block_steps, 1)
    streamed = time_streamed_forward(torch, A, ctx, stream, args, blk, block_list,
                                     (residual, emb, adaln, ctxt, rope), cache, fwd)
    return ms, first_ms, fwd, finite, streamed


def time_streamed_forward(torch, A, ctx, stream, args, blk, block_list, bufs, cache, resident_ms):
    """The same 28-block forward with every block's weights streamed from pinned host memory
    through a WeightStreamer of 2 device slots (WeightStreamer.swift:94-213, DitForward.swift:
    21-35): block i runs from one slot while the copy stream fills the other with block i+1.
    Each block's tensors sit 256-byte aligned in one host range, and the block template holds
    their offsets.  Returns ms per forward, bytes per block and the host-to-device rate the
    forward implies."""
    residual, emb, adaln, ctxt, rope = bufs
    names, norm_names = A.DiTBlockExecutor.NAMES, A.DiTBlockExecutor.NORMS
    templates, ranges, hosts = [], [], []
    for weights, norms in block_list:
        tensors = {}
        for n in names:
            for t in (weights[n].packed, weights[n].scale, weights[n].zero):
                tensors[t.data_ptr()] = t
        for n in norm_names:
            tensors[norms[n].data_ptr()] = norms[n]
        offs, off = {}, 0
        for ptr, t in tensors.items():
            off = (off + 255) // 256 * 256
            offs[ptr] = off
            off += t.numel() * t.element_size()
        host = torch.empty(off, dtype=torch.uint8, pin_memory=True)
        for ptr, t in tensors.items():
            nb = t.numel() * t.element_size()
            host[offs[ptr]:offs[ptr] + nb].copy_(t.reshape(-1).view(torch.uint8))
        tmpl = blk.weights_struct(weights, norms)
        for n in names:
            q = getattr(tmpl, n)
            for b in (q.packed, q.scale, q.zero):
                b.ptr = offs[b.ptr]
                b.length = 0
        for n in norm_names:
            b = getattr(tmpl, n)
            b.ptr = offs[b.ptr]
            b.length = 0
        templates.append(tmpl)
        ranges.append((host.data_ptr(), host.numel()))
        hosts.append(host)
    torch.cuda.synchronize()
    per_block = max(r[1] for r in ranges)
    st = A.WeightStreamer(ctx, capacity=per_block, slots=2)

    def fwd_streamed(i):
        blk.forward_streamed(st, templates, ranges, residual, emb, adaln, ctxt, rope, tokens=S, cache=cache)

    ms = time_region(torch, stream, fwd_streamed, args.block_steps, 1)
    total = sum(r[1] for r in ranges)
    st.close()
    del hosts
    return {"ms": round(ms, 3), "resident_ms": round(resident_ms, 3), "slots": 2,
            "bytes_per_block": int(per_block), "host_to_device_gbs": round(total / (ms * 1e-3) / 1e9, 1),
            "includes": "28 W4 blocks, weights copied from pinned host ranges into 2 device slots on the "
                        "streamer's copy stream, overlapped with the previous block's kernels"}


def time_qwen_layer(torch, A, ctx, stream, args):
    """ms per Qwen encoder layer (workload 4 shape: B=4 right-padded sequences of 512
    tokens, hidden 1024, 16/8 heads, MLP 3072, all seven linears W8 symmetric, group 64)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(1004)
    B, S, hidden, H, Hkv, D, inter = 4, 512, 1024, 16, 8, 128, 3072
    keep = []

    def w8(n, k):
        p = torch.randint(0, 256, (n, k), device="cuda", generator=g, dtype=torch.uint8)
        sc = (1e-4 + 2e-4 * torch.rand(n, k // 64, device="cuda", generator=g)).half()
        z = (-128 * sc.float()).half()
        keep.extend([p, sc, z])
        return A.QuantizedLinearWeightBuffers(1, p, sc, z, n, k, k)

    shapes = {"q": (H * D, hidden), "k": (Hkv * D, hidden), "v": (Hkv * D, hidden), "o": (hidden, H * D),
              "gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    weights = {n: w8(*s) for n, s in shapes.items()}
    norms = {"input_norm": (0.8 + 0.4 * torch.rand(hidden, device="cuda", generator=g)).half(),
             "post_attention_norm": (0.8 + 0.4 * torch.rand(hidden, device="cuda", generator=g)).half(),
             "q_norm": (0.8 + 0.4 * torch.rand(D, device="cuda", generator=g)).half(),
             "k_norm": (0.8 + 0.4 * torch.rand(D, device="cuda", generator=g)).half()}
    residual = torch.randn(B, S, hidden, device="cuda", generator=g)
    rope = torch.from_numpy(A.qwen_rope(S)).cuda()
    lengths = [115, 165, 240, 509]
    layer = A.QwenLayerExecutor(ctx)

    def step(i):
        layer.encode(weights, norms, residual, rope, batch=B, tokens=S, key_lengths=lengths)

    ms = time_region(torch, stream, step, args.block_steps, 2)
    rows = B * S
    lin = 2 * rows * sum(n * k for n, k in shapes.values())
    att = sum(2 * D * L * (L + 1) for L in lengths) * H
    return {"ms": round(ms, 5), "tflops": round((lin + att) / ms / 1e9, 2), "gflop": round((lin + att) / 1e9, 2),
            "mfma_frac": round((lin + att) / ms / 1e9 / FP16_PEAK_TFLOPS, 4), "key_lengths": lengths}


def _host_info():
    import subprocess
    import numpy
    import torch
    model = "?"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), "?")
    except (OSError, subprocess.SubprocessError):
        pass
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "torch": torch.__version__, "numpy": numpy.__version__}


def _median_of(fn, runs=5):
    """Median wall time (s) of ``runs`` calls after one untimed warm-up, and the spread."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], times[0], times[-1]


def _at_threads(torch, n, fn, runs=5):
    old = torch.get_num_threads()
    torch.set_num_threads(n)
    try:
        return _median_of(fn, runs)
    finally:
        torch.set_num_threads(old)


def _oracle_cases():
    """The five workloads as oracle calls, inputs built once outside the timed runs:
    C1 S=1024 self-attention, C2 S=4096 self-attention with q/k RMSNorm + DiT RoPE,
    C3 B4 cross attention 4096x512 with key lengths, C4 Qwen causal GQA B4 S512 with
    NeoX RoPE and padding, C5 one DiT block at S=4096 (W4 weights dequantised once)."""
    from oracle import attention as oatt
    from oracle import blocks as oblk
    from oracle import inputs as oin
    cases = {}
    d1 = oin.self_attention(1)
    cases["c1_self_attention_s1024"] = (lambda: oatt.sdpa(d1["q"], d1["k"], d1["v"]), attn_flops(1024, 1024))
    d2 = oin.self_attention(2)

    def c2():
        qq = oatt.qk_prologue(d2["q"], d2["q_norm_w"], d2["eps"], d2["rope"])
        kk = oatt.qk_prologue(d2["k"], d2["k_norm_w"], d2["eps"], d2["rope"])
        return oatt.sdpa(qq, kk, d2["v"])
    cases["c2_self_attention_s4096_norm_rope"] = (c2, attn_flops(S, S))
    d3 = oin.cross_attention()
    L3 = d3["key_lengths"].tolist()

    def c3():
        qq = oatt.qk_prologue(d3["q"], d3["q_norm_w"], d3["eps"], None)
        kk = oatt.qk_prologue(d3["k"], d3["k_norm_w"], d3["eps"], None)
        return oatt.sdpa(qq, kk, d3["v"], key_lengths=L3)
    cases["c3_cross_attention_b4_masked"] = (c3, sum(4.0 * H * 4096 * l * D for l in L3))
    d4 = oin.qwen_attention()
    L4 = d4["key_lengths"].tolist()

    def c4():
        qq = oatt.qk_prologue(d4["q"], d4["q_norm_w"], d4["eps"], d4["rope"])
        kk = oatt.qk_prologue(d4["k"], d4["k_norm_w"], d4["eps"], d4["rope"])
        return oatt.sdpa(qq, kk, d4["v"], causal=True, key_lengths=L4)
    cases["c4_qwen_causal_gqa_b4_s512"] = (c4, 4.0 * D * 16 * sum(sum(min(i + 1, l) for i in range(512)) for l in L4))
    d5 = oin.dit_block(S=4096)
    w5 = oblk.dequant_weights(d5)
    cases["c5_dit_block_s4096"] = (lambda: oblk.dit_block(d5, boundary="fp16", weights=w5), oblk.block_flops())
    return cases


def cpu_baseline():
    """The torch-CPU fp32 oracle on the headline workload (all 16 heads, S=4096,
    norm+RoPE): median of 5 timed runs after one warm-up, on all of this host's torch
    threads and again on 4 threads (the thread count the reference's own source oracle
    pins)."""
    import torch
    cases = _oracle_cases()
    fn, fl = cases["c2_self_attention_s4096_norm_rope"]
    threads = torch.get_num_threads()
    med, lo, hi = _at_threads(torch, threads, fn)
    med4, lo4, hi4 = _at_threads(torch, 4, fn)
    info = _host_info()
    print(f"# cpu oracle C2: {med:.3f} s/call on {threads} threads, {med4:.3f} s/call on 4 threads ({info})",
          file=sys.stderr, flush=True)
    out = {"value": round(fl / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "sample": "full workload: S=4096 H=16 D=128 self-attention with q/k RMSNorm + DiT RoPE, fp32 torch "
                     "oracle, median of 5 runs after 1 warm-up",
           "ms_per_call": round(med * 1e3, 2), "ms_min_max": [round(lo * 1e3, 2), round(hi * 1e3, 2)],
           "threads_4": {"value": round(fl / med4 / 1e12, 5), "ms_per_call": round(med4 * 1e3, 2),
                         "ms_min_max": [round(lo4 * 1e3, 2), round(hi4 * 1e3, 2)]}}
    out.update(info)
    return out


def cpu_table():
    """ms per call of the oracle on C1-C5 (C5 = ms per DiT block) at all threads and at
    4 threads, median of 5 after 1 warm-up each."""
    import torch
    threads = torch.get_num_threads()
    rows = {}
    for name, (fn, fl) in _oracle_cases().items():
        row = {}
        for n in (threads, 4):
            med, lo, hi = _at_threads(torch, n, fn)
            row[f"threads_{n}"] = {"ms": round(med * 1e3, 2), "ms_min_max": [round(lo * 1e3, 2), round(hi * 1e3, 2)],
                                   "tflops": round(fl / med / 1e12, 5)}
        rows[name] = row
        print(f"# cpu oracle {name}: {row}", file=sys.stderr, flush=True)
    return rows


if __name__ == "__main__":
    main()
