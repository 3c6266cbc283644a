#!/usr/bin/env python3
"""Paged-KV decode benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the configuration the north-star HBM target is
quoted on): 64 sequences with contexts U[512, 8192] (seed 2), 12 heads x 64,
block size 16, bf16 K/V, each block table a random shuffle over a shared
40000-block pool.  One step is one decode step of the paged path for one
layer over the whole batch: the batched append of each sequence's new token
(into its last slot) and the batched direct paged decode attention over the
full contexts - one mie_paged_decode_append launch (`--unfused`: the append
launch, then the decode launch).  Inputs are resident in HBM before timing.

Printed: ONE JSON line.  `value` is algorithmic bytes (attention + append) per
step over the measured step time, in GB/s.  `roofline` is the dominant
launch: its algorithmic bytes (attention + append fused; attention alone with
`--unfused`) over its average duration from HIP events recorded on the launch
stream: one event pair around the timed loop of back-to-back fused launches
(region / steps), or events around every attention call with `--unfused`.
`cpu_baseline` times the oracle's gather + scaled_dot_product_attention path
(the reference's CPU path) on a bounded sample of the same workload.
`secondary` carries the per-token end-to-end decode latency (config 1, and
its shape in bfloat16) and the single-layer, append/gather and long-context
figures (configs 2, 3, 5).
"""

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "moe-inference-engine_amd"))

METRIC = "paged-decode attention HBM GB/s (% of peak) + per-token decode latency ms"
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
SECONDARY_NAMES = ("launch_floor", "round_latency", "north_star_64x8192", "config2_single_layer", "config3_append_gather",
                   "config5_long_context", "fused_moe_decode", "config1_e2e_decode", "config1_context_sweep",
                   "config1_attention_micro", "config1_bf16_decode")
TRAFFIC_FILE = ROOT / "profiles" / "paged_decode_config4_traffic.json"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--partition-tokens", type=int, default=0, help="0 = the library's automatic choice")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--secondary", default="",
                   help="comma-separated secondary figures to run (default: all): " + ", ".join(SECONDARY_NAMES))
    p.add_argument("--unfused", action="store_true",
                   help="run the step's append and decode as two launches instead of mie_paged_decode_append")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline time budget")
    p.add_argument(
        "--copy-calibration-mib",
        type=int,
        default=0,
        help="first run 10 plain device copies of this many MiB (reads and writes that many bytes "
        "each), to scale hardware byte counters against a kernel of known traffic",
    )
    args = p.parse_args()
    unknown = sorted({n for n in args.secondary.split(",") if n} - set(SECONDARY_NAMES))
    if unknown:
        p.error(f"unknown secondary {', '.join(unknown)} (known: {', '.join(SECONDARY_NAMES)})")
    return args


def copy_calibration(torch, mib):
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 10 copies of {n * 4} bytes")
    del src, dst
    torch.cuda.empty_cache()


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


# ---- the measured step -----------------------------------------------------------


def run_config4(torch, args):
    from moe_engine import _native, workloads

    # The step object is the one tests/test_gpu_decode.py checks against the
    # oracle: the same workload, new rows and calls.
    step = workloads.config4_step(out_dtype=torch.bfloat16, partition_tokens=args.partition_tokens)
    w = step.w
    heads, dim = 12, 64
    attn_bytes = workloads.attention_bytes(w.lens, heads, dim, 16, 2)
    app_bytes = workloads.append_bytes(len(w.lens), heads, dim, 2)
    part, ws_bytes = _native.decode_plan(
        len(w.lens), heads, dim, 16, w.max_len, torch.bfloat16, args.partition_tokens
    )

    # Timed region: the whole step.  Fused, the step is one launch, so one
    # pair of HIP events around the timed loop gives its average duration
    # (region / steps: inter-launch gaps included, no per-call event packets,
    # which cost ~1-2 us of stream time each).  Unfused, events bracket every
    # attention call to separate it from the append launch.
    before, timed = (step.append, step.attend) if args.unfused else (None, step.fused)
    timed_bytes = attn_bytes if args.unfused else attn_bytes + app_bytes
    for _ in range(args.warmup):
        if before:
            before()
        timed()
    torch.cuda.synchronize()
    per_call = args.unfused
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps if per_call else 1)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps if per_call else 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if not per_call:
        starts[0].record()
    for i in range(args.steps):
        if before:
            before()
        if per_call:
            starts[i].record()
        timed()
        if per_call:
            ends[i].record()
    if not per_call:
        ends[0].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    if per_call:
        attn_ms = [s_.elapsed_time(e_) for s_, e_ in zip(starts, ends)]
    else:
        attn_ms = [starts[0].elapsed_time(ends[0]) / args.steps]
    attn_avg_s = sum(attn_ms) / len(attn_ms) / 1e3
    achieved = timed_bytes / attn_avg_s / 1e9
    median_ms = statistics.median(attn_ms) if per_call else None
    if not per_call:
        # After the timed region: 50 further launches, each between its own
        # pair of events, for the per-launch median (the event packets add a
        # little to each).
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(50)]
        for s_, e_ in pairs:
            s_.record()
            timed()
            e_.record()
        torch.cuda.synchronize()
        median_ms = statistics.median(s_.elapsed_time(e_) for s_, e_ in pairs)
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
    return {
        "workload": w,
        "value": (attn_bytes + app_bytes) * args.steps / elapsed / 1e9,
        "ms_per_step": elapsed / args.steps * 1e3,
        "attn_bytes": attn_bytes,
        "append_bytes": app_bytes,
        "partition_tokens": part,
        "workspace_bytes": ws_bytes,
        "roofline": {
            "bound": "hbm",
            "kernel": ("mie_paged_decode (" if args.unfused else "mie_paged_decode_append (")
            + ("paged_decode_wg_kernel, one workgroup per (sequence, head)" if ws_bytes == 0
               else "paged_decode_flat_kernel + paged_decode_reduce_kernel")
            + ("" if args.unfused or ws_bytes else ", the step's append fused in")
            + ")",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": timed_bytes,
            "avg_duration_us": round(attn_avg_s * 1e6, 2),
            "median_duration_us": round(median_ms * 1e3, 2),
            "duration_source": "HIP events around every attention call" if per_call
            else "average: one HIP event pair around the timed loop of back-to-back launches (region / steps); "
            "median: 50 further launches, each between its own event pair",
        },
    }


# ---- CPU baseline (the oracle's gather + SDPA path, on the host cores) -------------


def cpu_model_name() -> str:
    """The host CPU's model name from /proc/cpuinfo ("unknown" elsewhere)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, w, budget_s):
    from oracle import paged_ref as ref
    from moe_engine import workloads

    threads = torch.get_num_threads()
    k_pool, v_pool = w.k_pool[w.layer : w.layer + 1].cpu(), w.v_pool[w.layer : w.layer + 1].cpu()
    q = w.q.cpu()
    sample = list(range(0, len(w.lens), 8))  # every 8th sequence: 8 of 64
    lens = [w.lens[b] for b in sample]
    tables = [w.tables[b] for b in sample]
    sample_bytes = workloads.attention_bytes(lens, q.shape[1], q.shape[2], w.block_size, 2)
    ref.batched_gather_sdpa(q[sample], k_pool, v_pool, 0, tables, lens)  # warm-up
    passes, t0 = 0, time.perf_counter()
    while True:
        ref.batched_gather_sdpa(q[sample], k_pool, v_pool, 0, tables, lens)
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s or passes >= 100000:
            break
    return {
        "value": round(sample_bytes * passes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"sequences {sample} of config 4 ({sum(lens)} tokens, bf16), {passes} passes of "
            f"per-sequence gather + torch scaled_dot_product_attention in {elapsed:.1f} s; "
            f"host {os.cpu_count()} logical CPUs ({cpu_model_name()}), torch threads {threads}"
        ),
        "ms_per_pass": round(elapsed / passes * 1e3, 2),
    }


# ---- secondary figures -------------------------------------------------------------


def timed_us(torch, fn, iters=50, warmup=5):
    for _ in range(warmup):
        fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters * 1e3


# Bytes one replay must read to be "cold": more than MI355X's 256 MB last-level
# (Infinity) cache.
COLD_BYTES = 320 * 10**6


def graph_replay_us(torch, calls, reps=5):
    """Device time per call of `calls` (a list of callables) captured back to
    back in one HIP graph: no host launch overhead between calls."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in calls:
            fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for fn in calls:
            fn()
    times = []
    for _ in range(reps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        stop.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) * 1e3 / len(calls))
    return sorted(times)[len(times) // 2]


def secondary_config2(torch):
    """Single layer, batch 1, context 2048, bf16.  Device time per call from
    graph replays of 64 calls: warm (the same blocks every call) and cold (64
    disjoint sequences in turn, 403 MB > the 256 MB MALL); plus the host-launched
    time per call through the Python wrapper."""
    from moe_engine import paged_attention, workloads

    w = workloads.make_workload([2048] * 64, block_size=16, num_blocks=64 * 128, dtype=torch.bfloat16, seed=1)
    nbytes = workloads.attention_bytes([2048], 12, 64, 16, 2)
    k0, v0 = w.k_pool[0], w.v_pool[0]
    tables = [w.block_tables[b : b + 1] for b in range(64)]  # [1, 128] rows
    qs = [w.q[b : b + 1] for b in range(64)]

    def call(b):
        return lambda: paged_attention.decode_layer(qs[b], k0, v0, tables[b], context_len=2048)

    warm = graph_replay_us(torch, [call(0)] * 64)
    cold = graph_replay_us(torch, [call(b) for b in range(64)])
    launched = timed_us(torch, call(0))
    return {
        "warm_us": round(warm, 2),
        "warm_gbs": round(nbytes / warm / 1e3, 1),
        "cold_us": round(cold, 2),
        "cold_gbs": round(nbytes / cold / 1e3, 1),
        "host_launched_us": round(launched, 2),
        "bytes": nbytes,
        "note": "warm/cold: device time per call, 64 calls replayed from one HIP graph; "
        "host_launched: back-to-back calls through the Python wrapper",
    }


def secondary_config3(torch):
    """12 layers, bf16, 12 x 64, block 16, random tables
    over a 65536-block pool, contexts 128, 1024 and 8192.  Per context: the
    per-layer append of one token and the per-layer gather of the whole
    context, as device time per layer (the 12 layers' calls replayed from one
    HIP graph) and host-launched time per layer through the validating
    wrapper; at 8192 also the prefill scatter of the whole context."""
    from moe_engine import kv_ops, workloads

    L, NB, H, BS, D = 12, 65536, 12, 16, 64
    k_pool = torch.zeros(L, NB, H, BS, D, dtype=torch.bfloat16, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    new = torch.randn(1, H, 1, D, device="cuda").to(torch.bfloat16)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3)).to(torch.int32).cuda()
    res = {}
    for C in (128, 1024, 8192):
        nblk = -(-C // BS)
        table = torch.zeros(NB, dtype=torch.int32, device="cuda")
        table[:nblk] = perm[:nblk]
        outk = torch.empty(1, H, C, D, dtype=torch.bfloat16, device="cuda")
        outv = torch.empty_like(outk)
        appends = [lambda l=l: kv_ops.append(k_pool, v_pool, l, new, new, table, position=C - 1) for l in range(L)]
        gathers = [lambda l=l: kv_ops.gather(k_pool, v_pool, l, table, C, outk, outv) for l in range(L)]
        append_dev = graph_replay_us(torch, appends)
        gather_dev = graph_replay_us(torch, gathers)
        append_host = timed_us(torch, lambda: [f() for f in appends]) / L
        gb = workloads.gather_bytes(C, H, D, 2)
        ab = workloads.append_bytes(1, H, D, 2)
        # Cold: S sequences with disjoint blocks, each gathered through all
        # layers, so one replay reads more than the 256 MB last-level cache.
        S = max(2, min(NB // nblk, -(-COLD_BYTES // (L * gb // 2))))
        tables = []
        for i in range(S):
            t = torch.zeros(NB, dtype=torch.int32, device="cuda")
            t[:nblk] = perm[i * nblk:(i + 1) * nblk]
            tables.append(t)
        cold = [lambda l=l, t=t: kv_ops.gather(k_pool, v_pool, l, t, C, outk, outv) for t in tables for l in range(L)]
        gather_cold = graph_replay_us(torch, cold)
        # Copy ceiling: the same bytes moved by the runtime's device-to-device
        # copy (read gb / 2, write gb / 2) from 12 distinct sources into one
        # destination, as the 12 layers' gathers read 12 pool slices into one
        # output, replayed from one graph.
        srcs = torch.empty(L, gb // 4, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty(gb // 4, dtype=torch.bfloat16, device="cuda")
        copy_dev = graph_replay_us(torch, [lambda l=l: dst.copy_(srcs[l]) for l in range(L)])
        del srcs, dst
        res[f"c{C}"] = {
            "append_device_us_per_layer": round(append_dev, 2),
            "append_host_launched_us_per_layer": round(append_host, 2),
            "append_bytes_per_layer": ab,
            "gather_device_us_per_layer": round(gather_dev, 2),
            "gather_gbs": round(gb / gather_dev / 1e3, 1),
            "gather_cold_device_us_per_layer": round(gather_cold, 2),
            "gather_cold_gbs": round(gb / gather_cold / 1e3, 1),
            "copy_device_us_per_layer": round(copy_dev, 2),
            "copy_gbs": round(gb / copy_dev / 1e3, 1),
            "gather_bytes_per_layer": gb,
        }
        del tables
    # Prefill scatter: the whole context written through the table in one launch per layer.
    C = 8192
    table = torch.zeros(NB, dtype=torch.int32, device="cuda")
    table[: C // BS] = perm[: C // BS]
    prefill = torch.randn(1, H, C, D, device="cuda").to(torch.bfloat16)
    prefill_dev = graph_replay_us(
        torch, [lambda l=l: kv_ops.append(k_pool, v_pool, l, prefill, prefill, table, position=0) for l in range(L)]
    )
    pb = workloads.append_bytes(C, H, D, 2)  # C tokens, K and V read and written
    res["prefill_scatter_c8192"] = {"device_us_per_layer": round(prefill_dev, 2), "gbs": round(pb / prefill_dev / 1e3, 1)}
    res["note"] = ("device: the 12 layers' calls replayed from one HIP graph, time per layer; "
                   "gather_cold: the same for several sequences with disjoint blocks in one graph, more than "
                   "256 MB read per replay; host_launched: back-to-back calls through the Python wrapper")
    del k_pool, v_pool
    torch.cuda.empty_cache()
    return res


def secondary_moe(torch):
    """Fused MoE decode at config 1's shape: d 768, FFN 2048, top-2
    of 8, float32.  Bytes per call: the router and the two selected experts'
    W1, b1, W2, b2, read once."""
    from moe_engine.model import MoEFeedForward

    torch.manual_seed(0)
    layer = MoEFeedForward(768, 2048, 8, 2).to("cuda").eval()
    layer.set_mode("direct")
    x = torch.randn(1, 1, 768, device="cuda")
    nbytes = 4 * (8 * 768 + 2 * (2048 * 768 + 2048 + 768 * 2048 + 768))
    with torch.no_grad():
        device_us = graph_replay_us(torch, [lambda: layer(x, decode=True)] * 32)
        us = timed_us(torch, lambda: layer(x, decode=True), iters=200, warmup=20)
        layer.set_mode("reference")
        ref_us = timed_us(torch, lambda: layer(x, decode=True), iters=50, warmup=5)
    return {
        "fused_device_us_per_call": round(device_us, 2),
        "fused_device_gbs": round(nbytes / device_us / 1e3, 1),
        "fused_host_launched_us_per_call": round(us, 2),
        "pytorch_path_us_per_call": round(ref_us, 2),
        "bytes_per_call": nbytes,
        "note": "device: 32 calls (three launches each) replayed from one HIP graph; host_launched: back-to-back "
        "calls through the Python module; the PyTorch path synchronizes per expert and cannot be captured",
    }


def secondary_config5(torch):
    """BASELINE config 5, the long-context split decode: batch 1 and 8,
    contexts 32768 and 131072, block 16 and 32, bf16 and fp32, 1 % of keys
    x20.  Device time per call from 10 graph-replayed calls, GB/s of the
    algorithmic bytes; cells under COLD_BYTES also from calls cycling over
    copies of the workload in separate pools (cold_us, cold_gbs), so that one
    replay reads more than the last-level cache holds."""
    from moe_engine import paged_attention, workloads

    res = {}
    for dtype, tag in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
        for batch in (1, 8):
            for ctx in (32768, 131072):
                for bs in (16, 32):
                    w = workloads.make_workload([ctx] * batch, block_size=bs, dtype=dtype, seed=5, heavy_fraction=0.01)
                    nbytes = workloads.attention_bytes(w.lens, 12, 64, bs, w.k_pool.element_size())
                    call = lambda w=w: paged_attention.decode_batched(
                        w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, w.max_len, context_lens_host=w.lens
                    )
                    us = graph_replay_us(torch, [call] * 10)
                    cell = {"us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1)}
                    if nbytes < COLD_BYTES:
                        # Cold: copies of the workload in separate pools, cycled so one replay reads more
                        # than the 256 MB last-level cache.
                        copies = [w] + [
                            workloads.make_workload([ctx] * batch, block_size=bs, dtype=dtype, seed=5 + i,
                                                    heavy_fraction=0.01)
                            for i in range(1, -(-COLD_BYTES // nbytes))
                        ]
                        calls = [lambda c=c: paged_attention.decode_batched(
                            c.q, c.k_pool, c.v_pool, 0, c.block_tables, c.context_lens, c.max_len,
                            context_lens_host=c.lens) for c in copies] * 3
                        cold = graph_replay_us(torch, calls)
                        cell.update(cold_us=round(cold, 2), cold_gbs=round(nbytes / cold / 1e3, 1))
                        del copies, calls
                    res[f"{tag}_b{batch}_c{ctx}_bs{bs}"] = cell
                    del w, call
                    torch.cuda.empty_cache()
    return res


def secondary_north_star(torch, launches=100):
    """The north star's literal target shape: 64 sequences x 8192 tokens,
    12 x 64, block 16, bf16 (workloads.north_star_step, the object
    tests/test_gpu_decode.py checks): the same one-launch decode step as the
    headline, timed the same way (one HIP event pair around `launches`
    back-to-back launches), as GB/s of its algorithmic bytes and a fraction
    of HBM peak."""
    from moe_engine import workloads

    step = workloads.north_star_step()
    w = step.w
    nbytes = workloads.attention_bytes(w.lens, 12, 64, 16, 2) + workloads.append_bytes(len(w.lens), 12, 64, 2)
    for _ in range(10):
        step.fused()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(launches):
        step.fused()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / launches * 1e3
    del step, w
    return {"us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1), "hbm_fraction": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
            "bytes": nbytes, "launches": launches,
            "note": "64 x 8192 uniform, bf16, shuffled tables over a 40000-block pool; mie_paged_decode_append "
            "(append fused), average of back-to-back launches between one HIP event pair"}


def secondary_launch_floor(torch):
    """The floor a launch-bound call cannot go under on this box: device time
    per call of 64 calls replayed from one HIP graph, each call one or two
    launches of an empty kernel (256 workgroups) - the same way the config 2,
    3 and 5 figures are timed."""
    from moe_engine import _native

    lib = _native.lib()

    def noop():
        if lib.mie_empty_launch(256, torch.cuda.current_stream().cuda_stream):
            raise RuntimeError("mie_empty_launch failed")

    one = graph_replay_us(torch, [noop] * 64)
    two = graph_replay_us(torch, [lambda: (noop(), noop())] * 64)
    return {"one_launch_us": round(one, 3), "two_launch_us": round(two, 3),
            "note": "empty kernel, 256 workgroups x 256 threads; 64 calls per graph, device time per call"}


def secondary_round_latency(torch, calls=64, reps=7):
    """Dependent memory rounds on this box, measured with product kernels
    replayed from HIP graphs of `calls` launches each: the empty kernel
    (mie_empty_launch, one workgroup) and mie_embed of one token, which makes
    two dependent rounds (the token id, then its table row) around a trivial
    sum and store.  Each call reads its own id and row; `cold` replays follow
    a 1 GiB fill that evicts the L2s and the last-level cache, `warm` replays
    repeat without it.  embed - empty is what two rounds add to a launch in a
    graph; a kernel trace of the same command gives their durations."""
    from moe_engine import _native

    lib = _native.lib()
    dev = "cuda"
    vocab, dim = 8192, 768
    gen = torch.Generator().manual_seed(0)
    tok = torch.randn(vocab, dim, generator=gen).to(dev)
    pos = torch.randn(16, dim, generator=gen).to(dev)
    ids = torch.zeros(calls, 64, dtype=torch.int64)
    ids[:, 0] = torch.randperm(vocab, generator=gen)[:calls]
    ids = ids.to(dev)  # one id per 512-byte line
    out = torch.empty(calls, dim, device=dev)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)

    def run(rc, what):
        if rc:
            raise RuntimeError(f"{what} failed: {lib.mie_last_error()}")

    kinds = {
        "empty": lambda i, st: run(lib.mie_empty_launch(1, st), "mie_empty_launch"),
        "embed": lambda i, st: run(lib.mie_embed(ids[i].data_ptr(), None, i % 16, 1, tok.data_ptr(), vocab,
                                                 pos.data_ptr(), 16, dim, out[i].data_ptr(), 0, st), "mie_embed"),
    }
    res = {}
    for name, fn in kinds.items():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(calls):
                fn(i, side.cuda_stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for i in range(calls):
                fn(i, side.cuda_stream)
        for mode in ("cold", "warm"):
            times = []
            for r in range(reps):
                if mode == "cold":
                    flush.fill_(r & 0xFF)
                start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                graph.replay()
                stop.record()
                torch.cuda.synchronize()
                times.append(start.elapsed_time(stop) * 1e3 / calls)
            res[f"{name}_{mode}_us"] = round(statistics.median(times), 3)
        del graph
    for mode in ("cold", "warm"):
        res[f"two_rounds_{mode}_us"] = round(res[f"embed_{mode}_us"] - res[f"empty_{mode}_us"], 3)
    res["note"] = ("device time per call, 64 calls per graph (median of 7 replays); each call reads its own id and "
                   "row; cold replays follow a 1 GiB fill")
    del flush, tok
    return res


def add_floor_fractions(secondary):
    """Latency-bound figures as fractions of the launch floor (floor / time:
    1.0 would be a call that costs no more than its empty launches) next to
    their fractions of HBM peak."""
    floor = secondary.get("launch_floor")
    if not floor or "error" in floor:
        return
    one, two = floor["one_launch_us"], floor["two_launch_us"]
    c2 = secondary.get("config2_single_layer")
    if c2 and "warm_us" in c2:
        c2["launch_floor_us"] = two
        c2["floor_over_time"] = round(two / c2["warm_us"], 3)
        c2["hbm_fraction"] = round(c2["warm_gbs"] / PEAK_HBM_GBS, 3)
    c3 = secondary.get("config3_append_gather")
    if c3:
        for key, cell in c3.items():
            if isinstance(cell, dict) and "gather_device_us_per_layer" in cell:
                cell["launch_floor_us"] = one
                cell["gather_floor_over_time"] = round(one / cell["gather_device_us_per_layer"], 3)
                cell["gather_hbm_fraction"] = round(cell["gather_gbs"] / PEAK_HBM_GBS, 3)
    c5 = secondary.get("config5_long_context")
    if c5:
        for key, cell in c5.items():
            if isinstance(cell, dict) and "_b1_c32768_" in key:
                cell["launch_floor_us"] = two  # partitions + the merge launch
                cell["floor_over_time"] = round(two / cell["us"], 3)
                cell["hbm_fraction"] = round(cell["gbs"] / PEAK_HBM_GBS, 3)


def secondary_context_sweep(torch, rounds=21):
    """BASELINE config 1's model: decode step latency at contexts 16, 64, 256
    and 1024 (benchmarks/context_sweep.py:50-126) for contiguous,
    paged-gather, paged-direct, contiguous-direct and the two graph systems,
    `rounds` interleaved rounds, each system on a fresh cache behind a
    random pad in every round (moe_engine.harness.context_sweep), with
    paired paging-cost intervals per context."""
    from moe_engine import harness

    model = harness.make_model(harness.CONFIG1, seed=0, device="cuda")
    return harness.context_sweep(model, contexts=(16, 64, 256, 1024), rounds=rounds)


def secondary_attention_micro(torch, rounds=21):
    """One layer's decode attention at config 1's shape (12 x 64, fp32,
    block 16; benchmarks/attention_micro.py:27-85): us per call for
    contiguous read + SDPA, paged gather + SDPA, the paged direct kernel and
    the same kernel on the contiguous layout, `rounds` rounds on freshly
    placed caches, with device time (graph replays) and paired paging costs
    for the direct kernel (moe_engine.harness.attention_micro)."""
    from moe_engine import harness

    return harness.attention_micro(harness.CONFIG1, contexts=(16, 64, 256, 1024), rounds=rounds)


def secondary_e2e(torch, rounds=21, new_tokens=64, cpu_rounds=2):
    """BASELINE config 1 (random init from seed 0, fp32, block 16, 32-token
    prompt, 64 greedy tokens).

    GPU: per-token greedy decode latency of the reference's systems
    (contiguous, paged-gather, paged-direct), the graph-replayed step
    (paged-direct-graph), and contiguous-direct(-graph): the contiguous
    layout run by the same fused kernels, so paged-direct minus it is the cost
    of paging alone - interleaved rounds with paired Student-t intervals
    (moe_engine.harness.ab_compare, benchmarks/ab_compare.py:75-144).

    CPU (the reference CPU path, on this host's cores): contiguous and
    paged-gather per-token decode latency, prefill excluded, median over the
    decode steps of `cpu_rounds` interleaved rounds (benchmarks/bench.py:
    217-231).

    Parity: the reference's report (scripts/check_parity.py:64-93) of the GPU
    paged-direct path against the CPU path, and the GPU tokens against the
    reference engine's own tokens for this configuration
    (tests/golden/reference_config1.json, written by the reference's code).

    MoE A/B: the contiguous system's decode with the PyTorch per-expert MoE
    against the fused kernels (moe_engine.harness.moe_ab_compare,
    benchmarks/moe_ab_compare.py:66-200), 3 rounds of 16 tokens."""
    from moe_engine import harness

    model = harness.make_model(harness.CONFIG1, seed=0, device="cuda")
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, harness.CONFIG1["vocab_size"], (32,), generator=gen).cuda()
    systems = harness.SYSTEMS + (harness.GRAPH_SYSTEM, harness.CONTIGUOUS_DIRECT, harness.CONTIGUOUS_DIRECT_GRAPH)
    report = harness.ab_compare(model, prompt, systems, rounds=rounds, new_tokens=new_tokens)

    log("config 1 on the CPU")
    cpu_model = harness.make_model(harness.CONFIG1, seed=0, device="cpu")
    start = time.perf_counter()
    cpu = harness.ab_compare(cpu_model, prompt.cpu(), ("contiguous", "paged-gather"), rounds=cpu_rounds,
                             new_tokens=new_tokens)
    cpu["wall_s"] = round(time.perf_counter() - start, 1)
    cpu["torch_threads"] = torch.get_num_threads()
    cpu["os_cpu_count"] = os.cpu_count()
    cpu["cpu_model"] = cpu_model_name()
    cpu["tokens_equal_gpu"] = cpu["tokens_identical"] and cpu.pop("tokens") == report.pop("tokens")
    report["cpu"] = cpu

    log("config 1 parity report")
    parity = harness.parity_report(model, cpu_model, prompt, new_tokens=new_tokens)
    fixture = ROOT / "tests" / "golden" / "reference_config1.json"
    if fixture.exists():
        golden = json.loads(fixture.read_text())
        if golden["prompt"] == prompt.tolist() and golden["new_tokens"] == new_tokens:
            parity["tokens_equal_reference_engine"] = parity["tokens"] == golden["tokens"]["paged_gather"]
    parity.pop("tokens")
    report["parity"] = parity

    log("config 1 MoE A/B")
    # The reference's MoE A/B (benchmarks/moe_ab_compare.py): contiguous cache,
    # PyTorch per-expert MoE against the fused kernels, interleaved rounds.
    moe_ab = harness.moe_ab_compare(model, prompt, rounds=3, new_tokens=16, system="contiguous")
    report["moe_ab"] = {
        "system": moe_ab["system"],
        "decode_median_ms": {mode: s["decode_median_ms"] for mode, s in moe_ab["summary"].items()},
        "paired_delta_direct_minus_reference_ms": moe_ab["paired_delta_direct_minus_reference"],
        "tokens_identical": moe_ab["tokens_identical"],
        "rounds": moe_ab["rounds"],
        "new_tokens": moe_ab["new_tokens"],
    }
    return report


def secondary_e2e_bf16(torch, rounds=3, new_tokens=32):
    """Config 1's model in bfloat16 (not a BASELINE config): per-token greedy
    decode of paged-direct, eagerly and replayed from a graph, interleaved
    rounds as in config1_e2e_decode, and the same cache system with the
    PyTorch MoE (moe_ab_compare), which the reference's bfloat16 models take
    because its fused MoE is float32 only."""
    from moe_engine import harness

    model = harness.make_model(harness.CONFIG1, seed=0, device="cuda", dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, harness.CONFIG1["vocab_size"], (32,), generator=gen).cuda()
    rep = harness.ab_compare(model, prompt, ("paged-direct", harness.GRAPH_SYSTEM), rounds=rounds,
                             new_tokens=new_tokens)
    ab = harness.moe_ab_compare(model, prompt, rounds=2, new_tokens=8, system="paged-direct")
    return {
        "decode_median_ms": {s: v["decode_median_ms"] for s, v in rep["summary"].items()},
        "pytorch_moe_decode_median_ms": ab["summary"]["reference"]["decode_median_ms"],
        "tokens_identical": rep["tokens_identical"] and ab["tokens_identical"],
        "note": "config 1's shape in bfloat16, random init seed 0; the reference's fused MoE is float32 only",
    }


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): "
            "the paged decode path shards by sequence, head or layer with no exchange, "
            "so multi-GPU figures are not produced by this build",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    from moe_engine import _native

    _native.lib()  # fail loudly when the HIP library is missing
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a ROCm GPU")
    torch.cuda.set_device(0)
    if args.copy_calibration_mib > 0:
        copy_calibration(torch, args.copy_calibration_mib)
    log("config 4: building workload")
    main_res = run_config4(torch, args)
    log(f"config 4: {main_res['value']:.1f} GB/s, attention {main_res['roofline']['achieved']} GB/s")
    w = main_res.pop("workload")
    total_tokens = sum(w.lens)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(torch, w, args.cpu_seconds)
    del w
    torch.cuda.empty_cache()

    secondary = {}
    if not args.no_secondary:
        chosen = [n for n in args.secondary.split(",") if n] or list(SECONDARY_NAMES)
        for name, fn in (
            ("launch_floor", secondary_launch_floor),
            ("round_latency", secondary_round_latency),
            ("north_star_64x8192", secondary_north_star),
            ("config2_single_layer", secondary_config2),
            ("config3_append_gather", secondary_config3),
            ("config5_long_context", secondary_config5),
            ("fused_moe_decode", secondary_moe),
            ("config1_e2e_decode", secondary_e2e),
            ("config1_context_sweep", secondary_context_sweep),
            ("config1_attention_micro", secondary_attention_micro),
            ("config1_bf16_decode", secondary_e2e_bf16),
        ):
            if name not in chosen:
                continue
            log(f"secondary {name}")
            try:
                secondary[name] = fn(torch)
            except Exception as exc:  # a secondary figure never hides the main line
                secondary[name] = {"error": f"{type(exc).__name__}: {exc}"}
            torch.cuda.empty_cache()
        add_floor_fractions(secondary)

    line = {
        "metric": METRIC,
        "value": round(main_res["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "batched paged decode step, BASELINE config 4: batched KV append + direct paged decode attention, one layer",
            "batch": 64,
            "context_lens": "U[512, 8192], seed 2",
            "total_tokens": total_tokens,
            "num_heads": 12,
            "head_dim": 64,
            "block_size": 16,
            "pool_blocks": 40000,
            "partition_tokens": main_res["partition_tokens"],
            "attention_bytes_per_step": main_res["attn_bytes"],
            "append_bytes_per_step": main_res["append_bytes"],
            "parallelism": "single GPU",
        },
        "roofline": main_res["roofline"],
        "cpu_baseline": cpu,
        "per_token_decode_ms": per_token_decode_ms(secondary.get("config1_e2e_decode"),
                                                   secondary.get("config1_context_sweep")),
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


def per_token_decode_ms(e2e, sweep=None):
    """The metric's second half: BASELINE config 1's median greedy decode
    latency per token for each system, from the config1_e2e_decode secondary
    (None when it did not run), with the paging-cost intervals of the e2e
    rounds and of the context sweep at every context."""
    if not e2e or "summary" not in e2e:
        return None
    out = {system: s["decode_median_ms"] for system, s in e2e["summary"].items()}
    out["tokens_identical"] = e2e.get("tokens_identical")
    paired = e2e.get("paired_deltas", {})
    for name in ("paged-direct_minus_contiguous-direct", "paged-direct-graph_minus_contiguous-direct-graph"):
        if name in paired:
            out[f"paging_cost_{name.split('_minus_')[0]}_ms"] = {
                "mean_delta_ms": paired[name]["mean_delta_ms"], "ci95_ms": paired[name]["ci95_ms"]}
    cpu = e2e.get("cpu")
    if cpu and "summary" in cpu:
        for system, s in cpu["summary"].items():
            out[f"cpu_{system}"] = s["decode_median_ms"]
        out["cpu_threads"] = cpu.get("torch_threads")
        out["cpu_model"] = cpu.get("cpu_model")
        out["cpu_tokens_identical_to_gpu"] = cpu.get("tokens_equal_gpu")
    parity = e2e.get("parity")
    if parity:
        out["parity"] = {k: parity[k] for k in ("engine_cache", "max_abs_logit_diff", "max_rel_logit_diff",
                                                "greedy_tokens_compared", "first_greedy_mismatch",
                                                "tokens_equal_reference_engine") if k in parity}
    if sweep and "paging_cost_ms" in sweep:
        out["context_sweep"] = {
            "median_step_ms": sweep["median_step_ms"],
            "paging_cost_ms": sweep["paging_cost_ms"],
            "rounds": sweep["rounds"],
            "placement_sampled": sweep["placement_sampled"],
        }
    out["rounds"] = e2e.get("rounds")
    out["placement_sampled"] = e2e.get("placement_sampled")
    out["workload"] = ("BASELINE config 1: 12 layers, d 768, 12 x 64 heads, top-2 of 8, FFN 2048, vocab 50257, "
                       "fp32, random init seed 0, 32-token prompt, 64 greedy tokens, block 16")
    return out


if __name__ == "__main__":
    main()
