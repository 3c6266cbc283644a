"""Latency harnesses for the paged decode path (random-init miniMoE models).

Counterparts of the reference's benchmarks, with random-init weights because
the real checkpoint and tokenizer are not available here:

  attention_micro  one layer's decode attention, us per call, for contiguous
                   read + SDPA, paged gather + SDPA and paged direct
                   (benchmarks/attention_micro.py:27-85), plus the direct
                   kernel on the contiguous layout
  context_sweep    decode step latency against context length per system
                   (benchmarks/context_sweep.py:50-126), in interleaved rounds
                   with paired deltas per context
  ab_compare       interleaved rounds of every system with a rotating start,
                   paired per-round deltas and a Student-t 95 % interval
                   (benchmarks/ab_compare.py:49-198)
  moe_ab_compare   the same for the MoE decode path: 'reference' (PyTorch
                   per-expert) against 'direct' (fused HIP) on one cache
                   system (benchmarks/moe_ab_compare.py:66-200)

On a GPU, ab_compare, context_sweep and attention_micro (rounds > 1) start
every round from fresh memory: cached blocks are handed back to the driver,
a random-size pad is allocated, and then every system's cache (and graph) is
allocated anew, in the round's order, so paired deltas average over where the
pools land in device memory instead of inheriting one placement.

System names are the reference's: "contiguous", "paged-gather",
"paged-direct", plus
  "paged-direct-graph"       paged-direct with each decode step replayed from
                             a captured HIP graph (moe_engine.graphs),
                             captured again in every round;
  "contiguous-direct"        the contiguous cache's layout run by the same
                             fused kernels as paged-direct (a one-block pool,
                             contiguous_direct_cache), so that paged-direct
                             minus it is the cost of paging alone;
  "contiguous-direct-graph"  the same, replayed from a graph.
The reference's "contiguous" system runs PyTorch attention (and, on a GPU,
this engine's fused MoE half), so paged-direct minus contiguous also counts
the fused attention kernels.  Run as a module for a JSON report:

    python -m moe_engine.harness ab --rounds 21 --new-tokens 64
    python -m moe_engine.harness sweep --rounds 21 --contexts 16,64,256,1024
    python -m moe_engine.harness micro --rounds 21
    python -m moe_engine.harness moe-ab --rounds 9 --systems contiguous
"""

import argparse
import gc
import json
import math
import random
import statistics
import time

import torch
import torch.nn.functional as F

from moe_engine import _native, paged_attention, projection
from moe_engine.model import BlockAllocator, KVCache, Model, ModelConfig

SYSTEMS = ("contiguous", "paged-gather", "paged-direct")
GRAPH_SYSTEM = "paged-direct-graph"
CONTIGUOUS_DIRECT = "contiguous-direct"
CONTIGUOUS_DIRECT_GRAPH = "contiguous-direct-graph"
ALL_SYSTEMS = SYSTEMS + (GRAPH_SYSTEM, CONTIGUOUS_DIRECT, CONTIGUOUS_DIRECT_GRAPH)

# the miniMoE-shaped decoder.
CONFIG1 = dict(max_seq_length=1024, vocab_size=50257, num_layers=12, hidden_dim=768, num_heads=12,
               num_experts=8, top_k=2, ffn_dim=2048)


def sync(device) -> None:
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize()


def time_calls(fn, sync_fn, iters=200, warmup=20) -> float:
    """Average microseconds per call over back-to-back calls (no per-call sync)."""
    for _ in range(warmup):
        fn()
    sync_fn()
    start = time.perf_counter()
    for _ in range(iters):
        fn()
    sync_fn()
    return (time.perf_counter() - start) / iters * 1e6


def make_model(config=None, seed=0, device="cuda", dtype=torch.float32):
    torch.manual_seed(seed)
    return Model(ModelConfig(**(config or CONFIG1))).to(device, dtype).eval()


def contiguous_direct_cache(model):
    """The contiguous cache (KVCache, model.py:30-58) in the form the fused
    kernels take: one pool block of max_seq_length tokens.  The pools are
    [layers, 1, heads, max_seq_length, head_dim] - KVCache's k / v tensors
    for batch 1, element for element - and the block table is [0], so token t
    sits at offset t * head_dim of its head's row, as in KVCache.  The
    append, the decode and the graph step run unchanged on it."""
    return model.new_block_allocator(1, model.max_seq_length, attention_mode="direct").new_cache()


def is_graph_system(system) -> bool:
    return system.endswith("-graph")


def make_cache(model, system, block_size=16):
    """A fresh cache for `system`; paged pools hold one max-length sequence
    (scripts/serve.py:147-155)."""
    if system == "contiguous":
        return model.new_cache()
    if system in (CONTIGUOUS_DIRECT, CONTIGUOUS_DIRECT_GRAPH):
        return contiguous_direct_cache(model)
    num_blocks = -(-model.max_seq_length // block_size)
    mode = "direct" if system == GRAPH_SYSTEM else system[len("paged-"):]
    return model.new_block_allocator(num_blocks, block_size, attention_mode=mode).new_cache()


def release(cache):
    if hasattr(cache, "free"):
        cache.free()


def greedy_pick(logits):
    """The next token from [1, S, vocab] logits: the argmax of the last
    position, as the reference's timed loop takes it
    (benchmarks/ab_compare.py:58,64).  On a ROCm device it is one library
    launch, the pick Model.generate makes at temperature 0 (the merge of the
    LM head's kept picks, or mie_argmax over a float32 row); else
    torch.argmax.  Both give torch.argmax's index (first maximum, NaN largest)."""
    last = logits[:, -1, :]
    if last.is_contiguous() and projection.can_argmax(last.reshape(-1)):
        return projection.argmax(last.reshape(-1)).view(1, 1)
    return last.argmax(dim=-1, keepdim=True)


def run_round(model, cache, prompt_ids, new_tokens, warm_steps=0):
    """One prefill, `warm_steps` untimed greedy decode steps, then
    `new_tokens` timed ones; returns (prefill seconds, per-step seconds,
    generated tokens - the warm steps' included)."""
    device = prompt_ids.device
    tokens = []
    with torch.no_grad():
        sync(device)
        start = time.perf_counter()
        logits = model(prompt_ids.unsqueeze(0), cache)
        sync(device)
        prefill_s = time.perf_counter() - start
        step_input = greedy_pick(logits)
        for _ in range(warm_steps):
            step_input = greedy_pick(model(step_input, cache))
            tokens.append(int(step_input))
        steps = []
        for _ in range(new_tokens):
            sync(device)
            start = time.perf_counter()
            logits = model(step_input, cache)
            step_input = greedy_pick(logits)
            sync(device)
            steps.append(time.perf_counter() - start)
            tokens.append(int(step_input))
    return prefill_s, steps, tokens


def run_round_graphed(model, cache, prompt_ids, new_tokens):
    """run_round for a graph system on a fresh cache: the prefill, one untimed
    step that runs eagerly and captures the step graph (moe_engine.graphs),
    then `new_tokens` timed replays."""
    from moe_engine.graphs import GraphedDecoder

    device = prompt_ids.device
    tokens = []
    with torch.no_grad():
        sync(device)
        start = time.perf_counter()
        logits = model(prompt_ids.unsqueeze(0), cache)
        sync(device)
        prefill_s = time.perf_counter() - start
        decoder = GraphedDecoder(model, cache)
        decoder.prime(greedy_pick(logits))
        tokens.append(int(decoder.step()))  # eager step + capture
        steps = []
        for _ in range(new_tokens):
            sync(device)
            start = time.perf_counter()
            step_input = decoder.step()
            sync(device)
            steps.append(time.perf_counter() - start)
            tokens.append(int(step_input))
    return prefill_s, steps, tokens


# Placement sampling: the largest random pad (MiB) taken before a round's
# caches are allocated.
PAD_MAX_MIB = 256


def fresh_placement(rng, device):
    """Hand every cached block back to the driver and take a pad allocation of
    1 .. PAD_MAX_MIB MiB (drawn from `rng`), so that the caches, graphs and
    launch-plan buffers allocated next land somewhere else in device memory
    than in the last round.  Returns the pad (None off the GPU); hold it until
    the round's allocations are made."""
    if torch.device(device).type != "cuda":
        return None
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return torch.empty(rng.randint(1, PAD_MAX_MIB) << 20, dtype=torch.uint8, device=device)


def round_order(systems, r):
    """Round r's order: the systems rotated by r // 2, and reversed in odd
    rounds, so each system starts (and allocates first) in turn and every
    pair runs in both orders equally often over each two rounds (the
    reference's sweep reverses its order on odd passes,
    benchmarks/context_sweep.py:104-110)."""
    k = (r // 2) % len(systems)
    order = systems[k:] + systems[:k]
    return order[::-1] if r % 2 else order


def paired_t_summary(deltas):
    """Mean and two-sided 95 % Student-t interval of paired per-round deltas (ms)."""
    n = len(deltas)
    mean = sum(deltas) / n
    if n < 2:
        return {"per_round_delta_ms": deltas, "mean_delta_ms": round(mean, 4), "ci95_ms": None}
    from scipy.stats import t as student_t

    half = student_t.ppf(0.975, n - 1) * math.sqrt(statistics.variance(deltas) / n)
    return {
        "per_round_delta_ms": [round(d, 4) for d in deltas],
        "mean_delta_ms": round(mean, 4),
        "ci95_ms": [round(mean - half, 4), round(mean + half, 4)],
    }


# Pairs (a, b) reported as a - b when both systems ran.  The two paging-cost
# pairs compare the same kernels on the two layouts.
PAIRS = (("paged-direct", "contiguous"), ("paged-direct", "paged-gather"), ("paged-gather", "contiguous"),
         (GRAPH_SYSTEM, "paged-direct"), (GRAPH_SYSTEM, "contiguous"),
         ("paged-direct", CONTIGUOUS_DIRECT), (GRAPH_SYSTEM, CONTIGUOUS_DIRECT_GRAPH))
PAGING_COST_PAIRS = (("paged-direct", CONTIGUOUS_DIRECT), (GRAPH_SYSTEM, CONTIGUOUS_DIRECT_GRAPH))


def paired_deltas(round_means, systems):
    """Paired per-round deltas of PAIRS from per-system per-round means (ms)."""
    return {f"{a}_minus_{b}": paired_t_summary([x - y for x, y in zip(round_means[a], round_means[b])])
            for a, b in PAIRS if a in systems and b in systems}


def ab_compare(model, prompt_ids, systems=SYSTEMS, rounds=21, new_tokens=64, block_size=16, seed=0,
               placement=True):
    """Interleaved rounds of every system (benchmarks/ab_compare.py:75-144).

    Each round takes its own order of the systems (round_order).  With `placement` (on a
    GPU) every round also starts from fresh memory: the caching allocator's
    blocks are handed back and a random-size pad is taken (fresh_placement),
    then every system's cache is allocated, in the round's order, and each
    graph system captures its step again, so paired deltas average over
    memory placement instead of inheriting one.  Each system decodes one
    untimed step after the prefill (for a graph system the eager step that
    captures), then `new_tokens` timed steps; a warm-up round runs first."""
    systems = list(systems)
    rng = random.Random(seed)
    device = prompt_ids.device

    def one_round(order):
        pad = fresh_placement(rng, device) if placement else None
        caches = {s: make_cache(model, s, block_size) for s in order}
        out = {}
        try:
            for s in order:
                if is_graph_system(s):
                    out[s] = run_round_graphed(model, caches[s], prompt_ids, new_tokens)
                else:
                    out[s] = run_round(model, caches[s], prompt_ids, new_tokens, warm_steps=1)
                release(caches[s])
        finally:
            for c in caches.values():
                release(c)
            del caches, pad
        return out

    one_round(systems)  # warm-up, outside the timed rounds
    results = {s: {"prefill_s": [], "rounds": [], "tokens": None} for s in systems}
    for r in range(rounds):
        for system, (prefill_s, steps, tokens) in one_round(round_order(systems, r)).items():
            results[system]["prefill_s"].append(prefill_s)
            results[system]["rounds"].append(steps)
            results[system]["tokens"] = tokens
    summary = {}
    for system in systems:
        pooled = sorted(t for steps in results[system]["rounds"] for t in steps)
        summary[system] = {
            "prefill_ms": round(statistics.median(results[system]["prefill_s"]) * 1e3, 3),
            "decode_median_ms": round(pooled[len(pooled) // 2] * 1e3, 3),
            "decode_mean_ms": round(sum(pooled) / len(pooled) * 1e3, 3),
            "decode_p90_ms": round(pooled[int(len(pooled) * 0.9)] * 1e3, 3),
            "decode_tok_per_sec": round(len(pooled) / sum(pooled), 2),
        }
    round_means = {s: [sum(steps) / len(steps) * 1e3 for steps in results[s]["rounds"]] for s in systems}
    tokens = [results[s]["tokens"] for s in systems]
    return {
        "summary": summary,
        "paired_deltas": paired_deltas(round_means, systems),
        "tokens_identical": all(t == tokens[0] for t in tokens),
        "tokens": tokens[0],
        "rounds": rounds,
        "new_tokens": new_tokens,
        "prompt_tokens": int(prompt_ids.numel()),
        "placement_sampled": bool(placement and device.type == "cuda"),
    }


MOE_AB_MODES = ("reference", "direct")


def moe_ab_compare(model, prompt_ids, rounds=9, new_tokens=64, system="contiguous", block_size=16):
    """The MoE decode path A/B of benchmarks/moe_ab_compare.py:66-200: the
    same prompt and cache system decoded greedily with the MoE in
    'reference' mode (the PyTorch per-expert path) and in 'direct' mode (the
    fused HIP kernels), interleaved over `rounds` rounds whose first mode
    alternates, after one short warm-up round per mode.  Reports each mode's
    step statistics with per-round totals, the paired per-round delta
    direct - reference with its 95 % interval, and whether both modes chose
    the same tokens.  The model's MoE modes are restored afterwards."""
    if rounds < 2 or new_tokens < 1:
        raise ValueError("moe_ab_compare needs at least 2 rounds and 1 new token")
    if is_graph_system(system):
        raise ValueError("moe_ab_compare runs eager systems; the reference MoE path cannot be captured")
    saved = [block.moe.mode for block in model.MoEBlocks]

    def decode(mode, tokens):
        model.set_moe_mode(mode)
        cache = make_cache(model, system, block_size)
        try:
            return run_round(model, cache, prompt_ids, tokens)
        finally:
            release(cache)

    try:
        for mode in MOE_AB_MODES:
            decode(mode, min(new_tokens, 8))
        runs = {mode: [] for mode in MOE_AB_MODES}
        for r in range(rounds):
            first = r % 2
            for mode in MOE_AB_MODES[first:] + MOE_AB_MODES[:first]:
                runs[mode].append(decode(mode, new_tokens))
    finally:
        for block, mode in zip(model.MoEBlocks, saved):
            block.moe.set_mode(mode)

    summary, round_means = {}, {}
    for mode, results in runs.items():
        pooled = sorted(t for _, steps, _ in results for t in steps)
        totals = [sum(steps) for _, steps, _ in results]
        round_means[mode] = [sum(steps) / len(steps) * 1e3 for _, steps, _ in results]
        summary[mode] = {
            "prefill_median_ms": round(statistics.median(p for p, _, _ in results) * 1e3, 3),
            "total_decode_steps": len(pooled),
            "total_decode_s": round(sum(pooled), 6),
            "decode_median_ms": round(statistics.median(pooled) * 1e3, 3),
            "decode_p90_ms": round(pooled[int(len(pooled) * 0.9)] * 1e3, 3),
            "decode_tok_per_sec": round(len(pooled) / sum(pooled), 3),
            "per_round_total_decode_ms": [round(t * 1e3, 3) for t in totals],
            "per_round_decode_tok_per_sec": [round(new_tokens / t, 3) for t in totals],
            "per_round_mean_ms": [round(m, 4) for m in round_means[mode]],
        }
    token_sets = {mode: [tokens for _, _, tokens in results] for mode, results in runs.items()}
    reference_tokens = token_sets["reference"][0]
    return {
        "system": system,
        "summary": summary,
        "paired_delta_direct_minus_reference": paired_t_summary(
            [d - r for d, r in zip(round_means["direct"], round_means["reference"])]),
        "tokens_identical": all(t == reference_tokens for ts in token_sets.values() for t in ts),
        "rounds": rounds,
        "new_tokens": new_tokens,
        "prompt_tokens": int(prompt_ids.numel()),
    }


def stepwise_logits(model, seq, cache, prompt_len):
    """Logits [T, vocab] for every position of `seq` ([1, T] ids): the prompt
    as one prefill, then one decode step per later token (teacher forcing)."""
    with torch.no_grad():
        rows = [model(seq[:, :prompt_len], cache)[0]]
        for t in range(prompt_len, seq.shape[1]):
            rows.append(model(seq[:, t:t + 1], cache)[0])
    return torch.cat(rows).float()


def parity_report(model, cpu_model, prompt_ids, new_tokens=64, block_size=16, system="paged-direct"):
    """The reference's parity report (scripts/check_parity.py:64-93) for
    `system` on `model`'s device against the CPU contiguous path of the same
    weights (`cpu_model`): greedy tokens of both, and the logits at every
    position of the CPU's greedy sequence - the prefill and each decode step,
    with the same token fed to both - compared as the reference does
    (relative difference over |reference logit| clamped to at least 1)."""
    prompt_cpu = prompt_ids.cpu()
    with torch.no_grad():
        want = cpu_model.generate(prompt_cpu, new_tokens, temperature=0, cache=cpu_model.new_cache())
        cache = make_cache(model, system, block_size)
        got = model.generate(prompt_ids, new_tokens, temperature=0, cache=cache)
        release(cache)
        ref_logits = stepwise_logits(cpu_model, want, cpu_model.new_cache(), len(prompt_cpu))
        cache = make_cache(model, system, block_size)
        logits = stepwise_logits(model, want.to(prompt_ids.device), cache, len(prompt_cpu)).cpu()
        release(cache)
    abs_diff = (ref_logits - logits).abs()
    rel_diff = abs_diff / ref_logits.abs().clamp(min=1.0)
    want, got = want[0].tolist(), got[0].tolist()
    first = next((i for i, (a, b) in enumerate(zip(want, got)) if a != b), None)
    if first is None and len(want) != len(got):
        first = min(len(want), len(got))
    return {
        "engine_cache": system,
        "device": str(prompt_ids.device),
        "reference_path": "CPU, contiguous cache, same seed-0 weights",
        "dtype": str(next(model.parameters()).dtype),
        "prompt_tokens": len(prompt_cpu),
        "positions_compared": int(logits.shape[0]),
        "max_abs_logit_diff": abs_diff.max().item(),
        "max_rel_logit_diff": rel_diff.max().item(),
        "greedy_tokens_compared": len(want) - len(prompt_cpu),
        "first_greedy_mismatch": first,
        "tokens": got,
    }


SWEEP_SYSTEMS = ("contiguous", "paged-gather", "paged-direct", CONTIGUOUS_DIRECT, GRAPH_SYSTEM,
                 CONTIGUOUS_DIRECT_GRAPH)
FILLER_TOKEN = 100  # the fixed token of the sweep's prompts and steps (benchmarks/context_sweep.py:28)


def _sweep_cell(model, cache, system, ctx, steps, filler):
    """One system at one context: a prefill of ctx - steps - 1 filler tokens,
    one untimed decode step (for a graph system the eager step that captures
    the graph), then `steps` timed one-token steps, the last attending over
    `ctx` tokens.  Eager steps feed the fixed filler token, as the reference's
    sweep does (benchmarks/context_sweep.py:50-78); a graph step feeds back its
    own pick.  Returns the per-step seconds."""
    device = model.token_embedding.weight.device
    prefill = max(1, ctx - steps - 1)
    n = min(steps, model.max_seq_length - prefill - 1)
    prompt = torch.full((1, prefill), filler, device=device, dtype=torch.long)
    token = torch.full((1, 1), filler, device=device, dtype=torch.long)
    times = []
    with torch.no_grad():
        model(prompt, cache)
        if is_graph_system(system):
            from moe_engine.graphs import GraphedDecoder

            decoder = GraphedDecoder(model, cache)
            decoder.prime(token)
            decoder.step()
            step = decoder.step
        else:
            model(token, cache)
            step = lambda: model(token, cache)  # noqa: E731
        for _ in range(n):
            sync(device)
            start = time.perf_counter()
            step()
            sync(device)
            times.append(time.perf_counter() - start)
    return times


def context_sweep(model, contexts=(16, 64, 256, 1024), systems=SWEEP_SYSTEMS, rounds=21, steps=16, block_size=16,
                  filler=FILLER_TOKEN, seed=0, placement=True):
    """Decode-step latency against context length (benchmarks/context_sweep.py:
    50-126), in interleaved rounds with paired deltas.

    Each round visits every context; at each context the systems run in the
    round's order (round_order), each on a fresh cache allocated (in that order)
    behind a fresh random pad (fresh_placement, with `placement` on a GPU).
    Reports per context: the median step time of every system over the pooled
    steps of all rounds, and the paired per-round deltas of PAIRS with 95 %
    Student-t intervals - among them the cost of paging alone,
    paged-direct - contiguous-direct, eager and graphed."""
    systems = list(systems)
    rng = random.Random(seed)
    device = model.token_embedding.weight.device

    def visit(ctx, order):
        pad = fresh_placement(rng, device) if placement else None
        caches = {s: make_cache(model, s, block_size) for s in order}
        try:
            return {s: _sweep_cell(model, caches[s], s, ctx, steps, filler) for s in order}
        finally:
            for c in caches.values():
                release(c)
            del caches, pad

    visit(contexts[0], systems)  # warm-up, outside the timed rounds
    times = {ctx: {s: [] for s in systems} for ctx in contexts}
    for r in range(rounds):
        for ctx in contexts:
            for system, steps_s in visit(ctx, round_order(systems, r)).items():
                times[ctx][system].append(steps_s)
    median_ms, deltas, paging = {s: {} for s in systems}, {}, {}
    for ctx in contexts:
        round_means = {}
        for s in systems:
            pooled = sorted(t for rnd in times[ctx][s] for t in rnd)
            median_ms[s][ctx] = round(pooled[len(pooled) // 2] * 1e3, 4)
            round_means[s] = [sum(rnd) / len(rnd) * 1e3 for rnd in times[ctx][s]]
        deltas[ctx] = paired_deltas(round_means, systems)
        paging[ctx] = {f"{a}_minus_{b}": {k: deltas[ctx][f"{a}_minus_{b}"][k] for k in ("mean_delta_ms", "ci95_ms")}
                       for a, b in PAGING_COST_PAIRS if f"{a}_minus_{b}" in deltas[ctx]}
    return {
        "median_step_ms": median_ms,
        "paired_deltas": deltas,
        "paging_cost_ms": paging,
        "rounds": rounds,
        "steps_per_context": steps,
        "placement_sampled": bool(placement and device.type == "cuda"),
    }


def _graph_device_us(calls, reps=5):
    """Device time per call of `calls` captured back to back in one HIP graph
    (median of `reps` replays, HIP events around each)."""
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
    del graph
    return statistics.median(times)


MICRO_VARIANTS = ("contiguous_read_sdpa_us", "paged_gather_sdpa_us", "paged_direct_kernel_us",
                  "contiguous_direct_kernel_us")


def attention_micro(config=None, contexts=(16, 64, 256, 1024), device="cuda", dtype=torch.float32, iters=200,
                    rounds=1, seed=0, placement=True):
    """One layer's decode attention in isolation, us per call
    (benchmarks/attention_micro.py:27-85): contiguous read + SDPA, paged
    gather + SDPA and the paged direct kernel, plus the same kernel on the
    contiguous layout (a one-block pool: contiguous_direct_kernel_us), timed
    as back-to-back calls without per-call syncs after 20 warm-up calls, in
    each round's order of the variants (round_order).

    With rounds > 1 every round allocates the caches afresh behind a random
    pad (fresh_placement) and refills them; the report then gives each
    variant's median over rounds, and for the two direct variants also the
    device time per call from 64 calls replayed from a HIP graph, with the
    paired per-round deltas paged - contiguous (host-launched and device)."""
    cfg = ModelConfig(**(config or CONFIG1))
    max_ctx = cfg.max_seq_length
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    shape = (1, cfg.num_heads, max_ctx, cfg.head_dim)
    k = torch.randn(shape, generator=gen).to(device, dtype)
    v = torch.randn(shape, generator=gen).to(device, dtype)
    q = torch.randn(1, cfg.num_heads, 1, cfg.head_dim, generator=gen).to(device, dtype)
    s = lambda: sync(device)  # noqa: E731
    on_gpu = torch.device(device).type == "cuda"
    per = {ctx: {name: [] for name in MICRO_VARIANTS + ("paged_direct_device_us", "contiguous_direct_device_us")}
           for ctx in contexts}
    for r in range(rounds):
        pad = fresh_placement(rng, device) if placement and rounds > 1 else None
        contiguous = KVCache(cfg, 1, device, dtype)
        paged = BlockAllocator(cfg, max_ctx // 16, 16, device, dtype).new_cache()
        contiguous_direct = BlockAllocator(cfg, 1, max_ctx, device, dtype, attention_mode="direct").new_cache()
        for cache in (contiguous, paged, contiguous_direct):
            cache.write(0, 0, k, v)
        direct = paged_attention.is_supported(q, cfg.head_dim)
        for ctx in contexts:
            row = per[ctx]
            calls = {
                "contiguous_read_sdpa_us": lambda: F.scaled_dot_product_attention(q, *contiguous.read(0, ctx)),
                "paged_gather_sdpa_us": lambda: F.scaled_dot_product_attention(q, *paged.read(0, ctx)),
            }
            if direct:
                calls["paged_direct_kernel_us"] = lambda: paged_attention.decode(q, paged, 0, ctx)
                calls["contiguous_direct_kernel_us"] = lambda: paged_attention.decode(q, contiguous_direct, 0, ctx)
            for name in round_order(list(calls), r):
                row[name].append(time_calls(calls[name], s, iters))
            if direct and on_gpu:
                graphed = {"paged_direct_device_us": calls["paged_direct_kernel_us"],
                           "contiguous_direct_device_us": calls["contiguous_direct_kernel_us"]}
                for name in round_order(list(graphed), r):
                    row[name].append(_graph_device_us([graphed[name]] * 64))
        release(paged)
        release(contiguous_direct)
        del contiguous, paged, contiguous_direct, pad
    results = {}
    for ctx in contexts:
        row = {name: round(statistics.median(vals), 2) for name, vals in per[ctx].items() if vals}
        if rounds > 1:
            for kind, a, b in (("host_launched", "paged_direct_kernel_us", "contiguous_direct_kernel_us"),
                               ("device", "paged_direct_device_us", "contiguous_direct_device_us")):
                if per[ctx][a] and per[ctx][b]:
                    # paired_t_summary is unit-free apart from its key names;
                    # the deltas go in as us, so its 4 decimals are 0.1 ns.
                    d = paired_t_summary([x - y for x, y in zip(per[ctx][a], per[ctx][b])])
                    row[f"paging_cost_{kind}_us"] = {"mean_delta_us": d["mean_delta_ms"], "ci95_us": d["ci95_ms"]}
        results[ctx] = row
    return results


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("mode", choices=["ab", "moe-ab", "micro", "sweep"])
    parser.add_argument("--rounds", type=int, default=21)
    parser.add_argument("--new-tokens", type=int, default=64)
    parser.add_argument("--prompt-tokens", type=int, default=32)
    parser.add_argument("--contexts", default="16,64,256,1024")
    parser.add_argument("--systems", default=None,
                        help="any of " + ", ".join(ALL_SYSTEMS) + " (moe-ab: one eager system, default contiguous)")
    parser.add_argument("--device", default="cuda")
    parser.add_argument("--copy-calibration-mib", type=int, default=0,
                        help="first run 10 plain device copies of this many MiB (each reads and writes that many "
                        "bytes), to scale hardware byte counters against a kernel of known traffic")
    args = parser.parse_args(argv)
    if args.copy_calibration_mib > 0:
        src = torch.ones(args.copy_calibration_mib << 18, dtype=torch.float32, device=args.device)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        sync(args.device)
        del src, dst
    contexts = [int(c) for c in args.contexts.split(",")]
    default_systems = {"moe-ab": "contiguous", "sweep": ",".join(SWEEP_SYSTEMS)}.get(args.mode, ",".join(SYSTEMS))
    systems = (args.systems or default_systems).split(",")
    if args.mode == "moe-ab" and (len(systems) != 1 or systems[0] not in ALL_SYSTEMS or is_graph_system(systems[0])):
        parser.error("moe-ab takes one eager system: " + ", ".join(s for s in ALL_SYSTEMS if not is_graph_system(s)))
    if args.mode == "moe-ab" and (args.rounds < 2 or args.new_tokens < 1):
        parser.error("--rounds must be at least 2 and --new-tokens positive")
    if args.mode == "micro":
        report = attention_micro(contexts=contexts, device=args.device, rounds=args.rounds)
    else:
        model = make_model(device=args.device)
        if args.mode in ("ab", "moe-ab"):
            gen = torch.Generator().manual_seed(0)
            prompt = torch.randint(0, CONFIG1["vocab_size"], (args.prompt_tokens,), generator=gen).to(args.device)
            if args.mode == "ab":
                report = ab_compare(model, prompt, systems, args.rounds, args.new_tokens)
            else:
                report = moe_ab_compare(model, prompt, args.rounds, args.new_tokens, systems[0])
        else:
            report = context_sweep(model, contexts, systems, rounds=args.rounds)
    print(json.dumps(report, indent=2))


if __name__ == "__main__":
    main()
