"""Latency harnesses for the paged decode path (random-init miniMoE models).

Counterparts of the reference's benchmarks, with random-init weights because
the real checkpoint and tokenizer are not available here:

  attention_micro  one layer's decode attention, us per call, for contiguous
                   read + SDPA, paged gather + SDPA and paged direct
                   (benchmarks/attention_micro.py:27-85)
  context_sweep    decode step latency against context length per system
                   (benchmarks/context_sweep.py:50-113)
  ab_compare       interleaved rounds of every system with a rotating start,
                   paired per-round deltas and a Student-t 95 % interval
                   (benchmarks/ab_compare.py:49-198)
  moe_ab_compare   the same for the MoE decode path: 'reference' (PyTorch
                   per-expert) against 'direct' (fused HIP) on one cache
                   system (benchmarks/moe_ab_compare.py:66-200)

System names are the reference's: "contiguous", "paged-gather",
"paged-direct", plus
  "paged-direct-graph"       paged-direct with each decode step replayed from
                             one captured HIP graph (moe_engine.graphs),
                             captured once in the warm-up and reused for every
                             later round;
  "contiguous-direct"        the contiguous cache's layout run by the same
                             fused kernels as paged-direct (a one-block pool,
                             contiguous_direct_cache), so that paged-direct
                             minus it is the cost of paging alone;
  "contiguous-direct-graph"  the same, replayed from a graph.
The reference's "contiguous" system runs PyTorch attention (and, on a GPU,
this engine's fused MoE half), so paged-direct minus contiguous also counts
the fused attention kernels.  Run as a module for a JSON report:

    python -m moe_engine.harness ab --rounds 5 --new-tokens 64
    python -m moe_engine.harness moe-ab --rounds 9 --systems contiguous
"""

import argparse
import json
import math
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


def attention_micro(config=None, contexts=(16, 64, 256, 1024), device="cuda", dtype=torch.float32, iters=200):
    """One layer's decode attention in isolation, us per call."""
    cfg = ModelConfig(**(config or CONFIG1))
    max_ctx = cfg.max_seq_length
    contiguous = KVCache(cfg, 1, device, dtype)
    allocator = BlockAllocator(cfg, max_ctx // 16, 16, device, dtype)
    paged = allocator.new_cache()
    torch.manual_seed(0)
    shape = (1, cfg.num_heads, max_ctx, cfg.head_dim)
    k = torch.randn(shape, device=device, dtype=dtype)
    v = torch.randn(shape, device=device, dtype=dtype)
    contiguous.write(0, 0, k, v)
    paged.write(0, 0, k, v)
    q = torch.randn(1, cfg.num_heads, 1, cfg.head_dim, device=device, dtype=dtype)
    s = lambda: sync(device)  # noqa: E731
    results = {}
    for ctx in contexts:
        row = {
            "contiguous_read_sdpa_us": time_calls(lambda: F.scaled_dot_product_attention(q, *contiguous.read(0, ctx)), s, iters),
            "paged_gather_sdpa_us": time_calls(lambda: F.scaled_dot_product_attention(q, *paged.read(0, ctx)), s, iters),
        }
        if paged_attention.is_supported(q, cfg.head_dim):
            row["paged_direct_kernel_us"] = time_calls(lambda: paged_attention.decode(q, paged, 0, ctx), s, iters)
        results[ctx] = {key: round(val, 2) for key, val in row.items()}
    return results


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


def run_round(model, cache, prompt_ids, new_tokens):
    """One prefill and `new_tokens` greedy decode steps; returns
    (prefill seconds, per-step seconds, generated tokens)."""
    device = prompt_ids.device
    tokens = []
    with torch.no_grad():
        sync(device)
        start = time.perf_counter()
        logits = model(prompt_ids.unsqueeze(0), cache)
        sync(device)
        prefill_s = time.perf_counter() - start
        step_input = greedy_pick(logits)
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


def run_round_graphed(model, state, prompt_ids, new_tokens):
    """run_round for GRAPH_SYSTEM.  `state` holds one paged-direct cache and its
    GraphedDecoder across rounds: the cache is freed between rounds (its
    device block table, which the graph reads, stays), so the graph captured
    in the first round is replayed in every later one."""
    from moe_engine.graphs import GraphedDecoder

    cache = state["cache"]
    device = prompt_ids.device
    tokens = []
    with torch.no_grad():
        sync(device)
        start = time.perf_counter()
        logits = model(prompt_ids.unsqueeze(0), cache)
        sync(device)
        prefill_s = time.perf_counter() - start
        step_input = greedy_pick(logits)
        if state.get("decoder") is None:
            state["decoder"] = GraphedDecoder(model, cache)
        decoder = state["decoder"]
        decoder.prime(step_input)
        steps = []
        for _ in range(new_tokens):
            sync(device)
            start = time.perf_counter()
            step_input = decoder.step()
            sync(device)
            steps.append(time.perf_counter() - start)
            tokens.append(int(step_input))
    return prefill_s, steps, tokens


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


def ab_compare(model, prompt_ids, systems=SYSTEMS, rounds=5, new_tokens=64, block_size=16):
    """Interleaved rounds of every system, rotating which starts each round."""
    systems = list(systems)
    graph_states = {}

    def run(system):
        if is_graph_system(system):
            state = graph_states.setdefault(system, {})
            if "cache" not in state:
                state["cache"] = make_cache(model, system, block_size)
            try:
                return run_round_graphed(model, state, prompt_ids, new_tokens)
            finally:
                release(state["cache"])
        cache = make_cache(model, system, block_size)
        try:
            return run_round(model, cache, prompt_ids, new_tokens)
        finally:
            release(cache)

    for system in systems:  # warm-up outside the timed rounds
        run(system)
    results = {s: {"prefill_s": [], "rounds": [], "tokens": None} for s in systems}
    for r in range(rounds):
        order = systems[r % len(systems):] + systems[: r % len(systems)]
        for system in order:
            prefill_s, steps, tokens = run(system)
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

    def mean_steps_ms(system):
        return [sum(steps) / len(steps) * 1e3 for steps in results[system]["rounds"]]

    paired = {}
    for a, b in (("paged-direct", "contiguous"), ("paged-direct", "paged-gather"), ("paged-gather", "contiguous"),
                 (GRAPH_SYSTEM, "paged-direct"), (GRAPH_SYSTEM, "contiguous"),
                 ("paged-direct", CONTIGUOUS_DIRECT), (GRAPH_SYSTEM, CONTIGUOUS_DIRECT_GRAPH)):
        if a in systems and b in systems:
            paired[f"{a}_minus_{b}"] = paired_t_summary([x - y for x, y in zip(mean_steps_ms(a), mean_steps_ms(b))])
    tokens = [results[s]["tokens"] for s in systems]
    return {
        "summary": summary,
        "paired_deltas": paired,
        "tokens_identical": all(t == tokens[0] for t in tokens),
        "tokens": tokens[0],
        "rounds": rounds,
        "new_tokens": new_tokens,
        "prompt_tokens": int(prompt_ids.numel()),
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


def context_sweep(model, contexts=(16, 64, 256, 1024), systems=SYSTEMS, steps=16, block_size=16, filler=0):
    """Median decode-step latency (ms) at roughly each context length."""
    device = model.token_embedding.weight.device
    report = {s: {} for s in systems}
    for ctx in contexts:
        for system in systems:
            prefill = max(1, ctx - steps)
            cache = make_cache(model, system, block_size)
            prompt = torch.full((1, prefill), filler, device=device, dtype=torch.long)
            step = torch.full((1, 1), filler, device=device, dtype=torch.long)
            times = []
            with torch.no_grad():
                model(prompt, cache)
                for _ in range(min(steps, model.max_seq_length - prefill)):
                    sync(device)
                    start = time.perf_counter()
                    model(step, cache)
                    sync(device)
                    times.append(time.perf_counter() - start)
            release(cache)
            report[system][ctx] = round(statistics.median(times) * 1e3, 3)
    return report


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("mode", choices=["ab", "moe-ab", "micro", "sweep"])
    parser.add_argument("--rounds", type=int, default=5)
    parser.add_argument("--new-tokens", type=int, default=64)
    parser.add_argument("--prompt-tokens", type=int, default=32)
    parser.add_argument("--contexts", default="16,64,256,1024")
    parser.add_argument("--systems", default=None,
                        help="any of " + ", ".join(ALL_SYSTEMS) + " (moe-ab: one eager system, default contiguous)")
    parser.add_argument("--device", default="cuda")
    args = parser.parse_args(argv)
    contexts = [int(c) for c in args.contexts.split(",")]
    systems = (args.systems or ("contiguous" if args.mode == "moe-ab" else ",".join(SYSTEMS))).split(",")
    if args.mode == "moe-ab" and (len(systems) != 1 or systems[0] not in ALL_SYSTEMS or is_graph_system(systems[0])):
        parser.error("moe-ab takes one eager system: " + ", ".join(s for s in ALL_SYSTEMS if not is_graph_system(s)))
    if args.mode == "moe-ab" and (args.rounds < 2 or args.new_tokens < 1):
        parser.error("--rounds must be at least 2 and --new-tokens positive")
    if args.mode == "micro":
        report = attention_micro(contexts=contexts, device=args.device)
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
            report = context_sweep(model, contexts, systems)
    print(json.dumps(report, indent=2))


if __name__ == "__main__":
    main()
