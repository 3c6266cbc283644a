"""Host-side pieces of the latency harness on the CPU: the contiguous-direct
system's cache is the contiguous cache's layout, the parity report (the
reference's scripts/check_parity.py schema) of a path against itself, and the
timed loop's greedy pick (torch.argmax's index; on the GPU through mie_argmax)."""

import pytest
import torch

from moe_engine import harness
from moe_engine.model import Model, ModelConfig

TINY = dict(max_seq_length=40, vocab_size=96, num_layers=2, hidden_dim=32, num_heads=4, num_experts=4, top_k=2)


def test_contiguous_direct_cache_is_the_contiguous_layout():
    """One pool block of max_seq_length tokens: after the same writes the
    pools hold KVCache's k / v element for element."""
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).eval()
    paged = harness.contiguous_direct_cache(model)
    contiguous = model.new_cache()
    assert paged.allocator.k_pool.shape == contiguous.k.shape  # [L, 1, H, max_seq, D]
    assert paged.attention_mode == "direct" and paged.allocator.block_size == TINY["max_seq_length"]
    k = torch.randn(1, 4, 7, 8)
    v = torch.randn(1, 4, 7, 8)
    for cache in (paged, contiguous):
        cache.write(1, 0, k, v)
        cache.write(1, 7, k[:, :, :1], v[:, :, :1])
    assert paged.block_table == [0]
    assert torch.equal(paged.allocator.k_pool, contiguous.k) and torch.equal(paged.allocator.v_pool, contiguous.v)


def test_parity_report_of_a_path_against_itself():
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).eval()
    prompt = torch.randint(0, TINY["vocab_size"], (5,), generator=torch.Generator().manual_seed(1))
    rep = harness.parity_report(model, model, prompt, new_tokens=6, block_size=4, system="paged-gather")
    assert rep["max_abs_logit_diff"] < 1e-5 and rep["max_rel_logit_diff"] < 1e-5
    assert rep["first_greedy_mismatch"] is None
    assert rep["positions_compared"] == len(rep["tokens"]) == 5 + rep["greedy_tokens_compared"]


def test_graph_systems_and_pairs_are_named():
    assert harness.is_graph_system(harness.GRAPH_SYSTEM) and harness.is_graph_system("contiguous-direct-graph")
    assert not harness.is_graph_system("paged-direct")
    assert set(harness.SYSTEMS) < set(harness.ALL_SYSTEMS)


def _pick_cases(device):
    g = torch.Generator().manual_seed(4)
    base = torch.randn(1, 3, 1000, generator=g)
    tie = base.clone()
    tie[0, -1, [17, 400, 901]] = 50.0  # the first of equal maxima
    nan = base.clone()
    nan[0, -1, [33, 700]] = float("nan")  # NaN counts as the largest
    only_last_row = base.clone()
    only_last_row[0, 0, 5] = 99.0  # a larger value outside the last position is ignored
    return [t.to(device) for t in (base, tie, nan, only_last_row)]


def test_greedy_pick_is_torch_argmax_of_the_last_position():
    for logits in _pick_cases("cpu"):
        assert torch.equal(harness.greedy_pick(logits), logits[:, -1, :].argmax(dim=-1, keepdim=True))


@pytest.mark.gpu
def test_greedy_pick_on_the_gpu_is_one_mie_argmax_with_torch_order():
    """On a ROCm device the harness picks through mie_argmax (as Model.generate
    does): the same index as torch.argmax, ties and NaN included."""
    for logits in _pick_cases("cuda"):
        want = logits[:, -1, :].float().cpu().argmax(dim=-1, keepdim=True)
        got = harness.greedy_pick(logits)
        assert got.shape == (1, 1) and got.dtype == torch.int64
        assert torch.equal(got.cpu(), want)


def test_moe_ab_rejects_what_the_reference_rejects():
    model = Model(ModelConfig(**TINY)).eval()
    prompt = torch.zeros(3, dtype=torch.long)
    with pytest.raises(ValueError, match="2 rounds"):
        harness.moe_ab_compare(model, prompt, rounds=1)
    with pytest.raises(ValueError, match="2 rounds"):
        harness.moe_ab_compare(model, prompt, rounds=2, new_tokens=0)
    with pytest.raises(ValueError, match="eager"):
        harness.moe_ab_compare(model, prompt, rounds=2, system=harness.GRAPH_SYSTEM)
    # The command line refuses the same before it builds a model.
    for argv in (["moe-ab", "--rounds", "1"], ["moe-ab", "--new-tokens", "0"],
                 ["moe-ab", "--systems", "paged-direct-graph"], ["moe-ab", "--systems", "contiguous,paged-direct"],
                 ["moe-ab", "--systems", "no-such-system"]):
        with pytest.raises(SystemExit):
            harness.main(argv + ["--device", "cpu"])


def test_moe_ab_alternates_modes_and_restores_them(monkeypatch):
    """Warm-up of each mode at min(new_tokens, 8) tokens, then rounds whose
    first mode alternates; every round decodes on a fresh cache of the
    chosen system; the summary's per-round figures and the paired delta come
    from the rounds' step times; the blocks get their own modes back."""
    model = Model(ModelConfig(**TINY)).eval()
    model.MoEBlocks[1].moe.set_mode("reference")
    calls = []
    step_ms = {"reference": 3.0, "direct": 1.0}

    def fake_round(m, cache, prompt_ids, new_tokens):
        modes = {block.moe.mode for block in m.MoEBlocks}
        assert len(modes) == 1  # the whole model runs one mode at a time
        mode = modes.pop()
        calls.append((mode, new_tokens, type(cache).__name__))
        r = sum(1 for c in calls if c[0] == mode)
        return 0.5, [(step_ms[mode] + 0.1 * r) * 1e-3] * new_tokens, [7] * new_tokens

    monkeypatch.setattr(harness, "run_round", fake_round)
    prompt = torch.zeros(4, dtype=torch.long)
    rep = harness.moe_ab_compare(model, prompt, rounds=3, new_tokens=12, system="paged-gather")
    assert [c[:2] for c in calls] == [("reference", 8), ("direct", 8),
                                      ("reference", 12), ("direct", 12),
                                      ("direct", 12), ("reference", 12),
                                      ("reference", 12), ("direct", 12)]
    assert {c[2] for c in calls} == {"PagedKVCache"}
    assert [block.moe.mode for block in model.MoEBlocks] == ["auto", "reference"]
    ref, direct = rep["summary"]["reference"], rep["summary"]["direct"]
    assert ref["total_decode_steps"] == direct["total_decode_steps"] == 36
    assert ref["per_round_mean_ms"] == pytest.approx([3.2, 3.3, 3.4])
    assert direct["per_round_total_decode_ms"] == pytest.approx([12 * 1.2, 12 * 1.3, 12 * 1.4])
    delta = rep["paired_delta_direct_minus_reference"]
    assert delta["mean_delta_ms"] == pytest.approx(-2.0) and delta["ci95_ms"] == pytest.approx([-2.0, -2.0])
    assert rep["tokens_identical"] and rep["system"] == "paged-gather" and rep["prompt_tokens"] == 4


def test_moe_ab_restores_modes_when_a_round_fails(monkeypatch):
    model = Model(ModelConfig(**TINY)).eval()

    def failing_round(m, cache, prompt_ids, new_tokens):
        if m.MoEBlocks[0].moe.mode == "direct":
            raise RuntimeError("direct MoE decode is unavailable")
        return 0.1, [1e-3] * new_tokens, [1] * new_tokens

    monkeypatch.setattr(harness, "run_round", failing_round)
    with pytest.raises(RuntimeError, match="unavailable"):
        harness.moe_ab_compare(model, torch.zeros(2, dtype=torch.long), rounds=2, new_tokens=2)
    assert [block.moe.mode for block in model.MoEBlocks] == ["auto", "auto"]


@pytest.mark.gpu
def test_moe_ab_on_the_gpu_decodes_the_same_tokens_both_ways():
    """The real A/B on a small model: the PyTorch per-expert MoE and the fused
    HIP MoE choose the same greedy tokens on the contiguous and paged-direct
    systems, and the report carries both modes and the paired delta."""
    cfg = dict(max_seq_length=64, vocab_size=512, num_layers=2, hidden_dim=64, num_heads=4, num_experts=4, top_k=2)
    model = harness.make_model(cfg, device="cuda")
    assert all(block.moe.direct_configuration_supported(1) for block in model.MoEBlocks)
    prompt = torch.randint(0, cfg["vocab_size"], (6,), generator=torch.Generator().manual_seed(3)).cuda()
    for system in ("contiguous", "paged-direct"):
        rep = harness.moe_ab_compare(model, prompt, rounds=2, new_tokens=5, system=system)
        assert rep["tokens_identical"], system
        assert set(rep["summary"]) == {"reference", "direct"}
        assert rep["summary"]["direct"]["total_decode_steps"] == 10
        assert len(rep["paired_delta_direct_minus_reference"]["per_round_delta_ms"]) == 2
    assert {block.moe.mode for block in model.MoEBlocks} == {"auto"}


def test_rounds_rotate_the_systems_and_allocate_in_that_order(monkeypatch):
    """ab_compare and context_sweep: a warm-up visit, then in round r the
    systems allocate their caches and run in round_order(systems, r) -
    rotated by r // 2, reversed in odd rounds; the paired deltas come from
    the per-round means."""
    model = Model(ModelConfig(**TINY)).eval()
    systems = ["contiguous", "paged-gather", "paged-direct"]
    made, ran = [], []
    step_ms = {"contiguous": 2.0, "paged-gather": 3.0, "paged-direct": 1.0}

    def fake_cache(m, system, block_size=16):
        made.append(system)
        return system

    def fake_cell(m, cache, system, ctx, steps, filler):
        ran.append((system, ctx))
        return [step_ms[system] * 1e-3] * steps

    monkeypatch.setattr(harness, "make_cache", fake_cache)
    monkeypatch.setattr(harness, "_sweep_cell", fake_cell)
    rep = harness.context_sweep(model, contexts=(16, 24), systems=systems, rounds=3, steps=2)
    visits = [made[i:i + 3] for i in range(0, len(made), 3)]
    assert visits[0] == systems  # warm-up
    a, b, c = systems
    # rounds 0, 1, 2, each at contexts 16 and 24
    assert visits[1:] == [[a, b, c], [a, b, c], [c, b, a], [c, b, a], [b, c, a], [b, c, a]]
    assert [s for s, _ in ran] == made
    assert rep["median_step_ms"]["paged-direct"] == {16: 1.0, 24: 1.0}
    d = rep["paired_deltas"][24]["paged-direct_minus_contiguous"]
    assert d["mean_delta_ms"] == pytest.approx(-1.0) and d["ci95_ms"] == pytest.approx([-1.0, -1.0])
    assert not rep["placement_sampled"]  # no pad on the CPU

    made.clear()

    def fake_round(m, cache, prompt_ids, new_tokens, warm_steps=0):
        assert warm_steps == 1
        return 0.1, [step_ms[cache] * 1e-3] * new_tokens, [5] * (new_tokens + 1)

    monkeypatch.setattr(harness, "run_round", fake_round)
    rep = harness.ab_compare(model, torch.zeros(3, dtype=torch.long), systems, rounds=4, new_tokens=3)
    assert made[:3] == systems and made[3:6] == systems and made[6:9] == systems[::-1]
    assert made[9:12] == systems[1:] + systems[:1] and made[12:15] == (systems[1:] + systems[:1])[::-1]
    assert rep["paired_deltas"]["paged-gather_minus_contiguous"]["mean_delta_ms"] == pytest.approx(1.0)
    assert rep["tokens_identical"] and rep["rounds"] == 4


def test_round_order_runs_every_pair_both_ways():
    systems = list(harness.SWEEP_SYSTEMS)
    for x in systems:
        for y in systems:
            if x != y:
                before = [o.index(x) < o.index(y) for o in (harness.round_order(systems, r) for r in range(12))]
                assert sum(before) == 6
    assert {harness.round_order(systems, r)[0] for r in range(0, 12, 2)} == set(systems)


def test_fresh_placement_takes_no_pad_off_the_gpu():
    import random

    assert harness.fresh_placement(random.Random(0), "cpu") is None


@pytest.mark.gpu
def test_context_sweep_and_attention_micro_on_the_gpu():
    """The sweep and the micro on a small model with every system: each round
    places the caches afresh (a pad is taken), graph systems capture again,
    and the report has a median for every (system, context) and the
    paging-cost intervals at every context."""
    cfg = dict(max_seq_length=64, vocab_size=512, num_layers=2, hidden_dim=64, num_heads=4, num_experts=4, top_k=2)
    model = harness.make_model(cfg, device="cuda")
    rep = harness.context_sweep(model, contexts=(16, 40, 64), rounds=3, steps=4, filler=7)
    assert rep["placement_sampled"] and rep["rounds"] == 3
    for system in harness.SWEEP_SYSTEMS:
        assert set(rep["median_step_ms"][system]) == {16, 40, 64}
        assert all(v > 0 for v in rep["median_step_ms"][system].values())
    for ctx in (16, 40, 64):
        cost = rep["paging_cost_ms"][ctx]
        assert set(cost) == {"paged-direct_minus_contiguous-direct",
                             "paged-direct-graph_minus_contiguous-direct-graph"}
        assert all(c["ci95_ms"][0] <= c["mean_delta_ms"] <= c["ci95_ms"][1] for c in cost.values())
    micro = harness.attention_micro(cfg, contexts=(16, 64), rounds=2, iters=10)
    for ctx in (16, 64):
        row = micro[ctx]
        assert set(harness.MICRO_VARIANTS) <= set(row)
        assert row["paged_direct_device_us"] > 0 and row["contiguous_direct_device_us"] > 0
        assert "paging_cost_device_us" in row and "paging_cost_host_launched_us" in row


@pytest.mark.gpu
def test_graph_ab_round_captures_again_and_matches_eager_tokens():
    """ab_compare with placement: every round allocates fresh caches and each
    graph system captures its step again; the graphed, eager, paged and
    contiguous-layout systems all choose the same greedy tokens."""
    cfg = dict(max_seq_length=96, vocab_size=512, num_layers=2, hidden_dim=64, num_heads=4, num_experts=4, top_k=2)
    model = harness.make_model(cfg, device="cuda")
    prompt = torch.randint(0, cfg["vocab_size"], (7,), generator=torch.Generator().manual_seed(5)).cuda()
    systems = ("paged-direct", harness.CONTIGUOUS_DIRECT, harness.GRAPH_SYSTEM, harness.CONTIGUOUS_DIRECT_GRAPH)
    rep = harness.ab_compare(model, prompt, systems, rounds=3, new_tokens=20)
    assert rep["tokens_identical"] and rep["placement_sampled"]
    assert len(rep["tokens"]) == 21
    for a, b in harness.PAGING_COST_PAIRS:
        assert len(rep["paired_deltas"][f"{a}_minus_{b}"]["per_round_delta_ms"]) == 3
    want = model.generate(prompt, 21, temperature=0)[0, len(prompt):].tolist()
    assert rep["tokens"] == want
