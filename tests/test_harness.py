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
