"""Fused MoE decode (moe_engine.fused_moe -> mie_moe_route / mie_moe_decode)
against the reference's PyTorch MoE path.

Mirrors the reference's tests/test_fused_moe.py:52-236, and checks the
block form (x + MoE(LayerNorm(x)), mie_moe_decode_block) against the
reference block's own sequence.  The PyTorch path
(model.py:443-461) is the oracle: same module, same input, mode 'reference'
vs 'direct'.  Expert ids must match torch.topk exactly; route weights match
softmax to 2e-6 (reference :66-69); outputs agree to float32 GEMV-vs-GEMM
rounding, checked at 1e-5 of the output scale (the reference allows 3e-4 /
2e-4 for its Triton kernel, :107, :117, :134).  End-to-end token identity with
the reference engine runs through tests/test_gpu_golden.py, where 'auto'
selects these kernels for decode steps.
"""

import os

import pytest
import torch
import torch.nn.functional as F

from conftest import print_case
from moe_engine import fused_moe
from moe_engine.model import Model, ModelConfig, MoEFeedForward

pytestmark = pytest.mark.gpu

TINY = dict(max_seq_length=32, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)


def moe(dim, hidden, experts, top_k, seed=0, mode="direct"):
    torch.manual_seed(seed)
    return MoEFeedForward(dim, hidden, experts, top_k, mode=mode).to("cuda").eval()


def assert_output_close(got, want):
    scale = max(want.abs().max().item(), 1.0)
    err = (got - want).abs().max().item()
    assert err <= 1e-5 * scale, f"max error {err:.3e} at output scale {scale:.3e}"


def route_with_workspace(layer, x):
    fused_moe.route(x, layer.router.weight, layer._router_logits, layer._expert_ids, layer._route_weights)
    return layer._router_logits.clone(), layer._expert_ids.clone(), layer._route_weights.clone()


@pytest.mark.parametrize(
    "dim,hidden,experts,top_k",
    [(768, 2048, 8, 2), (768, 3072, 8, 2), (32, 128, 4, 2), (64, 256, 16, 4), (128, 64, 3, 1), (96, 192, 64, 8)],
)
def test_fused_decode_matches_pytorch_path(dim, hidden, experts, top_k):
    print_case("moe", dim, hidden, experts, top_k)
    layer = moe(dim, hidden, experts, top_k)
    gen = torch.Generator(device="cuda").manual_seed(1)
    for _ in range(8):
        x = torch.randn(1, 1, dim, generator=gen, device="cuda")
        with torch.no_grad():
            want = layer._forward_reference(x)
            got = layer(x, decode=True).clone()
        assert_output_close(got, want)


@pytest.mark.parametrize("seed", range(int(os.environ.get("MIE_MOE_RANDOM_CASES", "16"))))
def test_random_fused_decode_and_block_match_pytorch_path(seed):
    """Drawn widths (multiples of 4 up to 2048), hidden sizes, expert counts
    (up to 64) and top-k (up to 8): the fused decode and the block form
    against the module's PyTorch path, as in the fixed cases."""
    import random

    rng = random.Random(seed)
    dim = rng.choice((4, 16, 36, 64, 100, 256, 768, 2048))
    hidden = rng.choice((4, 12, 64, 200, 1024, 2048))
    experts = rng.choice((1, 2, 3, 8, 17, 64))
    top_k = rng.randint(1, min(8, experts))
    print_case("random moe", seed, dim, hidden, experts, top_k)
    layer = moe(dim, hidden, experts, top_k, seed=seed)
    if not layer.direct_configuration_supported(1):
        pytest.skip(f"dim {dim} hidden {hidden} experts {experts} top_k {top_k} is not built")
    norm = torch.nn.LayerNorm(dim).to("cuda")
    with torch.no_grad():
        norm.weight.uniform_(0.5, 1.5)
        norm.bias.uniform_(-0.1, 0.1)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for _ in range(3):
        x = torch.randn(1, 1, dim, generator=gen, device="cuda")
        with torch.no_grad():
            assert_output_close(layer(x, decode=True).clone(), layer._forward_reference(x))
            want = x + layer._forward_reference(norm(x))
            got = layer.fused_block_decode(x, norm)
            assert got is not None
            assert_output_close(got.clone(), want)


@pytest.mark.parametrize("experts,top_k", [(8, 2), (16, 4), (64, 8)])
def test_router_logits_topk_ids_and_normalized_weights_match_pytorch(experts, top_k):
    layer = moe(768, 256, experts, top_k)
    x = torch.randn(1, 1, 768, device="cuda")
    logits, ids, weights = route_with_workspace(layer, x)
    want_logits = F.linear(x.reshape(1, 768), layer.router.weight).squeeze(0)
    want_top, want_ids = torch.topk(want_logits, top_k)
    torch.testing.assert_close(logits, want_logits, atol=2e-5, rtol=1e-5)
    assert torch.equal(ids.long(), want_ids)
    torch.testing.assert_close(weights, F.softmax(want_top, dim=0), atol=2e-6, rtol=1e-6)
    torch.testing.assert_close(weights.sum(), torch.ones((), device="cuda"))


def test_top_k_ties_take_the_lower_expert_id():
    layer = moe(64, 64, 8, 3)
    x = torch.ones(1, 1, 64, device="cuda")
    with torch.no_grad():
        layer.router.weight.copy_(torch.tensor([1, 3, 2, 3, 0, 2, 3, 1], device="cuda")[:, None].expand(8, 64) / 64)
    _, ids, weights = route_with_workspace(layer, x)
    assert ids.tolist() == [1, 3, 6]
    torch.testing.assert_close(weights, torch.full((3,), 1 / 3, device="cuda"))


def test_every_expert_is_addressed_in_both_routes():
    """Distinct weights and biases per expert, each expert first and second in
    turn (reference tests/test_fused_moe.py:73-110)."""
    layer = moe(768, 3072, 8, 2)
    x = torch.ones(1, 1, 768, device="cuda")
    firsts, seconds = [], []
    with torch.no_grad():
        for e, expert in enumerate(layer.experts):
            expert.net[0].weight.zero_()
            expert.net[0].weight[0, 0] = 0.2 * (e + 1)
            expert.net[0].bias.copy_(torch.linspace(-0.3, 0.3, 3072, device="cuda") + 0.05 * e)
            expert.net[2].weight.zero_()
            expert.net[2].weight[:, 0].copy_(torch.linspace(0.01, 0.02, 768, device="cuda") * (e + 1))
            expert.net[2].bias.copy_(torch.linspace(-0.2, 0.2, 768, device="cuda") + 0.1 * e)
        for first in range(8):
            second = (first + 3) % 8
            logits = -2.0 - 0.1 * torch.arange(8, device="cuda")
            logits[first] = 1.0
            logits[second] = 0.25
            layer.router.weight.copy_(logits[:, None].expand(8, 768) / 768)
            _, ids, _ = route_with_workspace(layer, x)
            firsts.append(int(ids[0]))
            seconds.append(int(ids[1]))
            assert_output_close(layer(x, decode=True).clone(), layer._forward_reference(x))
    assert firsts == list(range(8))
    assert seconds == [(e + 3) % 8 for e in range(8)]


def test_both_expert_biases_and_exact_gelu_semantics_match_oracle():
    layer = moe(768, 3072, 8, 2)
    x = torch.linspace(-1.5, 1.5, 768, device="cuda").view(1, 1, 768)
    with torch.no_grad():
        for e, expert in enumerate(layer.experts):
            expert.net[0].bias.copy_(torch.linspace(-2.0, 2.0, 3072, device="cuda") + e * 0.01)
            expert.net[2].bias.fill_((e + 1) * 0.025)
        assert_output_close(layer(x, decode=True).clone(), layer._forward_reference(x))
        # Exact (erf) GELU on the selected rows, against torch's.
        ids = layer._expert_ids.tolist()
        flat = x.reshape(768)
        for slot, e in enumerate(ids):
            pre = layer.experts[e].net[0](flat)
            torch.testing.assert_close(layer._expert_hidden[slot], F.gelu(pre), atol=1e-5, rtol=1e-5)


def test_decode_returns_the_layer_output_buffer():
    layer = moe(64, 128, 4, 2)
    x = torch.randn(1, 1, 64, device="cuda")
    with torch.no_grad():
        out = layer(x, decode=True)
    assert out.shape == (1, 1, 64)
    assert out.data_ptr() == layer._direct_out.data_ptr()


def test_decode_rejects_non_canonical_weights():
    layer = moe(64, 128, 4, 2)
    s = layer._expert_storage
    x = torch.randn(1, 1, 64, device="cuda")
    with pytest.raises(ValueError, match="canonical"):
        fused_moe.decode(x, layer.router.weight, s["w1"].transpose(1, 2), s["b1"], s["w2"], s["b2"],
                         router_logits=layer._router_logits, expert_ids=layer._expert_ids,
                         route_weights=layer._route_weights, hidden=layer._expert_hidden, out=layer._direct_out)
    with pytest.raises(RuntimeError, match="float32"):
        fused_moe.decode(x.double(), layer.router.weight, s["w1"], s["b1"], s["w2"], s["b2"],
                         router_logits=layer._router_logits, expert_ids=layer._expert_ids,
                         route_weights=layer._route_weights, hidden=layer._expert_hidden, out=layer._direct_out)


def test_auto_falls_back_on_float64_and_forced_direct_fails():
    layer = moe(768, 3072, 8, 2, mode="auto").double()
    x = torch.randn(1, 1, 768, device="cuda", dtype=torch.float64)
    with torch.no_grad():
        torch.testing.assert_close(layer(x, decode=True), layer._forward_reference(x), atol=0, rtol=0)
    layer.set_mode("direct")
    with pytest.raises(RuntimeError, match="float32"):
        layer(x, decode=True)


def test_canonical_storage_survives_device_apply():
    from test_engine_cpu import assert_canonical_storage

    layer = MoEFeedForward(32, 128, 4, 2).to("cuda")
    assert_canonical_storage(layer, device_type="cuda", dtype=torch.float32)
    layer.cpu()
    assert_canonical_storage(layer, device_type="cpu", dtype=torch.float32)


def test_forced_direct_preflight_preserves_paged_cache_at_block_boundary():
    # The reference's case (tests/test_fused_moe.py:167-197) makes the direct
    # MoE unavailable through bfloat16, which its kernels lack; these kernels
    # take bfloat16, so float64 plays that part here.
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").double().eval()
    allocator = model.new_block_allocator(num_blocks=4, block_size=4)
    cache = allocator.new_cache()
    ids = torch.randint(0, 96, (1, 4), device="cuda")
    with torch.no_grad():
        model(ids, cache)
    assert cache.position == 4 and len(cache.block_table) == 1
    before = (cache.position, list(cache.block_table), sorted(allocator.free_blocks), cache._write_index_key)
    mirror = cache.block_table_device[:2].clone()
    k_before, v_before = allocator.k_pool.clone(), allocator.v_pool.clone()
    model.set_moe_mode("direct")
    with torch.no_grad(), pytest.raises(RuntimeError, match="direct"):
        model(ids[:, :1], cache)
    assert (cache.position, cache.block_table, sorted(allocator.free_blocks), cache._write_index_key) == before
    assert torch.equal(cache.block_table_device[:2], mirror)
    assert torch.equal(allocator.k_pool, k_before)
    assert torch.equal(allocator.v_pool, v_before)


def test_forced_direct_preflight_preserves_contiguous_cache():
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").double().eval()
    cache = model.new_cache()
    ids = torch.randint(0, 96, (1, 4), device="cuda")
    with torch.no_grad():
        model(ids, cache)
    position, k_before, v_before = cache.position, cache.k.clone(), cache.v.clone()
    model.set_moe_mode("direct")
    with torch.no_grad(), pytest.raises(RuntimeError, match="direct"):
        model(ids[:, :1], cache)
    assert cache.position == position
    assert torch.equal(cache.k, k_before)
    assert torch.equal(cache.v, v_before)


def test_auto_uses_fused_kernel_for_decode_and_pytorch_for_prefill():
    layer = moe(64, 128, 4, 2, mode="auto")
    x1 = torch.randn(1, 1, 64, device="cuda")
    x4 = torch.randn(1, 4, 64, device="cuda")
    assert layer.uses_direct(x1, decode=True)
    assert not layer.uses_direct(x4, decode=False)
    assert not layer.uses_direct(x1.double(), decode=True)
    layer.set_mode("reference")
    assert not layer.uses_direct(x1, decode=True)


@pytest.mark.parametrize("dim,hidden,experts,top_k", [(768, 2048, 8, 2), (64, 256, 16, 4), (128, 64, 3, 1)])
@pytest.mark.parametrize("norm", [True, False])
def test_block_decode_matches_norm_then_pytorch_path(dim, hidden, experts, top_k, norm):
    """decode_block: out = x + MoE(LayerNorm(x)) against the reference block's
    own sequence (model.py:494-498) with the PyTorch MoE path; routing outputs
    against torch.topk / softmax of the normalised token's router logits."""
    print_case("moe block", dim, hidden, experts, top_k, norm)
    layer = moe(dim, hidden, experts, top_k)
    ln = torch.nn.LayerNorm(dim).to("cuda")
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(dim, device="cuda"))
        ln.bias.copy_(0.1 * torch.randn(dim, device="cuda"))
    gen = torch.Generator(device="cuda").manual_seed(2)
    for _ in range(4):
        x = torch.randn(1, 1, dim, generator=gen, device="cuda") * 3 + 0.5
        with torch.no_grad():
            normed = ln(x) if norm else x
            want = x + layer._forward_reference(normed)
            s = layer._expert_storage
            got = fused_moe.decode_block(
                x, ln.weight if norm else None, ln.bias if norm else None, ln.eps, layer.router.weight,
                s["w1"], s["b1"], s["w2"], s["b2"], router_logits=layer._router_logits,
                expert_ids=layer._expert_ids, route_weights=layer._route_weights, hidden=layer._expert_hidden,
                out=layer._direct_out,
            ).clone()
            logits = F.linear(normed.reshape(1, -1), layer.router.weight)[0]
        assert_output_close(got, want)
        top = torch.topk(logits, top_k)
        assert torch.equal(layer._expert_ids.long(), top.indices)
        torch.testing.assert_close(layer._route_weights, F.softmax(top.values, dim=0), atol=2e-6, rtol=1e-6)
        torch.testing.assert_close(layer._router_logits, logits, atol=2e-5, rtol=1e-5)


def test_block_decode_output_may_alias_input():
    layer = moe(64, 128, 4, 2)
    x = torch.randn(1, 1, 64, device="cuda")
    s = layer._expert_storage
    with torch.no_grad():
        want = x + layer._forward_reference(x)
        fused_moe.decode_block(x, None, None, 1e-5, layer.router.weight, s["w1"], s["b1"], s["w2"], s["b2"],
                               router_logits=layer._router_logits, expert_ids=layer._expert_ids,
                               route_weights=layer._route_weights, hidden=layer._expert_hidden, out=x.view(64))
    assert_output_close(x, want)


def test_model_block_fusion_matches_reference_block():
    """The model's decode steps with the fused MoE half (mode auto) against
    mode 'reference' (the PyTorch path after the block's norm), float32."""
    torch.manual_seed(0)
    model = Model(ModelConfig(max_seq_length=128, vocab_size=512, num_layers=2, hidden_dim=128, num_heads=4,
                              num_experts=8, top_k=2)).to("cuda").eval()
    ids = torch.randint(0, 512, (1, 24), device="cuda")
    logits = {}
    for mode in ("reference", "auto"):
        model.set_moe_mode(mode)
        cache = model.new_block_allocator(num_blocks=16, block_size=16, attention_mode="direct").new_cache()
        with torch.no_grad():
            steps = [model(ids[:, :16], cache)[:, -1]]
            steps += [model(ids[:, t : t + 1], cache)[:, -1] for t in range(16, 24)]
        logits[mode] = torch.stack(steps, 1)
    torch.testing.assert_close(logits["auto"], logits["reference"], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dim,hidden,experts,top_k,tokens", [(768, 2048, 8, 2, 32), (768, 3072, 8, 2, 7),
                                                             (64, 256, 16, 4, 512), (128, 64, 3, 1, 1)])
def test_dense_prefill_matches_pytorch_path(dim, hidden, experts, top_k, tokens):
    """_forward_dense (every expert on every token, summed in id order with the
    unselected weights zero) against the reference path on the same layer:
    the same routing, outputs equal to float32 GEMM rounding."""
    print_case("dense prefill", dim, hidden, experts, top_k, tokens)
    layer = moe(dim, hidden, experts, top_k, mode="auto")
    x = torch.randn(1, tokens, dim, device="cuda")
    with torch.no_grad():
        assert layer.uses_dense_prefill(x, decode=False)
        got = layer(x)
        want = layer._forward_reference(x)
    assert_output_close(got, want)


def test_dense_prefill_applies_only_where_it_should():
    layer = moe(64, 128, 4, 2, mode="auto")
    x = torch.randn(1, 8, 64, device="cuda")
    assert layer.uses_dense_prefill(x, decode=False)
    assert not layer.uses_dense_prefill(x.double(), decode=False)
    assert not layer.uses_dense_prefill(torch.randn(1, 513, 64, device="cuda"), decode=False)
    assert not layer.uses_dense_prefill(x.cpu(), decode=False)
    layer.set_mode("reference")
    assert not layer.uses_dense_prefill(x, decode=False)


def test_model_prefill_with_dense_moe_matches_reference_mode():
    """A 40-token prefill through the whole model (float32), mode auto (dense
    MoE prefill) vs mode reference: logits within 1e-4."""
    torch.manual_seed(0)
    model = Model(ModelConfig(max_seq_length=128, vocab_size=512, num_layers=2, hidden_dim=128, num_heads=4,
                              num_experts=8, top_k=2)).to("cuda").eval()
    ids = torch.randint(0, 512, (1, 40), device="cuda")
    logits = {}
    for mode in ("reference", "auto"):
        model.set_moe_mode(mode)
        with torch.no_grad():
            logits[mode] = model(ids, model.new_cache())
    torch.testing.assert_close(logits["auto"], logits["reference"], atol=1e-4, rtol=1e-4)
