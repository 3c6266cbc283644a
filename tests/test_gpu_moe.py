"""Fused MoE decode (mie_moe_decode) against the reference's PyTorch MoE path.

The PyTorch path (model.py:443-461) is the oracle: same module, same input,
mode 'reference' vs 'direct'.  Outputs agree to float32 GEMV-vs-GEMM rounding
(checked relative to the output scale); the selected experts and routing
weights are checked exactly against torch.topk / softmax on the router logits.
End-to-end token identity with the reference engine runs through
tests/test_gpu_golden.py, where 'auto' selects this kernel for decode steps.
"""

import pytest
import torch
import torch.nn.functional as F

from conftest import print_case
from moe_engine import _native
from moe_engine.model import Model, ModelConfig, MoEFeedForward

pytestmark = pytest.mark.gpu


def moe(dim, hidden, experts, top_k, seed=0):
    torch.manual_seed(seed)
    return MoEFeedForward(dim, hidden, experts, top_k).to("cuda").eval()


@pytest.mark.parametrize(
    "dim,hidden,experts,top_k",
    [(768, 2048, 8, 2), (768, 3072, 8, 2), (32, 128, 4, 2), (64, 256, 16, 4), (128, 64, 3, 1)],
)
def test_fused_decode_matches_pytorch_path(dim, hidden, experts, top_k):
    print_case("moe", dim, hidden, experts, top_k)
    layer = moe(dim, hidden, experts, top_k)
    gen = torch.Generator(device="cuda").manual_seed(1)
    for _ in range(8):
        x = torch.randn(1, 1, dim, generator=gen, device="cuda")
        with torch.no_grad():
            layer.set_mode("reference")
            want = layer(x, decode=True)
            layer.set_mode("direct")
            got = layer(x, decode=True)
        scale = want.abs().max().item()
        assert (got - want).abs().max().item() <= 1e-5 * max(scale, 1.0)


def test_routing_ids_and_weights_are_exact():
    layer = moe(768, 2048, 8, 2)
    x = torch.randn(1, 1, 768, device="cuda")
    with torch.no_grad():
        layer.set_mode("direct")
        layer(x, decode=True)
        torch.cuda.synchronize()
        logits = F.linear(x.reshape(1, -1), layer.router.weight)[0]
    ws = layer._direct_workspace
    ids = ws[:8].view(torch.int32)[:2].tolist()
    weights = ws[128:136].view(torch.float32)[:2]
    top = torch.topk(logits, 2)
    order = sorted(range(2), key=lambda i: int(top.indices[i]))
    assert ids == sorted(top.indices.tolist())
    want = F.softmax(top.values, dim=-1)[order]
    torch.testing.assert_close(weights, want, atol=1e-6, rtol=1e-6)


def test_workspace_size_matches_library():
    layer = moe(768, 2048, 8, 2)
    assert layer._direct_workspace.numel() == _native.lib().mie_moe_decode_workspace_bytes(2, 2048)


def test_forced_direct_rejects_unsupported_dtype_before_cache_mutation():
    torch.manual_seed(0)
    model = Model(ModelConfig(max_seq_length=32, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4,
                              top_k=2)).to("cuda").bfloat16().eval()
    allocator = model.new_block_allocator(num_blocks=4, block_size=4)
    cache = allocator.new_cache()
    ids = torch.randint(0, 96, (1, 4), device="cuda")
    with torch.no_grad():
        model(ids, cache)
    before = (cache.position, list(cache.block_table), sorted(allocator.free_blocks), allocator.k_pool.clone())
    model.set_moe_mode("direct")
    with torch.no_grad(), pytest.raises(RuntimeError, match="direct"):
        model(ids[:, :1], cache)
    assert (cache.position, cache.block_table, sorted(allocator.free_blocks)) == before[:3]
    assert torch.equal(allocator.k_pool, before[3])


def test_auto_uses_fused_kernel_for_decode_and_pytorch_for_prefill():
    layer = moe(64, 128, 4, 2)
    x1 = torch.randn(1, 1, 64, device="cuda")
    x4 = torch.randn(1, 4, 64, device="cuda")
    assert layer.uses_direct(x1, decode=True)
    assert not layer.uses_direct(x4, decode=False)
    assert not layer.uses_direct(x1.double(), decode=True)
    layer.set_mode("reference")
    assert not layer.uses_direct(x1, decode=True)
