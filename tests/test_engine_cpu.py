"""Host-side engine semantics on the CPU (no GPU needed).

Mirrors the reference's CPU-runnable tests of the paged path
(tests/test_parity.py, tests/test_paged_attention.py:188-282,
tests/test_fused_moe.py:167-197): allocator reclaim and rollback, batch
rejection, dtype following, generate() validation, the prefill fast path,
fail-before-mutate for a forced 'direct' that cannot run, and the device
mirror of the block table.  The product's CPU paged cache is also compared
with the oracle's closed forms.
"""

import random

import numpy as np
import pytest
import torch

from moe_engine import paged_attention
from moe_engine.model import BlockAllocator, KVCache, Model, ModelConfig, MoEFeedForward, PagedKVCache
from oracle import paged_ref as ref

TINY = dict(max_seq_length=32, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)
TINY128 = dict(TINY, max_seq_length=128)


def make_engine(**overrides):
    torch.manual_seed(0)
    return Model(ModelConfig(**dict(TINY, **overrides))).eval()


def stepwise(engine, ids, cache, prefill):
    with torch.no_grad():
        steps = [engine(ids[:, :prefill], cache)[:, -1]]
        for t in range(prefill, ids.shape[1]):
            steps.append(engine(ids[:, t : t + 1], cache)[:, -1])
    return torch.stack(steps, dim=1)


def test_cached_decode_matches_full_forward():
    engine = make_engine()
    ids = torch.randint(0, TINY["vocab_size"], (1, 16))
    with torch.no_grad():
        full = engine(ids, engine.new_cache())
    torch.testing.assert_close(stepwise(engine, ids, engine.new_cache(), 4), full[:, 3:], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("mode", ["gather", "auto"])
def test_paged_decode_matches_full_forward(mode):
    engine = make_engine()
    ids = torch.randint(0, TINY["vocab_size"], (1, 16))
    with torch.no_grad():
        full = engine(ids, engine.new_cache())
    cache = engine.new_block_allocator(num_blocks=8, block_size=4, attention_mode=mode).new_cache()
    torch.testing.assert_close(stepwise(engine, ids, cache, 4), full[:, 3:], atol=1e-4, rtol=1e-4)


def test_paged_cache_shares_pool_without_leaking():
    engine = make_engine()
    ids_a = torch.randint(0, TINY["vocab_size"], (1, 16))
    ids_b = torch.randint(0, TINY["vocab_size"], (1, 16))
    allocator = engine.new_block_allocator(num_blocks=8, block_size=4)
    cache_a, cache_b = allocator.new_cache(), allocator.new_cache()
    with torch.no_grad():
        full_a = engine(ids_a, engine.new_cache())
        full_b = engine(ids_b, engine.new_cache())
        engine(ids_a[:, :4], cache_a)
        engine(ids_b[:, :4], cache_b)
        for t in range(4, 16):  # interleaved, so the two tables alternate in the pool
            logits_a = engine(ids_a[:, t : t + 1], cache_a)
            logits_b = engine(ids_b[:, t : t + 1], cache_b)
    assert not set(cache_a.block_table) & set(cache_b.block_table)
    torch.testing.assert_close(logits_a[:, -1], full_a[:, -1], atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(logits_b[:, -1], full_b[:, -1], atol=1e-4, rtol=1e-4)


def test_block_allocator_reclaims_freed_blocks():
    engine = make_engine()
    ids = torch.randint(0, TINY["vocab_size"], (1, 8))
    allocator = engine.new_block_allocator(num_blocks=2, block_size=4)
    cache_a, cache_b = allocator.new_cache(), allocator.new_cache()
    with torch.no_grad():
        engine(ids, cache_a)
        with pytest.raises(RuntimeError, match="no free KV cache blocks left"):
            engine(ids[:, :1], cache_b)
        cache_a.free()
        engine(ids[:, :1], cache_b)


def test_failed_allocation_rolls_back():
    engine = make_engine()
    allocator = engine.new_block_allocator(num_blocks=1, block_size=4)
    cache = allocator.new_cache()
    ids = torch.randint(0, TINY["vocab_size"], (1, 8))  # needs two blocks
    with torch.no_grad():
        with pytest.raises(RuntimeError, match="no free KV cache blocks left"):
            engine(ids, cache)
        assert cache.block_table == [] and cache.position == 0 and allocator.free_blocks == [0]
        engine(ids[:, :4], cache)  # still usable


def test_allocation_order_matches_oracle_lifo():
    engine = make_engine()
    allocator = engine.new_block_allocator(num_blocks=9, block_size=4)
    random.Random(5).shuffle(allocator.free_blocks)
    oracle_alloc = ref.LifoAllocator(9)
    oracle_alloc.free_blocks = list(allocator.free_blocks)
    cache = allocator.new_cache()
    table = []
    with torch.no_grad():
        engine(torch.randint(0, 96, (1, 7)), cache)
        ref.reserve(table, oracle_alloc, 7, 4)
        for n in range(8, 20):
            engine(torch.randint(0, 96, (1, 1)), cache)
            ref.reserve(table, oracle_alloc, n, 4)
    assert cache.block_table == table
    assert allocator.free_blocks == oracle_alloc.free_blocks
    assert cache.block_table_device[: len(table)].tolist() == table


def test_paged_cache_rejects_batches():
    engine = make_engine()
    allocator = engine.new_block_allocator(num_blocks=8, block_size=4)
    with torch.no_grad(), pytest.raises(ValueError, match="batch size 1"):
        engine(torch.randint(0, 96, (2, 4)), allocator.new_cache())


def test_generate_stops_at_context_limit():
    engine = make_engine()
    prompt = torch.randint(0, TINY["vocab_size"], (TINY["max_seq_length"] - 2,))
    out = engine.generate(prompt, max_new_tokens=10, temperature=0)
    assert out.shape[1] == TINY["max_seq_length"] + 1  # the last token never enters the cache


def test_generate_validates_prompt_and_cache():
    engine = make_engine()
    with pytest.raises(ValueError, match="max_seq_length"):
        engine.generate(torch.randint(0, 96, (TINY["max_seq_length"] + 1,)), max_new_tokens=1)
    allocator = engine.new_block_allocator(num_blocks=8, block_size=4)
    used = allocator.new_cache()
    prompt = torch.randint(0, 96, (1, 4))
    with torch.no_grad():
        engine(prompt, used)
    before = list(used.block_table)
    with pytest.raises(ValueError, match="fresh cache"):
        engine.generate(prompt, max_new_tokens=1, cache=used)
    assert used.block_table == before


def test_generate_validates_arguments():
    engine = make_engine()
    prompt = torch.randint(0, 96, (4,))
    for kwargs in (dict(temperature=-1), dict(temperature=float("nan")), dict(top_k=0), dict(max_new_tokens=0)):
        args = {"max_new_tokens": 4, **kwargs}
        with pytest.raises(ValueError):
            engine.generate(prompt, **args)


def test_cache_follows_model_dtype():
    """The contiguous cache (the comparator) takes the model's dtype too.
    Routing stays in float32 for every model dtype (model.py:448-452), and a
    one-row router product can differ from the batched one in its last float32
    bits, so float64 logits agree to float32 rounding, not float64's."""
    engine = make_engine().double()
    ids = torch.randint(0, 96, (1, 8))
    with torch.no_grad():
        full = engine(ids, engine.new_cache())
        cache = engine.new_cache()
        engine(ids[:, :4], cache)
        step = engine(ids[:, 4:5], cache)
    assert full.dtype == torch.float64 and step.dtype == torch.float64
    assert cache.k.dtype == torch.float64
    torch.testing.assert_close(step[:, -1], full[:, 4], atol=1e-5, rtol=1e-5)


def test_paged_cache_follows_model_dtype():
    engine = make_engine().double()
    ids = torch.randint(0, 96, (1, 8))
    with torch.no_grad():
        full = engine(ids, engine.new_cache())
        cache = engine.new_block_allocator(num_blocks=2, block_size=4).new_cache()
        engine(ids[:, :4], cache)
        step = engine(ids[:, 4:5], cache)
    assert step.dtype == torch.float64 and cache.allocator.k_pool.dtype == torch.float64
    torch.testing.assert_close(step[:, -1], full[:, 4], atol=1e-4, rtol=1e-4)


def test_auto_mode_matches_gather_mode_on_cpu():
    engine = make_engine(max_seq_length=128)
    ids = torch.randint(0, 96, (1, 16))
    logits = {}
    for mode in ("gather", "auto"):
        cache = engine.new_block_allocator(num_blocks=16, block_size=4, attention_mode=mode).new_cache()
        logits[mode] = stepwise(engine, ids, cache, 8)
    torch.testing.assert_close(logits["auto"], logits["gather"], atol=1e-5, rtol=1e-5)


def test_prefill_fast_path_matches_contiguous():
    engine = make_engine(max_seq_length=128)
    ids = torch.randint(0, 96, (1, 19))  # partial last block
    with torch.no_grad():
        contiguous = engine(ids, engine.new_cache())
        paged = engine(ids, engine.new_block_allocator(num_blocks=16, block_size=4).new_cache())
    torch.testing.assert_close(paged, contiguous, atol=1e-5, rtol=1e-5)


def assert_cache_untouched(cache, allocator, num_blocks):
    assert cache.position == 0
    assert cache.block_table == []
    assert sorted(allocator.free_blocks) == list(range(num_blocks))
    assert (cache.block_table_device == 0).all()
    assert cache._write_index_key is None


def test_direct_mode_raises_without_rocm_before_mutating():
    engine = make_engine()
    allocator = engine.new_block_allocator(num_blocks=8, block_size=4, attention_mode="direct")
    cache = allocator.new_cache()
    with torch.no_grad(), pytest.raises(RuntimeError, match="direct"):
        engine(torch.randint(0, 96, (1, 5)), cache)
    assert_cache_untouched(cache, allocator, 8)


def test_invalid_attention_mode_rejected():
    with pytest.raises(ValueError, match="attention_mode"):
        make_engine().new_block_allocator(num_blocks=4, block_size=4, attention_mode="turbo")


def test_device_block_table_mirrors_python_table():
    engine = make_engine()
    allocator = engine.new_block_allocator(num_blocks=16, block_size=4)
    random.Random(1).shuffle(allocator.free_blocks)
    cache = allocator.new_cache()
    ids = torch.randint(0, 96, (1, 10))
    with torch.no_grad():
        engine(ids, cache)  # 10 tokens -> 3 blocks
        for t in range(3):  # crosses into a 4th block
            engine(ids[:, t : t + 1], cache)
    assert len(cache.block_table) == 4
    assert cache.block_table_device[:4].tolist() == cache.block_table


def test_forced_direct_moe_preflight_preserves_paged_cache_at_block_boundary():
    engine = make_engine()
    allocator = engine.new_block_allocator(num_blocks=4, block_size=4)
    cache = allocator.new_cache()
    ids = torch.randint(0, 96, (1, 4))
    with torch.no_grad():
        engine(ids, cache)
    snapshot = (
        cache.position,
        list(cache.block_table),
        sorted(allocator.free_blocks),
        cache._write_index_key,
        cache.block_table_device.clone(),
        allocator.k_pool.clone(),
        allocator.v_pool.clone(),
    )
    engine.set_moe_mode("direct")
    with torch.no_grad(), pytest.raises(RuntimeError, match="direct"):
        engine(ids[:, :1], cache)  # the next token would open a new block
    assert cache.position == snapshot[0] and cache.block_table == snapshot[1]
    assert sorted(allocator.free_blocks) == snapshot[2] and cache._write_index_key == snapshot[3]
    for now, then in zip((cache.block_table_device, allocator.k_pool, allocator.v_pool), snapshot[4:]):
        assert torch.equal(now, then)


@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_cpu_paged_cache_matches_oracle_closed_forms(block_size):
    """The product's CPU write/read against the oracle's append_rows/gather_rows."""
    cfg = ModelConfig(**TINY128)
    allocator = BlockAllocator(cfg, num_blocks=40, block_size=block_size, device="cpu")
    random.Random(block_size).shuffle(allocator.free_blocks)
    cache = PagedKVCache(allocator)
    g = torch.Generator().manual_seed(block_size)
    H, D, ctx = cfg.num_heads, cfg.head_dim, 2 * block_size + 5
    k = torch.randn(1, H, ctx, D, generator=g)
    v = torch.randn(1, H, ctx, D, generator=g)
    ok, ov = allocator.k_pool.numpy().copy(), allocator.v_pool.numpy().copy()
    cache.write(1, 0, k[:, :, : ctx - 2], v[:, :, : ctx - 2])
    cache.write(1, ctx - 2, k[:, :, ctx - 2 : ctx - 1], v[:, :, ctx - 2 : ctx - 1])
    cache.write(1, ctx - 1, k[:, :, ctx - 1 :], v[:, :, ctx - 1 :])
    ref.append_rows(ok, ov, 1, cache.block_table, 0, k[0].numpy(), v[0].numpy())
    assert np.array_equal(allocator.k_pool.numpy(), ok) and np.array_equal(allocator.v_pool.numpy(), ov)
    rk, rv = cache.read(1, ctx)
    assert np.array_equal(rk[0].numpy(), ref.gather_rows(ok, 1, cache.block_table, ctx))
    assert np.array_equal(rv[0].numpy(), ref.gather_rows(ov, 1, cache.block_table, ctx))


def test_is_supported_is_false_off_device():
    x = torch.zeros(1, 1, 32)
    assert not paged_attention.is_supported(x)
    assert not paged_attention.is_supported(x.double(), head_dim=64)


def test_contiguous_kvcache_is_a_view():
    cfg = ModelConfig(**TINY)
    cache = KVCache(cfg, 1, "cpu")
    k = torch.randn(1, cfg.num_heads, 3, cfg.head_dim)
    cache.write(0, 2, k, -k)
    rk, rv = cache.read(0, 5)
    assert torch.equal(rk[:, :, 2:], k) and torch.equal(rv[:, :, 2:], -k)
    assert rk.data_ptr() == cache.k.data_ptr()


def assert_canonical_storage(moe, *, device_type, dtype):
    """Each expert parameter group is one contiguous storage whose slices are
    the experts' parameters (reference tests/test_fused_moe.py:239-259)."""
    for key, layer, name in (("w1", 0, "weight"), ("b1", 0, "bias"), ("w2", 2, "weight"), ("b2", 2, "bias")):
        storage = moe._expert_storage[key]
        params = [getattr(expert.net[layer], name) for expert in moe.experts]
        step = params[0].numel() * params[0].element_size()
        assert storage.device.type == device_type and storage.dtype == dtype
        assert storage.is_contiguous() and all(p.is_contiguous() for p in params)
        assert storage.shape == (moe.num_experts, *params[0].shape)
        assert [p.data_ptr() for p in params] == [storage.data_ptr() + e * step for e in range(moe.num_experts)]


def test_canonical_storage_survives_load_and_dtype_apply():
    moe = MoEFeedForward(32, 128, 4, 2)
    names = {f"experts.{e}.{layer}.{p}" for e in range(4) for layer in ("net.0", "net.2") for p in ("weight", "bias")}
    assert set(moe.state_dict()) == names | {"router.weight"}
    for assign in (False, True):
        checkpoint = {name: torch.randn_like(p) for name, p in moe.state_dict().items()}
        moe.load_state_dict(checkpoint, assign=assign)
        for name, p in moe.state_dict().items():
            assert torch.equal(p, checkpoint[name])
        assert_canonical_storage(moe, device_type="cpu", dtype=torch.float32)
    moe.double()
    assert_canonical_storage(moe, device_type="cpu", dtype=torch.float64)
    moe.float()
    assert_canonical_storage(moe, device_type="cpu", dtype=torch.float32)


def test_packed_experts_compute_what_unpacked_experts_compute():
    torch.manual_seed(0)
    moe = MoEFeedForward(32, 64, 4, 2)
    x = torch.randn(1, 5, 32)
    with torch.no_grad():
        got = moe(x)
        logits = moe.router(x[0])
        top, ids = torch.topk(logits, 2, dim=-1)
        weights = torch.softmax(top, dim=-1)
        want = torch.stack(
            [sum(weights[t, s] * moe.experts[int(ids[t, s])](x[0, t]) for s in range(2)) for t in range(5)]
        )
    torch.testing.assert_close(got[0], want, atol=1e-6, rtol=1e-5)


def test_moe_auto_falls_back_on_cpu_and_forced_direct_fails():
    torch.manual_seed(0)
    moe = MoEFeedForward(32, 128, 4, 2, mode="auto").eval()
    x = torch.randn(1, 1, 32)
    with torch.no_grad():
        torch.testing.assert_close(moe(x, decode=True), moe._forward_reference(x), atol=0, rtol=0)
    moe.set_mode("direct")
    with pytest.raises(RuntimeError, match="direct"):
        moe(x, decode=True)
    prefill = x.expand(1, 2, 32)
    with torch.no_grad():
        torch.testing.assert_close(moe(prefill, decode=False), moe._forward_reference(prefill), atol=0, rtol=0)
    with pytest.raises(ValueError, match="unknown MoE mode"):
        moe.set_mode("fast")


def test_decode_plans_are_dropped_when_parameters_can_change():
    """A block's one-token launch plan holds parameter addresses; conversions
    (.to / .float / .double), load_state_dict (copy and assign) and
    drop_decode_plan() forget it, so the next decode token builds a new one."""
    model = Model(ModelConfig(**TINY)).eval()
    blocks = list(model.MoEBlocks)

    def plant():
        for b in blocks:
            b._one_token = ("stale key", None)

    for change in (
        lambda: model.float(),
        lambda: model.to("cpu"),
        lambda: model.load_state_dict(model.state_dict()),
        lambda: model.load_state_dict({k: v.clone() for k, v in model.state_dict().items()}, assign=True),
        lambda: [b.drop_decode_plan() for b in blocks],
    ):
        plant()
        change()
        assert all(b._one_token is None for b in blocks)


def test_submodule_changes_advance_the_plan_epoch():
    """Launch plans hold tensor addresses; every conversion, load or
    assignment that can replace a tensor inside a block's modules advances
    the epoch that is part of each plan's key, including changes made on a
    submodule (the block itself is not told)."""
    from moe_engine import model as model_mod

    model = Model(ModelConfig(**TINY)).eval()
    block = model.MoEBlocks[0]
    for change in (
        lambda: block.moe.float(),
        lambda: block.moe.load_state_dict(block.moe.state_dict()),
        lambda: block.attention.to("cpu"),
        lambda: block.attention.load_state_dict({k: v.clone() for k, v in block.attention.state_dict().items()},
                                                assign=True),
        lambda: block.moe.router.float(),
        lambda: block.moe.experts[1].net[0].float(),
        lambda: block.attn_norm.float(),
        lambda: setattr(block.attention.out_proj, "weight", torch.nn.Parameter(torch.zeros(32, 32))),
        lambda: setattr(block.moe_norm, "bias", torch.nn.Parameter(torch.zeros(32))),
        # The embedding tables (the first block's plan and a captured decode
        # step read them) and a plan dropped by hand.
        lambda: setattr(model.positional_embedding, "weight", torch.nn.Parameter(torch.zeros(128, 32))),
        lambda: model.token_embedding.float(),
        lambda: model.load_state_dict({k: v.clone() for k, v in model.state_dict().items()}, assign=True),
        lambda: block.drop_decode_plan(),
    ):
        before = model_mod._TENSOR_EPOCH[0]
        change()
        assert model_mod._TENSOR_EPOCH[0] > before
    # Decoding leaves the epoch alone (a plan or a captured step built for it stays valid).
    before = model_mod._TENSOR_EPOCH[0]
    with torch.no_grad():
        cache = model.new_block_allocator(num_blocks=8, block_size=4).new_cache()
        model(torch.tensor([[1, 2, 3]]), cache)
        model(torch.tensor([[4]]), cache)
    assert model_mod._TENSOR_EPOCH[0] == before
    # State-dict names and module types the reference's callers check are unchanged.
    assert isinstance(block.attn_norm, torch.nn.LayerNorm) and isinstance(block.moe.router, torch.nn.Linear)
    assert isinstance(model.token_embedding, torch.nn.Embedding)
    assert "MoEBlocks.0.attention.out_proj.weight" in model.state_dict()


def test_mode_and_eps_changes_advance_the_plan_epoch():
    """A launch plan is built from a MoE layer's mode and each norm's eps:
    changing either retires every plan and decode step (the epoch moves);
    setting the value a module already holds does not."""
    from moe_engine.model import _TENSOR_EPOCH

    model = Model(ModelConfig(**TINY)).eval()
    block = model.MoEBlocks[0]
    before = _TENSOR_EPOCH[0]
    block.moe.set_mode(block.moe.mode)
    block.attn_norm.eps = block.attn_norm.eps
    assert _TENSOR_EPOCH[0] == before
    block.moe.set_mode("reference")
    assert _TENSOR_EPOCH[0] == before + 1
    block.moe_norm.eps = 1e-3
    assert _TENSOR_EPOCH[0] == before + 2


def test_copies_leave_launch_plans_and_steps_behind():
    """A plan or decode step points at its own model's tensors, so deepcopy
    and pickling give a model without them (it builds its own on first use);
    the original keeps its own."""
    import copy
    import ctypes
    import pickle

    model = Model(ModelConfig(**TINY)).eval()
    model._steps["key"] = (None, (ctypes.c_void_p * 2)(1, 2), [])  # pointers: not copyable themselves
    block = model.MoEBlocks[1]
    block._plans["key"] = ("key", None, None)
    block._one_token = ("key", None, None)
    for twin in (copy.deepcopy(model), pickle.loads(pickle.dumps(model))):
        assert not twin._steps and all(not b._plans and b._one_token is None for b in twin.MoEBlocks)
        for a, b in zip(model.state_dict().values(), twin.state_dict().values()):
            assert torch.equal(a, b)
    assert len(model._steps) == 1 and block._one_token is not None



def test_bfloat16_layers_keep_float32_routing_workspaces():
    """A dtype conversion follows the experts, the GELU activations and the
    output workspace, but the routing logits and weights stay float32 (the
    reference routes in float32); the canonical layout check accepts the
    bfloat16 layer, and the fused kernels stay off away from a ROCm device."""
    from moe_engine import fused_moe

    layer = MoEFeedForward(32, 64, 4, 2).to(torch.bfloat16)
    assert layer._router_logits.dtype == torch.float32 and layer._route_weights.dtype == torch.float32
    assert layer._expert_hidden.dtype == torch.bfloat16 and layer._direct_out.dtype == torch.bfloat16
    assert layer._expert_storage["w1"].dtype == torch.bfloat16
    assert layer._has_direct_layout()
    assert not layer.direct_configuration_supported(1)  # CPU
    layer = layer.float()
    assert layer._expert_hidden.dtype == torch.float32 and layer._has_direct_layout()
    s = layer._expert_storage
    # A routing workspace in the model dtype is not the canonical layout.
    assert not fused_moe.has_canonical_layout(
        layer.router.weight.bfloat16(), s["w1"].bfloat16(), s["b1"].bfloat16(), s["w2"].bfloat16(),
        s["b2"].bfloat16(), layer._router_logits.bfloat16(), layer._expert_ids, layer._route_weights,
        layer._expert_hidden.bfloat16(), layer._direct_out.bfloat16())


def _bf16_moe_path(layer, x, keep_gelu_float=False, reverse_sums=False):
    """The reference's bfloat16 MoE (model.py:443-461) written out with its
    rounding points: each Linear's float32 sum plus bias rounded once, GELU
    rounded, the route weight and the weighted product rounded, index_add_
    rounding each partial sum.  keep_gelu_float drops one rounding point;
    reverse_sums keeps them all and reverses the dot products' order."""
    import torch.nn.functional as F

    flat = x.reshape(-1, layer.dim)
    logits = F.linear(flat.float(), layer.router.weight.float())
    top_logits, top_ids = torch.topk(logits, layer.top_k)
    weights = F.softmax(top_logits, dim=-1)
    out = torch.zeros_like(flat)

    def linear(v, w, b):
        if reverse_sums:
            v, w = v.flip(-1), w.flip(-1)
        return (v.float() @ w.float().t() + b.float()).to(torch.bfloat16)

    for e, expert in enumerate(layer.experts):
        tok, slot = torch.where(top_ids == e)
        if tok.numel() == 0:
            continue
        first, second = expert.net[0], expert.net[2]
        h = F.gelu(linear(flat[tok], first.weight, first.bias).float())
        h = h if keep_gelu_float else h.to(torch.bfloat16)
        y = linear(h, second.weight, second.bias)
        out.index_add_(0, tok, weights[tok, slot].unsqueeze(-1).to(torch.bfloat16) * y)
    return out


def test_bf16_moe_identity_bar_separates_reordering_from_a_dropped_rounding():
    """The GPU bfloat16 MoE tests require at least 90 % of the outputs to be
    bit-identical to the PyTorch path's.  This pins what that bar can tell
    apart, on the CPU: summing the dot products in another order (what the
    fused kernels legitimately do) leaves nearly every output identical,
    while dropping one rounding point (GELU's) leaves well under 90 %."""
    torch.manual_seed(50)
    for dim, hidden, experts, top_k in ((256, 200, 17, 4), (128, 512, 8, 2)):
        layer = MoEFeedForward(dim, hidden, experts, top_k).to(torch.bfloat16).eval()
        x = torch.randn(16, 1, dim).to(torch.bfloat16)
        with torch.no_grad():
            base = _bf16_moe_path(layer, x)
            reference = layer._forward_reference(x).reshape(base.shape)
            reordered = _bf16_moe_path(layer, x, reverse_sums=True)
            dropped = _bf16_moe_path(layer, x, keep_gelu_float=True)
        same = lambda a, b: (a.float() == b.float()).float().mean().item()  # noqa: E731
        assert same(base, reference) >= 0.97  # the restatement has the reference path's rounding points
        assert same(base, reordered) >= 0.97
        assert same(base, dropped) < 0.75
