"""Engine-level parity on the GPU: the paged path inside the full model.

Mirrors the reference's model-level kernel tests
(tests/test_paged_attention.py:130-182, 249-259) and adds BASELINE config 1:
the miniMoE-shaped decoder (12 layers, d 768, 12 heads x 64, top-2 of 8,
FFN 2048, vocab 50257, float32, block 16) greedy-decoding 64 tokens after a
32-token prompt, token-identical across GPU paged-direct, GPU paged-gather,
GPU contiguous and the CPU contiguous path.
"""

import pytest
import torch

from conftest import print_case
from moe_engine import _native
from moe_engine.model import BlockAllocator, Model, ModelConfig

pytestmark = pytest.mark.gpu

TINY = dict(max_seq_length=128, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)
E2E = dict(max_seq_length=1024, vocab_size=50257, num_layers=12, hidden_dim=768, num_heads=12,
           num_experts=8, top_k=2, ffn_dim=2048)


def stepwise_logits(model, ids, cache, prefill):
    with torch.no_grad():
        steps = [model(ids[:, :prefill], cache)[:, -1]]
        for t in range(prefill, ids.shape[1]):
            steps.append(model(ids[:, t : t + 1], cache)[:, -1])
    return torch.stack(steps, dim=1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_direct_decode_logits_match_gather(dtype):
    """Production dims (768 hidden, 8 heads x 96), prefill 50 then 12 decode steps.

    float32: within 1e-4 (reference tests/test_paged_attention.py:148).
    bfloat16: the direct kernel and SDPA round their attention outputs to bf16
    independently, and a one-ULP difference grows through two layers into the
    logits, whose bf16 ULP is 0.125 at |logit| ~ 28.  So the bf16 check is a
    relative error below 1 % plus identical argmax wherever the top-2 margin
    exceeds the largest logit difference.
    """
    print_case("direct vs gather logits", dtype)
    torch.manual_seed(0)
    model = Model(ModelConfig(max_seq_length=256, num_layers=2)).to("cuda", dtype).eval()
    ids = torch.randint(0, 1000, (1, 62), device="cuda")
    logits = {}
    for mode in ("gather", "direct"):
        cache = model.new_block_allocator(num_blocks=16, block_size=16, attention_mode=mode).new_cache()
        logits[mode] = stepwise_logits(model, ids, cache, 50).float()
        cache.free()
    direct, gather = logits["direct"], logits["gather"]
    if dtype == torch.float32:
        torch.testing.assert_close(direct, gather, atol=1e-4, rtol=1e-4)
        return
    rel = ((direct - gather).norm() / gather.norm()).item()
    assert rel < 1e-2, f"relative logit error {rel:.3e}"
    worst = (direct - gather).abs().max()
    top2 = gather.topk(2, dim=-1).values
    decided = (top2[..., 0] - top2[..., 1]) > 2 * worst
    assert torch.equal(direct.argmax(-1)[decided], gather.argmax(-1)[decided])


def test_greedy_generation_matches_contiguous():
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").eval()
    prompt = torch.randint(0, TINY["vocab_size"], (8,), device="cuda")
    contiguous = model.generate(prompt, max_new_tokens=40, temperature=0)
    cache = model.new_block_allocator(num_blocks=16, block_size=4, attention_mode="direct").new_cache()
    direct = model.generate(prompt, max_new_tokens=40, temperature=0, cache=cache)
    cache.free()
    assert torch.equal(direct, contiguous)


def test_blocks_reused_after_generation():
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").eval()
    prompt = torch.randint(0, TINY["vocab_size"], (8,), device="cuda")
    allocator = model.new_block_allocator(num_blocks=16, block_size=4, attention_mode="direct")
    cache = allocator.new_cache()
    first = model.generate(prompt, max_new_tokens=20, temperature=0, cache=cache)
    cache.free()
    assert sorted(allocator.free_blocks) == list(range(16))
    cache = allocator.new_cache()
    second = model.generate(prompt, max_new_tokens=20, temperature=0, cache=cache)
    cache.free()
    assert torch.equal(first, second)


def test_device_mirror_follows_the_host_table_through_the_append_launch():
    """_reserve appends new block ids to the device mirror with one
    mie_block_table_append launch (ids in its arguments) for up to 16 new
    blocks, else an indexed copy; either way the mirror's first
    len(block_table) entries equal the host table, in LIFO order, and
    entries past it keep what they held."""
    torch.manual_seed(0)
    cfg = ModelConfig(**TINY)
    allocator = BlockAllocator(cfg, num_blocks=64, block_size=4, device="cuda", attention_mode="direct")
    cache = allocator.new_cache()
    lib = _native.lib()
    real = lib.mie_block_table_append
    launches = []

    def counted(*args):
        launches.append(args[4])
        return real(*args)

    lib.mie_block_table_append = counted
    try:
        cache._reserve(9)  # 3 blocks: one launch
        assert cache.block_table == [63, 62, 61] and launches == [3]
        for n in range(10, 41):  # one new block every 4 tokens
            cache._reserve(n)
        assert len(cache.block_table) == 10 and launches == [3] + [1] * 7
        cache._reserve(40 + 4 * 20)  # 20 new blocks at once: the indexed copy
        assert len(cache.block_table) == 30 and len(launches) == 8
    finally:
        lib.mie_block_table_append = real
    torch.cuda.synchronize()
    mirror = cache.block_table_device.cpu().tolist()
    assert mirror[:30] == cache.block_table == list(range(63, 33, -1))
    assert mirror[30:] == [0] * 34
    cache.free()
    assert cache.block_table == [] and sorted(allocator.free_blocks) == list(range(64))


def test_direct_mode_rejects_float64_before_mutating():
    model = Model(ModelConfig(**TINY)).to("cuda").double().eval()
    ids = torch.randint(0, TINY["vocab_size"], (1, 5), device="cuda")
    allocator = model.new_block_allocator(num_blocks=8, block_size=4, attention_mode="direct")
    cache = allocator.new_cache()
    with torch.no_grad(), pytest.raises(RuntimeError, match="direct"):
        model(ids, cache)
    assert cache.position == 0 and cache.block_table == []
    assert sorted(allocator.free_blocks) == list(range(8))
    assert (cache.block_table_device == 0).all() and cache._write_index_key is None


def test_auto_mode_uses_gather_for_float64_and_matches_contiguous():
    """auto falls back to the gather path (HIP gather + SDPA) where the direct
    kernel is not built; results follow the contiguous cache."""
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").double().eval()
    ids = torch.randint(0, TINY["vocab_size"], (1, 12), device="cuda")
    with torch.no_grad():
        full = model(ids, model.new_cache())
    cache = model.new_block_allocator(num_blocks=8, block_size=4).new_cache()
    torch.testing.assert_close(stepwise_logits(model, ids, cache, 4), full[:, 3:], atol=1e-10, rtol=1e-10)


def e2e_prompt():
    return torch.randint(0, E2E["vocab_size"], (32,), generator=torch.Generator().manual_seed(0))


def test_config1_greedy_tokens_identical_across_paths():
    """BASELINE config 1 (random init from seed 0, fp32, block 16, 32-token
    prompt, 64 greedy tokens): GPU paged-direct == GPU paged-gather == GPU
    contiguous == CPU contiguous, token for token."""
    torch.manual_seed(0)
    cpu_model = Model(ModelConfig(**E2E)).eval()
    prompt = e2e_prompt()
    print_case("config1 cpu")
    cpu_tokens = cpu_model.generate(prompt, max_new_tokens=64, temperature=0)
    with torch.no_grad():
        cpu_logits = cpu_model(cpu_tokens[:, :-1], cpu_model.new_cache())
    model = cpu_model.to("cuda")
    outs = {}
    for system in ("contiguous", "paged-gather", "paged-direct"):
        print_case("config1", system)
        cache = None
        if system != "contiguous":
            allocator = model.new_block_allocator(num_blocks=64, block_size=16, attention_mode=system[6:])
            cache = allocator.new_cache()
        outs[system] = model.generate(prompt.cuda(), max_new_tokens=64, temperature=0, cache=cache).cpu()
        if cache is not None:
            cache.free()
    for system, tokens in outs.items():
        assert torch.equal(tokens, cpu_tokens), f"{system} diverged from the CPU path"
    # Logits of the full sequence through the paged-direct decode, step by step.
    cache = model.new_block_allocator(num_blocks=64, block_size=16, attention_mode="direct").new_cache()
    gpu_logits = stepwise_logits(model, cpu_tokens[:, :-1].cuda(), cache, 32).cpu()
    diff = (gpu_logits - cpu_logits[:, 31:]).abs().max().item()
    print(f"config1 max |logit diff| GPU paged-direct vs CPU contiguous: {diff:.3e}", flush=True)
    assert diff < 1e-2


# head_dim 32: the block plan takes the four-launch form (attention fused with
# out_proj), which TINY's head_dim 4 lacks.
TINY_FUSED = dict(TINY, hidden_dim=64, num_heads=2)


@pytest.mark.parametrize("cfg,launches", [(TINY, 5), (TINY_FUSED, 4)], ids=["five_launch", "four_launch"])
def test_cached_one_token_plan_follows_cache_and_weight_changes(cfg, launches):
    """The eager one-token decode runs each block from a cached launch plan
    (TransformerMoEBlock._decode_one_token).  Every decode below must equal
    the same step with the plan disabled (the per-call fused path), to float32
    rounding, after changing what the plan depends on: a second cache on another
    allocator, reloaded weights (new tensors, assign=True), the MoE mode, a
    module conversion, a parameter replaced by hand (with drop_decode_plan),
    and the allocator's fuse_qkv switch."""
    print_case("cached one-token plan", launches)
    torch.manual_seed(0)
    model = Model(ModelConfig(**cfg)).to("cuda").eval()
    ids = torch.randint(0, cfg["vocab_size"], (1, 12), device="cuda")

    def run(cache_factory, use_plan):
        blocks = list(model.MoEBlocks)
        saved = [b._decode_one_token for b in blocks]
        if not use_plan:
            for b in blocks:
                b._decode_one_token = lambda *args, **kwargs: None
        try:
            cache = cache_factory()
            out = stepwise_logits(model, ids, cache, 5)
            cache.free()
            return out
        finally:
            for b, f in zip(blocks, saved):
                b._decode_one_token = f

    alloc_a = model.new_block_allocator(num_blocks=16, block_size=4, attention_mode="direct")
    alloc_b = model.new_block_allocator(num_blocks=24, block_size=8, attention_mode="direct")

    def check(factory):
        # The plan runs the four-launch block (attention fused with out_proj,
        # heads summed in fixed point): float32 rounding away from the
        # per-call five launches, far below what stale weights or a stale
        # cache would change.
        torch.testing.assert_close(run(factory, True), run(factory, False), rtol=1e-5, atol=1e-5)

    check(alloc_a.new_cache)
    assert all(b._one_token is not None and b._one_token[2] is not None for b in model.MoEBlocks)
    lib = _native.lib()
    assert all(lib.mie_block_plan_launches(b._one_token[2].plan, 11) == launches for b in model.MoEBlocks)
    check(alloc_b.new_cache)
    check(alloc_a.new_cache)
    # New parameter tensors at new addresses.
    state = {k: v.clone() * 0.5 for k, v in model.state_dict().items()}
    model.load_state_dict(state, assign=True)
    check(alloc_a.new_cache)
    # The PyTorch MoE path (no plan), then back.
    model.set_moe_mode("reference")
    check(alloc_a.new_cache)
    assert all(b._one_token[2] is None for b in model.MoEBlocks)
    model.set_moe_mode("auto")
    check(alloc_a.new_cache)
    # A conversion (.float() is one even when nothing changes) drops the plans.
    model.float()
    assert all(b._one_token is None for b in model.MoEBlocks)
    check(alloc_a.new_cache)
    # A parameter replaced by hand, then the plan dropped by hand.
    out_proj = model.MoEBlocks[1].attention.out_proj
    out_proj.weight = torch.nn.Parameter(out_proj.weight.detach() * 0.25)
    model.MoEBlocks[1].drop_decode_plan()
    check(alloc_a.new_cache)
    # Submodule-level conversions, loads and assignments, with no
    # drop_decode_plan: each one replaces tensors the plan points at.
    block = model.MoEBlocks[0]
    for change in (
        lambda: block.moe.float(),
        lambda: block.moe.load_state_dict({k: v.clone() * 0.5 for k, v in block.moe.state_dict().items()}),
        lambda: block.attention.to("cuda"),
        lambda: block.attention.load_state_dict(
            {k: v.clone() * 0.5 for k, v in block.attention.state_dict().items()}, assign=True),
        lambda: setattr(block.attn_norm, "weight", torch.nn.Parameter(block.attn_norm.weight.detach() + 0.5)),
        lambda: setattr(block.moe.router, "weight", torch.nn.Parameter(block.moe.router.weight.detach() * -1)),
    ):
        change()
        check(alloc_a.new_cache)
    # The reference's projection + append sequence for the attention half.
    alloc_a.fuse_qkv = False
    check(alloc_a.new_cache)
    assert all(b._one_token[2] is None for b in model.MoEBlocks)


def test_block_plans_do_not_keep_finished_caches_alive():
    """A plan refers to its cache weakly and holds only addresses: once a
    sequence's cache and allocator are dropped, their pools are freed even
    though every block still holds the plan built for them."""
    import gc
    import weakref

    print_case("plan does not hold the pools")
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").eval()
    ids = torch.randint(0, TINY["vocab_size"], (1, 8), device="cuda")
    alloc = model.new_block_allocator(num_blocks=16, block_size=4, attention_mode="direct")
    cache = alloc.new_cache()
    stepwise_logits(model, ids, cache, 4)
    assert all(b._one_token is not None and b._one_token[2] is not None for b in model.MoEBlocks)
    pool = weakref.ref(alloc.k_pool)
    del cache, alloc
    gc.collect()
    assert pool() is None, "a block's launch plan kept a finished cache's pools alive"
    # A new cache (possibly at the dead one's id) builds a new plan and decodes as the per-call path does.
    alloc = model.new_block_allocator(num_blocks=16, block_size=4, attention_mode="direct")
    got = stepwise_logits(model, ids, alloc.new_cache(), 4)
    for b in model.MoEBlocks:
        b.drop_decode_plan()
        b._decode_one_token = lambda *args, **kwargs: None
    try:
        want = stepwise_logits(model, ids, alloc.new_cache(), 4)
    finally:
        for b in model.MoEBlocks:
            del b._decode_one_token
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_hidden_states_is_the_callers_tensor():
    """For one decode token the last block leaves its output in a per-layer
    buffer; Model.hidden_states returns a copy, so a result kept across steps
    does not change (as the reference's does not)."""
    print_case("hidden_states copy")
    torch.manual_seed(0)
    model = Model(ModelConfig(**TINY)).to("cuda").eval()
    cache = model.new_block_allocator(num_blocks=16, block_size=4, attention_mode="direct").new_cache()
    with torch.no_grad():
        model.hidden_states(torch.tensor([[1, 2, 3]], device="cuda"), cache)
        first = model.hidden_states(torch.tensor([[4]], device="cuda"), cache)
        kept = first.clone()
        model.hidden_states(torch.tensor([[5]], device="cuda"), cache)
    assert torch.equal(first, kept)


def test_block_plan_switches_forms_at_1024_tokens():
    """A sequence that crosses 1024 cached tokens moves from the four-launch
    block (attention fused with out_proj; head_dim 32) to the five-launch one
    mid-sequence (the two-head decode then splits its context: six launches);
    every step's logits stay within float32 rounding of the per-call path."""
    print_case("block plan form switch")
    torch.manual_seed(2)
    cfg = dict(max_seq_length=1100, vocab_size=96, num_layers=2, hidden_dim=64, num_heads=2, num_experts=4, top_k=2)
    model = Model(ModelConfig(**cfg)).to("cuda").eval()
    ids = torch.randint(0, cfg["vocab_size"], (1, 1040), device="cuda")
    alloc = model.new_block_allocator(num_blocks=70, block_size=16, attention_mode="direct")
    cache = alloc.new_cache()
    calls = _CountedSteps()
    try:
        got = stepwise_logits(model, ids, cache, 1015)
    finally:
        calls.restore()
    cache.free()
    # The one-call step built at 1016 tokens (no workspace) met the split
    # context at 1024: it launched nothing, the blocks grew their workspaces
    # one by one, and a new step served the rest.
    assert calls.refused >= 1 and calls.done == (1040 - 1015 - 1) - calls.refused
    lib = _native.lib()
    for b in model.MoEBlocks:
        plan = b._one_token[2].plan
        assert lib.mie_block_plan_launches(plan, 1015) == 4 and lib.mie_block_plan_launches(plan, 1023) == 4
        assert lib.mie_block_plan_launches(plan, 1024) >= 5 and lib.mie_block_plan_launches(plan, 1038) >= 5
    for b in model.MoEBlocks:
        b.drop_decode_plan()
        b._decode_one_token = lambda *args, **kwargs: None
    try:
        want = stepwise_logits(model, ids, alloc.new_cache(), 1015)
    finally:
        for b in model.MoEBlocks:
            del b._decode_one_token
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_block_plan_grows_its_workspace_for_split_contexts():
    """Past 1024 cached tokens the plan takes the five-launch block, and with
    few heads the decode splits the context into partitions and needs a
    workspace: the block's launch plan (mie_block_decode) refuses such a
    position before launching anything, and the block sets the plan up again
    with a workspace.  Logits equal the per-call fused path's bit for bit at
    every step (the same five launches), and a plan holds a workspace after."""
    print_case("block plan workspace growth")
    torch.manual_seed(1)
    cfg = dict(max_seq_length=2200, vocab_size=96, num_layers=2, hidden_dim=64, num_heads=2, num_experts=4, top_k=2)
    model = Model(ModelConfig(**cfg)).to("cuda").eval()
    ids = torch.randint(0, cfg["vocab_size"], (1, 2070), device="cuda")
    alloc = model.new_block_allocator(num_blocks=140, block_size=16, attention_mode="direct")

    def run(use_plan):
        blocks = list(model.MoEBlocks)
        saved = [b._decode_one_token for b in blocks]
        if not use_plan:
            for b in blocks:
                b._decode_one_token = lambda *args, **kwargs: None
        try:
            cache = alloc.new_cache()
            out = stepwise_logits(model, ids, cache, 2055)
            cache.free()
            return out
        finally:
            for b, f in zip(blocks, saved):
                b._decode_one_token = f

    calls = _CountedSteps()
    try:
        assert torch.equal(run(True), run(False))
    finally:
        calls.restore()
    # The first decode token grew the workspaces block by block; the model's
    # one-call step, built after it, served the tokens that followed.
    assert calls.done == (2070 - 2055 - 1) - calls.refused
    for b in model.MoEBlocks:
        launcher = b._one_token[2]
        assert launcher is not None and launcher.held["ws"] is not None


class _CountedSteps:
    """Counts mie_blocks_decode calls (the model's one-call decode step):
    those that ran and those refused for want of a workspace."""

    def __init__(self):
        self.lib = _native.lib()
        self.real = self.lib.mie_blocks_decode
        self.done = self.refused = 0

        def counted(*args):
            rc = self.real(*args)
            if rc == _native.ERR_WORKSPACE:
                self.refused += 1
            elif rc == 0:
                self.done += 1
            return rc

        self.lib.mie_blocks_decode = counted

    def restore(self):
        self.lib.mie_blocks_decode = self.real


def test_decode_step_runs_every_block_in_one_call():
    """After a sequence's first decode token has built the blocks' launch
    plans, each later token runs the embedding and every block in one
    library call (mie_blocks_decode) - the same launches, so the logits equal
    the block-by-block path bit for bit.  Sequences decoded in turn keep their
    own steps; a MoE mode or norm eps change retires the step (the epoch
    moves) and the next tokens follow the change."""
    print_case("one-call decode step")
    torch.manual_seed(6)
    model = Model(ModelConfig(**TINY_FUSED)).to("cuda").eval()
    alloc = model.new_block_allocator(num_blocks=40, block_size=4, attention_mode="direct")
    ids = torch.randint(0, TINY_FUSED["vocab_size"], (2, 30), device="cuda")

    def block_by_block(rows, prefill):
        saved = model._run_decode_step
        model._run_decode_step = lambda *args, **kwargs: None
        try:
            cache = alloc.new_cache()
            return stepwise_logits(model, rows, cache, prefill)
        finally:
            cache.free()
            model._run_decode_step = saved

    calls = _CountedSteps()
    try:
        cache = alloc.new_cache()
        got = stepwise_logits(model, ids[:1], cache, 6)
        cache.free()
        assert calls.done == 30 - 6 - 1 and calls.refused == 0  # the first decode token builds the step
        assert torch.equal(got, block_by_block(ids[:1], 6))

        # Two sequences in turn: each finds its own step after its first token.
        calls.done = 0
        caches = [alloc.new_cache(), alloc.new_cache()]
        steps = [[], []]
        with torch.no_grad():
            for s in range(2):
                steps[s].append(model(ids[s : s + 1, :6], caches[s])[:, -1])
            for t in range(6, 30):
                for s in range(2):
                    steps[s].append(model(ids[s : s + 1, t : t + 1], caches[s])[:, -1])
        # The one-call steps took a new block every 4 tokens and wrote its id
        # into the device table from layer 0's QKV launch: the mirror matches.
        for c in caches:
            assert c.block_table_device[: len(c.block_table)].tolist() == c.block_table
            c.free()
        assert calls.done == 2 * (30 - 6 - 1)
        for s in range(2):
            assert torch.equal(torch.stack(steps[s], 1), block_by_block(ids[s : s + 1], 6))

        # A norm eps change retires the step; the next tokens use the new eps.
        calls.done = 0
        model.MoEBlocks[1].moe_norm.eps = 1e-2
        cache = alloc.new_cache()
        got = stepwise_logits(model, ids[:1], cache, 6)
        cache.free()
        assert calls.done == 30 - 6 - 1
        assert torch.equal(got, block_by_block(ids[:1], 6))

        # The reference MoE path has no launch plan: no step while it is set.
        calls.done = 0
        model.set_moe_mode("reference")
        cache = alloc.new_cache()
        ref = stepwise_logits(model, ids[:1], cache, 6)
        cache.free()
        assert calls.done == 0
        model.set_moe_mode("auto")
        torch.testing.assert_close(ref, got, rtol=1e-4, atol=1e-4)
    finally:
        calls.restore()


def test_embedding_folded_into_the_first_qkv_launch():
    """For one decode token of a float32 model (the dtype the block's launch
    plan serves), layer 0 forms x from the token id and the two
    embedding tables inside its QKV launch (mie_block_decode_embed) and keeps
    it as the block's residual.  Every step's logits equal those of the
    separate embedding launch bit for bit (the same float32 sum, rounded once),
    the residual row equals token_embedding[id] + positional_embedding[pos] as
    torch rounds it, and a token id outside the vocabulary makes the row NaN
    instead of reading past the table."""
    print_case("embedding fold")
    torch.manual_seed(3)
    model = Model(ModelConfig(max_seq_length=256, num_layers=2)).to("cuda").eval()
    ids = torch.randint(0, 1000, (1, 70), device="cuda")
    alloc = model.new_block_allocator(num_blocks=16, block_size=16, attention_mode="direct")
    first = model.MoEBlocks[0]
    cache = alloc.new_cache()
    got = stepwise_logits(model, ids, cache, 50)
    cache.free()
    assert first._one_token[0][-4] == model.token_embedding.weight.data_ptr(), "the folded plan did not run"
    row = first._embed_row.clone()
    with torch.no_grad():
        want_row = model.token_embedding(ids[:, -1:]) + model.positional_embedding.weight[69]
    assert torch.equal(row, want_row)
    first.decode_token_ids = lambda *args, **kwargs: None
    try:
        cache = alloc.new_cache()
        want = stepwise_logits(model, ids, cache, 50)
        cache.free()
    finally:
        del first.decode_token_ids
    assert torch.equal(got, want)
    # An id past the vocabulary: the row (and so the logits) become NaN.
    cache = alloc.new_cache()
    with torch.no_grad():
        model(ids[:, :5], cache)
        bad = torch.tensor([[model.config.vocab_size]], device="cuda")
        out = model(bad, cache)
    cache.free()
    assert torch.isnan(first._embed_row).all() and torch.isnan(out).all()


def test_sequences_decoded_in_turn_keep_their_plans():
    """Two sequences decoded in turn, one token each, find their own launch
    plans again - a block keeps its last few - instead of rebuilding them
    every token; each sequence's logits equal those it gets decoded alone,
    bit for bit (the same launches)."""
    print_case("plans of sequences in turn")
    torch.manual_seed(4)
    model = Model(ModelConfig(**TINY_FUSED)).to("cuda").eval()
    alloc = model.new_block_allocator(num_blocks=40, block_size=4, attention_mode="direct")
    ids = torch.randint(0, TINY_FUSED["vocab_size"], (2, 30), device="cuda")
    builds = []
    for b in model.MoEBlocks:
        build = b._build_one_token
        b._build_one_token = lambda *args, _build=build, **kwargs: builds.append(1) or _build(*args, **kwargs)
    try:
        alone = []
        for s in range(2):
            cache = alloc.new_cache()
            alone.append(stepwise_logits(model, ids[s : s + 1], cache, 6))
            cache.free()
        builds.clear()
        caches = [alloc.new_cache(), alloc.new_cache()]
        steps = [[], []]
        with torch.no_grad():
            for s in range(2):
                steps[s].append(model(ids[s : s + 1, :6], caches[s])[:, -1])
            for t in range(6, 30):
                for s in range(2):
                    steps[s].append(model(ids[s : s + 1, t : t + 1], caches[s])[:, -1])
        for s in range(2):
            assert torch.equal(torch.stack(steps[s], 1), alone[s])
        assert len(builds) == 2 * len(model.MoEBlocks), f"{len(builds)} plan builds for two sequences"
        for c in caches:
            c.free()
    finally:
        for b in model.MoEBlocks:
            b.__dict__.pop("_build_one_token", None)
