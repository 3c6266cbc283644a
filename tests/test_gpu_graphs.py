"""Whole decode steps replayed from a HIP graph (moe_engine.graphs) against
the eager paged-direct path.

Each test replays the captured step many times across block boundaries, with
eager work of the same model (another sequence in the same block pool) and a
device synchronization between replays, and checks every replay: its logits
against the eager step's for the same token and position, and the greedy
tokens against Model.generate (reference model.py:567-621).  Each block of
the captured step runs its launch plan with the device [position, length]
pair, sized for the model's capacity: up to 1024 positions that is the
four-launch block (attention fused with out_proj); at 2200 positions it is the
five-launch block, whose decode splits the context into partitions merged by
a second launch.  The eager launches are sized for the exact length, so
float32 logits agree to rounding, not always bit for bit.
"""

import pytest
import torch

from conftest import print_case
from moe_engine import _native
from moe_engine.graphs import GraphedDecoder, GraphedGenerator, generate_graphed
from moe_engine.model import Model, ModelConfig

pytestmark = pytest.mark.gpu

TINY = dict(max_seq_length=128, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)
E2E = dict(max_seq_length=1024, vocab_size=50257, num_layers=12, hidden_dim=768, num_heads=12,
           num_experts=8, top_k=2, ffn_dim=2048)


def tiny_model(dtype=torch.float32, max_seq_length=None, **over):
    torch.manual_seed(0)
    cfg = dict(TINY, **over)
    if max_seq_length is not None:
        cfg["max_seq_length"] = max_seq_length
    return Model(ModelConfig(**cfg)).to("cuda", dtype).eval()


# (hidden_dim, num_heads): head_dim 32 has the four-launch block (attention
# fused with out_proj) up to 1024 positions; TINY's head_dim 4 only the
# five-launch one.  A captured step serves positions up to a bound (127, 255,
# ... capped by the capacity); `captures` counts the captures a run needs.
@pytest.mark.parametrize("block_size,max_seq_length,num_blocks,hidden_dim,num_heads,prompt_len,steps,captures,launches", [
    (4, 128, 80, 64, 2, 9, 100, 1, 4),
    (16, 128, 80, 64, 2, 9, 100, 1, 4),
    (16, 128, 80, 32, 8, 9, 100, 1, 5),
    # past 128 positions the fused attention takes 8 waves per workgroup: the
    # step is captured again at position 128 for the bound 255
    (16, 2200, 140, 64, 2, 110, 40, 2, 4),
    # the bound 2047: the two-head decode splits its context (partitions + merge)
    (16, 2200, 160, 64, 2, 1100, 30, 1, 6),  # 160 blocks: both caches hold 1130 tokens
])
def test_every_replay_matches_eager_step(block_size, max_seq_length, num_blocks, hidden_dim, num_heads, prompt_len,
                                         steps, captures, launches):
    print_case("graph replay vs eager", block_size, max_seq_length, num_blocks, hidden_dim, num_heads, prompt_len)
    model = tiny_model(max_seq_length=max_seq_length, hidden_dim=hidden_dim, num_heads=num_heads)
    allocator = model.new_block_allocator(num_blocks=num_blocks, block_size=block_size, attention_mode="direct")
    graphed, eager = allocator.new_cache(), allocator.new_cache()
    prompt = torch.randint(0, TINY["vocab_size"], (1, prompt_len), device="cuda")
    with torch.no_grad():
        first = model(prompt, graphed)[:, -1]
        torch.testing.assert_close(model(prompt, eager)[:, -1], first)
        decoder = GraphedDecoder(model, graphed)
        token = first.argmax(-1, keepdim=True)
        decoder.prime(token)
        for step in range(steps):
            got = decoder.step()
            got_logits = decoder.logits.clone()
            # Eager work between replays: the same step on the other sequence,
            # whose blocks interleave with the graphed sequence's in the pool.
            want_logits = model(token, eager)[:, -1]
            torch.cuda.synchronize()
            torch.testing.assert_close(got_logits, want_logits, atol=2e-5, rtol=2e-5,
                                       msg=lambda m: f"step {step}: {m}")
            token = want_logits.argmax(-1, keepdim=True)
            assert torch.equal(got, token), f"step {step}"
            assert graphed.position == eager.position
    assert decoder.captures == captures and decoder.replays == steps - captures
    # The form the captured blocks took, for the capture's position bound.
    bound = decoder.position_bound(graphed.position)
    assert decoder.bound == bound
    lib = _native.lib()
    for plan in decoder._plans:
        assert plan is not None and plan[2] is not None
        assert lib.mie_block_plan_launches(plan[2].plan, bound) == launches
    assert graphed.block_table != eager.block_table
    graphed.free()
    eager.free()
    assert len(allocator.free_blocks) == allocator.num_blocks


def test_replays_keep_the_captured_plans_alive():
    """The captured step points at the block plans' rows, accumulators and
    workspaces.  After capture every block's plan is dropped, and the freed
    memory is handed out again (torch's small blocks of the rows' and the
    accumulator's sizes, filled with junk), while eager steps on another
    cache build new plans.  The replays must still give the eager step's
    logits: the decoder holds the plans it captured."""
    import gc

    print_case("graph keeps its plans")
    model = tiny_model(hidden_dim=64, num_heads=2)
    allocator = model.new_block_allocator(num_blocks=80, block_size=16, attention_mode="direct")
    graphed, eager = allocator.new_cache(), allocator.new_cache()
    prompt = torch.randint(0, TINY["vocab_size"], (1, 9), device="cuda")
    junk = []
    with torch.no_grad():
        first = model(prompt, graphed)[:, -1]
        model(prompt, eager)
        decoder = GraphedDecoder(model, graphed)
        token = first.argmax(-1, keepdim=True)
        decoder.prime(token)
        for step in range(12):
            got = decoder.step()  # step 0 runs eagerly and captures
            got_logits = decoder.logits.clone()
            if step == 1:
                for block in model.MoEBlocks:
                    block.drop_decode_plan()
                gc.collect()
                junk = [torch.full((n,), -7, dtype=torch.int64, device="cuda") for n in (64, 128) for _ in range(4096)]
            want = model(token, eager)[:, -1]
            torch.cuda.synchronize()
            torch.testing.assert_close(got_logits, want, atol=2e-5, rtol=2e-5, msg=lambda m: f"step {step}: {m}")
            token = want.argmax(-1, keepdim=True)
            assert torch.equal(got, token), f"step {step}"
    del junk
    graphed.free()
    eager.free()


def test_replaced_weights_are_captured_again():
    """A captured step reads the weights' addresses.  After the weights are
    replaced - an assigning load, then a parameter swapped by hand with
    drop_decode_plan - the next step captures again, and its logits follow
    the new weights (against the eager step on another cache)."""
    print_case("graph recaptures after replacement")
    model = tiny_model(hidden_dim=64, num_heads=2)
    allocator = model.new_block_allocator(num_blocks=80, block_size=16, attention_mode="direct")
    graphed, eager = allocator.new_cache(), allocator.new_cache()
    prompt = torch.randint(0, TINY["vocab_size"], (1, 9), device="cuda")
    with torch.no_grad():
        first = model(prompt, graphed)[:, -1]
        model(prompt, eager)
        decoder = GraphedDecoder(model, graphed)
        token = first.argmax(-1, keepdim=True)
        decoder.prime(token)
        captures = 0
        for step in range(9):
            if step == 3:
                model.load_state_dict({k: v.clone() * 0.5 for k, v in model.state_dict().items()}, assign=True)
            if step == 6:
                norm = model.MoEBlocks[1].attn_norm
                norm.weight.data = norm.weight.detach() * 2  # a new tensor behind the same parameter
                model.MoEBlocks[1].drop_decode_plan()
            replays = decoder.replays
            got = decoder.step()
            captures += decoder.replays == replays
            got_logits = decoder.logits.clone()
            want = model(token, eager)[:, -1]
            torch.cuda.synchronize()
            torch.testing.assert_close(got_logits, want, atol=2e-5, rtol=2e-5, msg=lambda m: f"step {step}: {m}")
            token = want.argmax(-1, keepdim=True)
            assert torch.equal(got, token), f"step {step}"
        assert captures == 3 and decoder.replays == 6
    graphed.free()
    eager.free()


def test_generator_captures_again_when_a_request_changes_the_position_bound():
    """GraphedGenerator keeps one captured step across requests while their
    positions stay inside its bound (127, 255, ...).  A longer request is
    captured again for the larger bound, a short one after it for the smaller
    one again; every request's tokens equal Model.generate's."""
    print_case("graph generator bounds")
    model = tiny_model(max_seq_length=512, hidden_dim=64, num_heads=2)
    allocator = model.new_block_allocator(num_blocks=40, block_size=16, attention_mode="direct")
    gen = GraphedGenerator(model, allocator.new_cache())
    g = torch.Generator().manual_seed(4)
    requests = [(5, 12, 1), (9, 20, 1), (200, 12, 2), (7, 10, 3)]  # prompt length, new tokens, captures after
    for prompt_len, new, captures in requests:
        prompt = torch.randint(0, TINY["vocab_size"], (1, prompt_len), generator=g).cuda()
        cache = allocator.new_cache()
        want = model.generate(prompt, max_new_tokens=new, temperature=0, cache=cache)
        cache.free()
        got = gen.generate(prompt, new)
        assert torch.equal(got, want), (prompt_len, new)
        assert gen.decoder.captures == captures, (prompt_len, gen.decoder.captures)
    assert gen.decoder.bound == 127
    assert len(allocator.free_blocks) == allocator.num_blocks


def test_generate_graphed_matches_generate():
    print_case("generate_graphed")
    model = tiny_model()
    prompt = torch.randint(0, TINY["vocab_size"], (7,), device="cuda")
    allocator = model.new_block_allocator(num_blocks=40, block_size=4, attention_mode="direct")
    cache = allocator.new_cache()
    want = model.generate(prompt, max_new_tokens=60, temperature=0, cache=cache)
    cache.free()
    cache = allocator.new_cache()
    got = generate_graphed(model, prompt, 60, cache)
    assert cache.position == want.shape[1] - 1
    cache.free()
    assert torch.equal(got, want)


def test_graph_decoder_needs_fused_moe():
    """Mode 'reference' runs the PyTorch expert loop, which synchronizes the
    host; the decoder refuses it, in either dtype, before touching the cache.
    (bfloat16 models with the fused MoE are captured: test_gpu_moe_bf16.)"""
    for dtype, mode in ((torch.bfloat16, "reference"), (torch.float32, "reference")):
        model = tiny_model(dtype).set_moe_mode(mode)
        cache = model.new_block_allocator(num_blocks=8, block_size=4, attention_mode="direct").new_cache()
        with torch.no_grad():
            model(torch.zeros(1, 3, dtype=torch.long, device="cuda"), cache)
        with pytest.raises(RuntimeError, match="fused MoE"):
            GraphedDecoder(model, cache)
        assert cache.position == 3


def test_generate_graphed_stops_at_max_seq_length():
    model = tiny_model()
    prompt = torch.randint(0, TINY["vocab_size"], (100,), device="cuda")
    allocator = model.new_block_allocator(num_blocks=32, block_size=4, attention_mode="direct")
    cache = allocator.new_cache()
    want = model.generate(prompt, max_new_tokens=64, temperature=0, cache=cache)
    cache.free()
    cache = allocator.new_cache()
    got = generate_graphed(model, prompt, 64, cache)
    assert got.shape[1] == want.shape[1] == TINY["max_seq_length"] + 1
    assert torch.equal(got, want)
    assert cache.position == TINY["max_seq_length"]


def test_graph_decoder_rejects_gather_cache_and_empty_cache():
    model = tiny_model()
    gather = model.new_block_allocator(num_blocks=8, block_size=4, attention_mode="gather").new_cache()
    with pytest.raises(ValueError, match="graph decode"):
        GraphedDecoder(model, gather)
    direct = model.new_block_allocator(num_blocks=8, block_size=4, attention_mode="direct").new_cache()
    with pytest.raises(ValueError, match="prefill"):
        GraphedDecoder(model, direct)


def test_config1_graphed_tokens_identical_to_eager():
    """BASELINE config 1 shape, 32-token prompt then 64 greedy tokens."""
    print_case("config1 graphed")
    torch.manual_seed(0)
    model = Model(ModelConfig(**E2E)).to("cuda").eval()
    prompt = torch.randint(0, E2E["vocab_size"], (32,), device="cuda")
    allocator = model.new_block_allocator(num_blocks=64, block_size=16, attention_mode="direct")
    cache = allocator.new_cache()
    want = model.generate(prompt, max_new_tokens=64, temperature=0, cache=cache)
    cache.free()
    cache = allocator.new_cache()
    got = generate_graphed(model, prompt, 64, cache)
    cache.free()
    assert torch.equal(got, want)


def test_argmax_kernel_matches_torch_argmax():
    """mie_argmax (the graph's greedy pick) against torch.argmax: random rows
    of several widths, ties (the first index wins), -inf, and NaN (counted as
    the largest, the first NaN wins)."""
    from moe_engine import _native

    def pick(x):
        out = torch.empty(1, dtype=torch.int64, device="cuda")
        _native.check(_native.lib().mie_argmax(x.data_ptr(), x.numel(), out.data_ptr(), 0,
                                               _native.stream_of(x)), "mie_argmax")
        return int(out)

    g = torch.Generator(device="cuda").manual_seed(3)
    for n in (1, 5, 64, 1000, 1024, 1025, 50257, 200003):
        x = torch.randn(n, generator=g, device="cuda")
        assert pick(x) == int(torch.argmax(x)), n
    x = torch.zeros(50257, device="cuda")
    x[[7, 300, 40000]] = 3.0
    assert pick(x) == 7 == int(torch.argmax(x))
    x = torch.full((4096,), -float("inf"), device="cuda")
    assert pick(x) == 0 == int(torch.argmax(x))
    x = torch.randn(50257, generator=g, device="cuda")
    x[[123, 9000]] = float("nan")
    assert pick(x) == 123 == int(torch.argmax(x))
