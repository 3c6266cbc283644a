"""The whole engine on the GPU against the reference CPU path, on drawn models.

Each case draws a float32 model (head_dim 32-128, 1-6 heads, 1-3 layers,
experts, top-k, expert width, vocabulary), a block size and a prompt, and
builds it once on the CPU.  A copy on the GPU decodes through paged-direct
(block launch plans, the one-call decode step, the head's kept picks); the
CPU model decodes through the contiguous cache, the reference's own system
and the north star's "reference CPU path" (src/moe_engine/model.py:30-58,
226-269).  Both see the same tokens at every position (the CPU's greedy
sequence), and their logits must agree within float32 rounding of the
different summation orders, 1e-4 of the logit scale.  Greedy tokens must be
identical wherever the CPU's top two logits are further apart than ten times
that bound; past the first closer pair the two may legitimately part.
Some cases start past 1024 cached tokens (the five-launch block, split
contexts).
"""

import copy
import os
import random

import pytest
import torch

from conftest import print_case
from moe_engine.model import Model, ModelConfig

pytestmark = pytest.mark.gpu

TOL = 1e-4


def draw(seed):
    rng = random.Random(1000 + seed)
    head_dim = rng.choice([32, 64, 96, 128])
    heads = rng.choice([1, 2, 3, 4, 6])
    experts = rng.choice([2, 4, 8])
    long = rng.random() < 0.25
    return dict(
        cfg=dict(hidden_dim=head_dim * heads, num_heads=heads, num_layers=rng.choice([1, 2, 3]),
                 num_experts=experts, top_k=rng.randint(1, min(experts, 4)), ffn_dim=rng.choice([64, 256, 512]),
                 vocab_size=rng.choice([97, 256, 1000])),
        block_size=rng.choice([1, 4, 16, 32]),
        prompt=rng.randint(1020, 1080) if long else rng.randint(1, 48),
        new_tokens=rng.randint(4, 10),
    )


def stepwise(model, seq, cache, prompt_len):
    """Logits at the last prompt position and at every later position of
    `seq`, the prompt as one prefill and then one token per step."""
    with torch.no_grad():
        rows = [model(seq[:, :prompt_len], cache)[0, -1]]
        for t in range(prompt_len, seq.shape[1] - 1):
            rows.append(model(seq[:, t : t + 1], cache)[0, -1])
    return torch.stack(rows).float().cpu()


# MIE_ENGINE_RANDOM_CASES widens the sweep for a one-off run.
CASES = list(range(int(os.environ.get("MIE_ENGINE_RANDOM_CASES", "16"))))


@pytest.mark.parametrize("seed", CASES)
def test_gpu_paged_direct_matches_the_cpu_contiguous_path(seed):
    c = draw(seed)
    cfg = dict(c["cfg"], max_seq_length=c["prompt"] + c["new_tokens"] + 1)
    print_case("engine vs cpu", seed, cfg, "block", c["block_size"], "prompt", c["prompt"], "new", c["new_tokens"])
    torch.manual_seed(seed)
    cpu = Model(ModelConfig(**cfg)).eval()
    gpu = copy.deepcopy(cpu).to("cuda")
    prompt = torch.randint(0, cfg["vocab_size"], (c["prompt"],), generator=torch.Generator().manual_seed(seed))

    want = cpu.generate(prompt, c["new_tokens"], temperature=0, cache=cpu.new_cache())
    blocks = -(-cfg["max_seq_length"] // c["block_size"])
    alloc = gpu.new_block_allocator(num_blocks=blocks, block_size=c["block_size"], attention_mode="direct")
    cache = alloc.new_cache()
    got = gpu.generate(prompt.cuda(), c["new_tokens"], temperature=0, cache=cache).cpu()
    cache.free()

    ref = stepwise(cpu, want, cpu.new_cache(), c["prompt"])
    cache = alloc.new_cache()
    out = stepwise(gpu, want.cuda(), cache, c["prompt"])
    cache.free()
    scale = ref.abs().amax(dim=-1, keepdim=True).clamp(min=1.0)
    err = ((out - ref).abs() / scale).max().item()
    assert err <= TOL, f"logits differ by {err:.2e} of their scale"

    # Tokens: identical up to the first step whose top two CPU logits are
    # within ten times the bound.
    top2 = ref.topk(2, dim=-1).values
    close = ((top2[:, 0] - top2[:, 1]) / scale[:, 0] <= 10 * TOL).nonzero()
    decided = c["new_tokens"] if len(close) == 0 else int(close[0])
    n = c["prompt"] + decided
    assert torch.equal(got[:, :n], want[:, :n]), f"greedy tokens part before step {decided}"
