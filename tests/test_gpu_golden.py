"""Greedy decode on the GPU through the paged-direct path against the
reference engine's CPU tokens (tests/golden/reference_*.json).

Tokens must be identical.  Logits differ from the reference CPU run only by
GPU GEMM rounding (hipBLASLt vs the CPU BLAS); they are checked within a bound
far below the logit scale (|logit| ~ 28 at d 768), with identical argmax.
"""

import pytest
import torch

from conftest import print_case
from test_golden import build, check_logits, load, step_logits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,atol", [("tiny", 1e-4), ("config1_ffn3072", 2e-2)])
@pytest.mark.parametrize("mode", ["direct", "gather"])
def test_gpu_paged_tokens_match_reference_cpu(name, atol, mode):
    print_case("golden", name, mode)
    fixture = load(name)
    model = build(fixture).to("cuda")
    prompt = torch.tensor(fixture["prompt"], device="cuda")
    bs = fixture["block_size"]
    allocator = model.new_block_allocator(-(-model.max_seq_length // bs), bs, attention_mode=mode)
    cache = allocator.new_cache()
    tokens = model.generate(prompt, fixture["new_tokens"], temperature=0, cache=cache)[0].tolist()
    cache.free()
    assert tokens == fixture["tokens"]["paged_gather"]
    cache = allocator.new_cache()
    check_logits(step_logits(model, fixture["tokens"]["contiguous"], len(prompt), cache), fixture, atol)
    cache.free()
