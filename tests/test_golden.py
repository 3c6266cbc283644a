"""The engine against golden vectors written by the reference engine itself.

tests/golden/make_reference_golden.py ran the reference's Model on the CPU
(seed-0 random init, greedy decode, contiguous and paged caches; the TINY
test model and BASELINE config 1's shape at expert widths 3072 and 2048,
config 1's own) and stored
per-tensor SHA-256 digests of the state dict, the token ids and logits
slices.  Here the same construction and decode run through this engine on the
CPU: the weights must be bit-identical (the random-init order is the
reference's), the tokens identical, and the logits equal to float32 rounding.
The GPU counterparts are in tests/test_gpu_golden.py.
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from moe_engine.model import Model, ModelConfig

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return json.loads((GOLDEN / f"reference_{name}.json").read_text())


def build(fixture):
    torch.manual_seed(fixture["seed"])
    return Model(ModelConfig(**fixture["config"])).eval()


def digest(t):
    return hashlib.sha256(t.detach().contiguous().cpu().numpy().tobytes()).hexdigest()


def step_logits(model, tokens, prompt_len, cache):
    seq = torch.tensor(tokens[:-1])[None].to(model.token_embedding.weight.device)
    out = []
    with torch.no_grad():
        out.append(model(seq[:, :prompt_len], cache)[0, -1])
        for t in range(prompt_len, seq.shape[1]):
            out.append(model(seq[:, t : t + 1], cache)[0, -1])
    return torch.stack(out).double().cpu()


def check_logits(logits, fixture, atol):
    """First 64 logits of every step within `atol`, identical argmax, and the
    per-step sum over the vocabulary within 4 * atol * sqrt(vocab) (independent
    rounding errors add in quadrature)."""
    np.testing.assert_allclose(np.array([row[:64].tolist() for row in logits]), fixture["logits_first_64"], rtol=0, atol=atol)
    assert logits.argmax(dim=1).tolist() == fixture["logits_argmax"]
    sum_atol = 4 * atol * logits.shape[1] ** 0.5
    np.testing.assert_allclose(logits.sum(dim=1).numpy(), fixture["logits_sum"], rtol=0, atol=sum_atol)


FIXTURES = ["tiny", "config1_ffn3072", "config1"]


@pytest.mark.parametrize("name", FIXTURES)
def test_seed0_weights_are_the_reference_weights(name):
    fixture = load(name)
    model = build(fixture)
    state = {k: digest(v) for k, v in model.state_dict().items()}
    assert set(state) == set(fixture["state_dict_sha256"])
    mismatched = [k for k in state if state[k] != fixture["state_dict_sha256"][k]]
    assert not mismatched, f"{len(mismatched)} tensors differ, first {mismatched[:3]}"


def test_config1_fixture_is_baseline_config1():
    """reference_config1.json is BASELINE config 1 itself: FFN 2048, 32-token
    prompt, 64 greedy tokens, block 16."""
    fixture = load("config1")
    cfg = fixture["config"]
    assert (cfg["num_layers"], cfg["hidden_dim"], cfg["num_heads"], cfg["num_experts"], cfg["top_k"],
            cfg["ffn_dim"], cfg["vocab_size"]) == (12, 768, 12, 8, 2, 2048, 50257)
    assert (len(fixture["prompt"]), fixture["new_tokens"], fixture["block_size"]) == (32, 64, 16)
    assert any(k.endswith("experts.0.net.0.weight") for k in fixture["state_dict_sha256"])


@pytest.mark.parametrize("name", FIXTURES)
def test_cpu_greedy_tokens_and_logits_match_reference(name):
    fixture = load(name)
    model = build(fixture)
    prompt = torch.tensor(fixture["prompt"])
    n = fixture["new_tokens"]
    assert model.generate(prompt, n, temperature=0)[0].tolist() == fixture["tokens"]["contiguous"]
    bs = fixture["block_size"]
    allocator = model.new_block_allocator(-(-model.max_seq_length // bs), bs, attention_mode="gather")
    cache = allocator.new_cache()
    assert model.generate(prompt, n, temperature=0, cache=cache)[0].tolist() == fixture["tokens"]["paged_gather"]
    cache.free()
    check_logits(step_logits(model, fixture["tokens"]["contiguous"], len(prompt), model.new_cache()), fixture, 1e-5)
