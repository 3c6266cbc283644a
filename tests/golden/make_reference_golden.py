"""Write golden vectors from the reference engine's CPU path.

Run once, in the build container where the reference checkout exists:

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_reference_golden.py /root/reference/src

Two things on the paged decode path are pinned only by the reference's own
code: that seeded random initialisation consumes the RNG in the reference's
module order (so a seeded model has the reference's weights), and the greedy
tokens and logits the reference CPU engine produces.  This script builds the
reference Model (src/moe_engine/model.py:501-516) on the CPU, records per-
tensor SHA-256 digests of its seed-0 state dict, then runs its greedy
generate() with the contiguous cache and with a paged cache (block size 16;
on the CPU the reference's paged path is gather + SDPA), and writes small
JSON fixtures next to this file.  Only data is written: digests, token ids,
logits slices and per-step logits checksums.

Configs: the reference's TINY test model (tests/test_parity.py:11), and the
BASELINE config 1 shape (12 layers, d 768, 12 heads x 64, top-2 of 8, vocab
50257) at two expert widths: the reference's fixed 4 * d = 3072
(model.py:487-489) and config 1's 2048.  The reference's MoEFeedForward takes
its width as an argument (model.py:288); only TransformerMoEBlock passes
4 * d.  For the 2048 fixture this script hands TransformerMoEBlock a
MoEFeedForward built at width 2048 (the module-level name is swapped for the
duration of the construction), so every module is still the reference's own
and consumes the RNG in the reference's order.  The fixture's "config" is
this engine's ModelConfig, which names the width (ffn_dim).
"""

import contextlib

import hashlib
import json
import sys
from pathlib import Path

sys.dont_write_bytecode = True
OUT = Path(__file__).resolve().parent


def digest(t):
    return hashlib.sha256(t.detach().contiguous().cpu().numpy().tobytes()).hexdigest()


@contextlib.contextmanager
def expert_width(ffn_dim):
    """Within the block, TransformerMoEBlock builds its MoEFeedForward at
    width ffn_dim instead of 4 * hidden_dim (None: unchanged)."""
    ref_model = sys.modules["moe_engine.model"]
    original = ref_model.MoEFeedForward
    if ffn_dim is not None:
        ref_model.MoEFeedForward = lambda dim, hidden, experts, top_k, **kw: original(dim, ffn_dim, experts, top_k, **kw)
    try:
        yield
    finally:
        ref_model.MoEFeedForward = original


def run_case(name, cfg_kwargs, prompt_len, new_tokens, block_size, torch, Model, ModelConfig, ffn_dim=None):
    torch.manual_seed(0)
    with expert_width(ffn_dim):
        model = Model(ModelConfig(**cfg_kwargs)).eval()
    if ffn_dim is not None:
        assert all(b.moe.hidden_dim == ffn_dim and b.moe.experts[0].net[0].out_features == ffn_dim
                   for b in model.MoEBlocks)
    state = {k: digest(v) for k, v in model.state_dict().items()}
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg_kwargs["vocab_size"], (prompt_len,), generator=gen)
    tokens = {}
    tokens["contiguous"] = model.generate(prompt, max_new_tokens=new_tokens, temperature=0)[0].tolist()
    num_blocks = -(-cfg_kwargs["max_seq_length"] // block_size)
    allocator = model.new_block_allocator(num_blocks=num_blocks, block_size=block_size, attention_mode="gather")
    cache = allocator.new_cache()
    tokens["paged_gather"] = model.generate(prompt, max_new_tokens=new_tokens, temperature=0, cache=cache)[0].tolist()
    cache.free()
    # Logits of every decode step through the contiguous cache.
    seq = torch.tensor(tokens["contiguous"][:-1])[None]
    cache = model.new_cache()
    steps = []
    with torch.no_grad():
        steps.append(model(seq[:, :prompt_len], cache)[0, -1])
        for t in range(prompt_len, seq.shape[1]):
            steps.append(model(seq[:, t : t + 1], cache)[0, -1])
    logits = torch.stack(steps).double()
    fixture = {
        "config": cfg_kwargs if ffn_dim is None else dict(cfg_kwargs, ffn_dim=ffn_dim),
        "seed": 0,
        "prompt_generator_seed": 0,
        "prompt": prompt.tolist(),
        "new_tokens": new_tokens,
        "block_size": block_size,
        "state_dict_sha256": state,
        "tokens": tokens,
        "logits_first_64": [row[:64].tolist() for row in logits],
        "logits_sum": logits.sum(dim=1).tolist(),
        "logits_sumsq": (logits * logits).sum(dim=1).tolist(),
        "logits_argmax": logits.argmax(dim=1).tolist(),
        "torch_version": torch.__version__,
    }
    (OUT / f"reference_{name}.json").write_text(json.dumps(fixture))
    print(name, "tokens", len(tokens["contiguous"]), "paged==contiguous", tokens["paged_gather"] == tokens["contiguous"])


def main():
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, ref_src)
    import torch
    from moe_engine.model import Model, ModelConfig  # the reference's package

    assert Path(sys.modules["moe_engine"].__file__).resolve().is_relative_to(Path(ref_src).resolve())
    torch.set_num_threads(8)
    tiny = dict(max_seq_length=32, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)
    run_case("tiny", tiny, 8, 12, 4, torch, Model, ModelConfig)
    e2e = dict(max_seq_length=1024, vocab_size=50257, num_layers=12, hidden_dim=768, num_heads=12,
               num_experts=8, top_k=2)
    run_case("config1_ffn3072", e2e, 32, 64, 16, torch, Model, ModelConfig)
    run_case("config1", e2e, 32, 64, 16, torch, Model, ModelConfig, ffn_dim=2048)


if __name__ == "__main__":
    main()
