"""Synchronous HTTP generation server with the reference's cache switches.

    python -m moe_engine.serve --device cuda --cache paged --paged-attention direct

Drop-in for the reference's scripts/serve.py: the same flags
(`--cache {contiguous,paged}`, `--paged-attention {auto,direct,gather}`,
`--moe {auto,direct,reference}`, `--device`), the same single-request lock, a
paged pool sized for one maximum-length request (ceil(max_seq_length / 16)
blocks, scripts/serve.py:147-155), blocks returned in `finally`
(scripts/serve.py:103-115), and the same response fields.

One addition: `--decode-graph` (paged cache on a ROCm device) serves greedy
requests (temperature 0) by replaying one captured HIP graph per decode step
(moe_engine.graphs); the graph is captured on the first such request and
reused by every later one.  Other requests take Model.generate.

Differences forced by this environment:
  * --checkpoint loads the reference's checkpoint format
    ({"model", "model_config", "step", ...}, read with weights_only=True,
    src/moe_engine/checkpoint.py:20-31) when the file exists; otherwise the
    model is random-initialised from --seed with --config (JSON ModelConfig
    fields, default the miniMoE shape of BASELINE config 1).
  * Text is tokenized with tiktoken's GPT-2 encoding when tiktoken is
    installed (as the reference does); without it a byte-level stand-in maps
    each UTF-8 byte to the token id of the same value.  Requests may also send
    `prompt_ids` directly.
"""

import argparse
import json
import threading
import time
from pathlib import Path
from typing import List, Optional

import torch
from fastapi import FastAPI, HTTPException
from pydantic import BaseModel, Field, model_validator

from moe_engine.model import Model, ModelConfig

DEFAULT_CONFIG = dict(max_seq_length=1024, vocab_size=50257, num_layers=12, hidden_dim=768, num_heads=12,
                      num_experts=8, top_k=2, ffn_dim=2048)
BLOCK_SIZE = 16


class ByteTokenizer:
    """UTF-8 bytes as token ids 0-255 (stand-in when tiktoken is absent)."""

    name = "bytes"

    def encode(self, text: str) -> List[int]:
        return list(text.encode("utf-8"))

    def decode(self, ids: List[int]) -> str:
        return bytes(i for i in ids if 0 <= i < 256).decode("utf-8", errors="replace")


def make_tokenizer():
    try:
        import tiktoken

        enc = tiktoken.get_encoding("gpt2")
        enc.name = "gpt2"
        return enc
    except Exception:  # tiktoken or its encoding files unavailable
        return ByteTokenizer()


class GenerateRequest(BaseModel):
    prompt: str = Field("", max_length=1_000_000)
    prompt_ids: Optional[List[int]] = None
    max_new_tokens: int = Field(64, ge=1)
    temperature: float = Field(0.8, ge=0.0, allow_inf_nan=False)

    @model_validator(mode="after")
    def _needs_a_prompt(self):
        if not self.prompt and not self.prompt_ids:
            raise ValueError("prompt or prompt_ids must be non-empty")
        return self


app = FastAPI(title="moe-engine")
enc = make_tokenizer()
model = None  # set by main() or by tests
cache_mode = "contiguous"
allocator = None  # shared paged pool, paged mode only
graph_generator = None  # --decode-graph: greedy requests replay a captured decode step
device = "cpu"
# The pool holds one max-length sequence, so requests run one at a time.
generate_lock = threading.Lock()


def new_request_cache():
    if cache_mode == "contiguous":
        return model.new_cache()
    return allocator.new_cache()


def release_request_cache(cache) -> None:
    if cache_mode == "paged":
        cache.free()


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(description="miniMoE generation server")
    parser.add_argument("--checkpoint", default="checkpoints/minimoe_sft.pt")
    parser.add_argument("--config", default=None, help="JSON ModelConfig fields for random init")
    parser.add_argument("--seed", type=int, default=0, help="random-init seed when no checkpoint exists")
    parser.add_argument("--port", type=int, default=8000)
    parser.add_argument("--host", default="127.0.0.1")
    parser.add_argument("--device", choices=["auto", "cpu", "cuda"], default="cpu",
                        help="execution device (default: CPU; the GPU needs explicit selection)")
    parser.add_argument("--cache", choices=["contiguous", "paged"], default="contiguous",
                        help="KV cache used for serving")
    parser.add_argument("--paged-attention", choices=["auto", "direct", "gather"], default="auto",
                        help="paged cache only: direct HIP kernel, gather oracle, or automatic fallback")
    parser.add_argument("--moe", choices=["auto", "direct", "reference"], default="auto",
                        help="MoE decode mode")
    parser.add_argument("--decode-graph", action="store_true",
                        help="paged cache on a GPU: replay greedy decode steps from a captured HIP graph")
    return parser


def load_model(args, device_name):
    path = Path(args.checkpoint)
    if path.exists():
        checkpoint = torch.load(path, map_location="cpu", weights_only=True)
        net = Model(ModelConfig(**checkpoint["model_config"]))
        net.load_state_dict(checkpoint["model"])
        meta = {"source": str(path), "step": checkpoint.get("step")}
    else:
        cfg = dict(DEFAULT_CONFIG, **(json.loads(args.config) if args.config else {}))
        torch.manual_seed(args.seed)
        net = Model(ModelConfig(**cfg))
        meta = {"source": f"random init, seed {args.seed}", "step": None}
    return net.to(device_name).eval(), meta


@app.post("/generate")
def generate(req: GenerateRequest):
    ids = req.prompt_ids if req.prompt_ids else enc.encode(req.prompt)
    if len(ids) == 0:
        raise HTTPException(status_code=400, detail="prompt tokenizes to zero tokens")
    if len(ids) > model.max_seq_length:
        raise HTTPException(
            status_code=400,
            detail=f"prompt is {len(ids)} tokens; the model's context is {model.max_seq_length}",
        )
    vocab = model.config.vocab_size
    if any(not 0 <= i < vocab for i in ids):
        raise HTTPException(status_code=400, detail=f"token ids must lie in [0, {vocab})")
    prompt_ids = torch.tensor(ids, device=device)

    with generate_lock:
        start = time.perf_counter()
        if graph_generator is not None and req.temperature == 0:
            out = graph_generator.generate(prompt_ids, req.max_new_tokens)
        else:
            cache = new_request_cache()
            try:
                out = model.generate(prompt_ids, max_new_tokens=req.max_new_tokens, temperature=req.temperature,
                                     top_k=50, cache=cache)
            finally:
                release_request_cache(cache)
        elapsed = time.perf_counter() - start

    new_ids = out[0, len(ids):].tolist()
    if len(new_ids) == req.max_new_tokens:
        finish_reason = "length"
    elif len(ids) + len(new_ids) > model.max_seq_length:
        finish_reason = "context_limit"
    else:
        finish_reason = "eos"
    return {
        "text": enc.decode(new_ids),
        "token_ids": new_ids,
        "new_tokens": len(new_ids),
        "finish_reason": finish_reason,
        "tokens_per_sec": round(len(new_ids) / elapsed, 1) if elapsed > 0 else None,
    }


def enable_decode_graph() -> None:
    """Serve greedy requests through a GraphedGenerator on its own paged cache
    (a second pool of the same size, so ordinary requests keep theirs)."""
    global graph_generator
    from moe_engine.graphs import GraphedGenerator

    if cache_mode != "paged" or allocator is None or not allocator.on_device:
        raise SystemExit("--decode-graph needs --cache paged on a GPU")
    pool = model.new_block_allocator(num_blocks=allocator.num_blocks, block_size=allocator.block_size,
                                     attention_mode=allocator.attention_mode)
    graph_generator = GraphedGenerator(model, pool.new_cache())


def configure(args) -> dict:
    """Set the server's model, device, cache switch and pool from parsed
    command-line arguments (scripts/serve.py:139-160); returns the model's
    provenance."""
    global model, cache_mode, allocator, device, graph_generator
    device = ("cuda" if torch.cuda.is_available() else "cpu") if args.device == "auto" else args.device
    if device == "cuda" and not torch.cuda.is_available():
        raise SystemExit("a GPU was requested but none is available")
    model, meta = load_model(args, device)
    model.set_moe_mode(args.moe)
    cache_mode = args.cache
    allocator = None
    if cache_mode == "paged":
        num_blocks = -(-model.max_seq_length // BLOCK_SIZE)
        allocator = model.new_block_allocator(num_blocks=num_blocks, block_size=BLOCK_SIZE,
                                              attention_mode=args.paged_attention)
    graph_generator = None
    if args.decode_graph:
        enable_decode_graph()
    return meta


def main(argv=None) -> None:
    args = build_parser().parse_args(argv)
    meta = configure(args)
    print(f"Serving {meta['source']} on {device} with {cache_mode} KV cache "
          f"({args.paged_attention} attention), {args.moe} MoE, tokenizer {enc.name}")
    import uvicorn

    uvicorn.run(app, host=args.host, port=args.port)


if __name__ == "__main__":
    main()
