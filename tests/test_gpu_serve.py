"""One request through the server with --cache paged --paged-attention direct on the GPU."""

import pytest
import torch
from fastapi.testclient import TestClient

from moe_engine import serve
from moe_engine.model import Model, ModelConfig

pytestmark = pytest.mark.gpu


def test_paged_direct_request_on_gpu_matches_contiguous_and_frees_blocks():
    torch.manual_seed(0)
    serve.model = Model(ModelConfig(max_seq_length=64, vocab_size=512, num_layers=2, hidden_dim=64,
                                    num_heads=4, num_experts=4, top_k=2)).to("cuda").eval()
    serve.device = "cuda"
    client = TestClient(serve.app, raise_server_exceptions=True)
    payload = {"prompt_ids": [7, 300, 42, 9], "max_new_tokens": 12, "temperature": 0}
    serve.cache_mode, serve.allocator = "contiguous", None
    want = client.post("/generate", json=payload).json()["token_ids"]
    serve.cache_mode = "paged"
    serve.allocator = serve.model.new_block_allocator(num_blocks=4, block_size=16, attention_mode="direct")
    got = client.post("/generate", json=payload).json()["token_ids"]
    assert got == want
    assert sorted(serve.allocator.free_blocks) == list(range(4))
    serve.graph_generator = None


def test_decode_graph_requests_match_eager_and_reuse_one_capture():
    """--decode-graph: greedy requests replay one captured decode step; the
    tokens equal the eager paged path's for several requests (different
    prompts and lengths, one capture), and sampling requests still take
    Model.generate."""
    torch.manual_seed(0)
    serve.model = Model(ModelConfig(max_seq_length=64, vocab_size=512, num_layers=2, hidden_dim=64,
                                    num_heads=4, num_experts=4, top_k=2)).to("cuda").eval()
    serve.device = "cuda"
    serve.cache_mode = "paged"
    serve.allocator = serve.model.new_block_allocator(num_blocks=4, block_size=16, attention_mode="direct")
    serve.graph_generator = None
    client = TestClient(serve.app, raise_server_exceptions=True)
    requests = [([7, 300, 42, 9], 12), ([1, 2, 3], 30), ([500] * 20, 40), ([11], 5)]
    eager = [client.post("/generate", json={"prompt_ids": p, "max_new_tokens": n, "temperature": 0}).json()
             for p, n in requests]
    serve.enable_decode_graph()
    graphed = [client.post("/generate", json={"prompt_ids": p, "max_new_tokens": n, "temperature": 0}).json()
               for p, n in requests]
    try:
        for e, g in zip(eager, graphed):
            assert g["token_ids"] == e["token_ids"] and g["finish_reason"] == e["finish_reason"]
        decoder = serve.graph_generator.decoder
        assert decoder is not None and decoder.graph is not None
        # A request of T tokens takes T - 1 decode steps; the first step of
        # the first request runs eagerly and captures, every other one replays.
        assert decoder.replays == sum(len(r["token_ids"]) - 1 for r in graphed) - 1
        sampled = client.post("/generate", json={"prompt_ids": [7, 8], "max_new_tokens": 4, "temperature": 1.0})
        assert sampled.status_code == 200 and len(sampled.json()["token_ids"]) <= 4
        assert sorted(serve.allocator.free_blocks) == list(range(4))
    finally:
        serve.graph_generator = None
