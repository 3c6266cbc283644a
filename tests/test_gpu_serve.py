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
