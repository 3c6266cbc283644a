"""The HTTP server and its cache switches (CPU), mirroring the reference's
tests/test_serve.py: CLI defaults, paged blocks returned after success, after
a validation failure and after an exception, finish reasons, and one request
at a time."""

import threading
import time
from concurrent.futures import ThreadPoolExecutor

import pytest
import torch
from fastapi.testclient import TestClient

from moe_engine import serve
from moe_engine.model import KVCache, Model, ModelConfig, PagedKVCache

TINY_SERVE = dict(max_seq_length=32, vocab_size=50257, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)


@pytest.fixture()
def client():
    torch.manual_seed(0)
    serve.model = Model(ModelConfig(**TINY_SERVE)).eval()
    serve.cache_mode = "contiguous"
    serve.allocator = None
    serve.device = "cpu"
    return TestClient(serve.app, raise_server_exceptions=False)


@pytest.fixture()
def paged_client(client):
    serve.cache_mode = "paged"
    serve.allocator = serve.model.new_block_allocator(num_blocks=2, block_size=16, attention_mode="gather")
    return client


def test_cli_defaults_and_paged_switch():
    defaults = serve.build_parser().parse_args([])
    assert (defaults.cache, defaults.paged_attention, defaults.moe, defaults.device) == (
        "contiguous", "auto", "auto", "cpu")
    paged = serve.build_parser().parse_args(["--cache", "paged", "--paged-attention", "direct"])
    assert paged.cache == "paged" and paged.paged_attention == "direct"
    with pytest.raises(SystemExit):
        serve.build_parser().parse_args(["--paged-attention", "turbo"])


def test_generate_uses_contiguous_cache_by_default(client):
    seen = []
    real = serve.model.generate

    def spy(*args, **kwargs):
        seen.append(kwargs["cache"])
        return real(*args, **kwargs)

    serve.model.generate = spy
    resp = client.post("/generate", json={"prompt": "hello", "max_new_tokens": 4})
    assert resp.status_code == 200
    assert isinstance(seen[0], KVCache) and not hasattr(seen[0], "free")


def test_paged_cache_frees_blocks_after_success(paged_client):
    seen = []
    real = serve.model.generate

    def spy(*args, **kwargs):
        seen.append(kwargs["cache"])
        return real(*args, **kwargs)

    serve.model.generate = spy
    resp = paged_client.post("/generate", json={"prompt": "hello", "max_new_tokens": 4})
    assert resp.status_code == 200
    assert isinstance(seen[0], PagedKVCache)
    assert len(serve.allocator.free_blocks) == 2


def test_prompt_ids_are_accepted(paged_client):
    resp = paged_client.post("/generate", json={"prompt_ids": [1, 2, 3], "max_new_tokens": 3, "temperature": 0})
    assert resp.status_code == 200
    body = resp.json()
    assert body["new_tokens"] == len(body["token_ids"]) <= 3


def test_finish_reason_length_and_context_limit(client):
    resp = client.post("/generate", json={"prompt_ids": [5, 6], "max_new_tokens": 2, "temperature": 0})
    assert resp.json()["finish_reason"] == "length"
    resp = client.post("/generate", json={"prompt_ids": [5, 6], "max_new_tokens": 64, "temperature": 0})
    body = resp.json()
    if body["finish_reason"] != "eos":
        assert body["finish_reason"] == "context_limit"
        assert body["new_tokens"] == TINY_SERVE["max_seq_length"] - 2 + 1


def test_over_length_prompt_returns_400(client):
    resp = client.post("/generate", json={"prompt_ids": list(range(40)), "max_new_tokens": 4})
    assert resp.status_code == 400 and "context" in resp.json()["detail"]


def test_invalid_fields_return_422(client):
    for payload in (
        {"prompt": "", "max_new_tokens": 4},
        {"prompt": "hi", "max_new_tokens": 0},
        {"prompt": "hi", "max_new_tokens": -3},
        {"prompt": "hi", "temperature": -1},
    ):
        assert client.post("/generate", json=payload).status_code == 422, payload


def test_paged_validation_failure_does_not_allocate_blocks(paged_client):
    assert paged_client.post("/generate", json={"prompt": "", "max_new_tokens": 4}).status_code == 422
    assert len(serve.allocator.free_blocks) == 2


def test_paged_blocks_freed_when_generation_raises(paged_client):
    def broken(*args, **kwargs):
        raise RuntimeError("boom")

    serve.model.generate = broken
    resp = paged_client.post("/generate", json={"prompt": "hello", "max_new_tokens": 4})
    assert resp.status_code == 500
    assert len(serve.allocator.free_blocks) == 2


def test_concurrent_requests_are_serialized(client):
    lock = threading.Lock()
    active = max_active = 0

    def slow(token_ids, *args, **kwargs):
        nonlocal active, max_active
        with lock:
            active += 1
            max_active = max(max_active, active)
        time.sleep(0.1)
        with lock:
            active -= 1
        return token_ids.unsqueeze(0)

    serve.model.generate = slow
    payload = {"prompt": "hello", "max_new_tokens": 4}
    with ThreadPoolExecutor(2) as pool:
        second = TestClient(serve.app, raise_server_exceptions=False)
        responses = list(pool.map(lambda c: c.post("/generate", json=payload), [client, second]))
    assert all(r.status_code == 200 for r in responses)
    assert max_active == 1


def test_byte_tokenizer_round_trips_text():
    tok = serve.ByteTokenizer()
    assert tok.decode(tok.encode("héllo")) == "héllo"
