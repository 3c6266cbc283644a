"""The generation server on the CPU, checked against the cache-switch
contract: the flags pick the cache and the paged attention mode, every
request's cache is returned whatever happens to the request, results do not
depend on the cache chosen, a forced 'direct' that cannot run fails before it
touches the pool, and the single pool serves one request at a time.

Servers are built the way `python -m moe_engine.serve` builds them
(serve.configure on parsed flags, a small random-init model from --config),
and every cache a request opens is recorded by a ledger around the server's
own new/release hooks.
"""

import json
import queue
import threading

import pytest
from fastapi.testclient import TestClient

from moe_engine import serve
from moe_engine.model import KVCache, PagedKVCache

# Small enough for the CPU, with the GPT-2 vocabulary the byte tokenizer's ids fall in.
SMALL = dict(max_seq_length=48, vocab_size=50257, num_layers=2, hidden_dim=32, num_heads=4, num_experts=4, top_k=2)


class Ledger:
    """Wraps serve.new_request_cache / release_request_cache: which caches
    were opened, and which of them were handed back."""

    def __init__(self, monkeypatch):
        self.opened, self.released = [], []
        new, release = serve.new_request_cache, serve.release_request_cache

        def tracked_new():
            cache = new()
            self.opened.append(cache)
            return cache

        def tracked_release(cache):
            self.released.append(cache)
            release(cache)

        monkeypatch.setattr(serve, "new_request_cache", tracked_new)
        monkeypatch.setattr(serve, "release_request_cache", tracked_release)

    def balanced(self) -> bool:
        return [id(c) for c in self.opened] == [id(c) for c in self.released]


def start(monkeypatch, *flags, config=SMALL):
    """serve.configure on these flags (no checkpoint file, so the model is
    random-initialised from --config at seed 0); returns (client, ledger)."""
    args = serve.build_parser().parse_args(
        ["--checkpoint", "/nonexistent/checkpoint.pt", "--config", json.dumps(config), "--device", "cpu", *flags])
    serve.configure(args)
    return TestClient(serve.app, raise_server_exceptions=False), Ledger(monkeypatch)


def pool_is_full():
    return sorted(serve.allocator.free_blocks) == list(range(serve.allocator.num_blocks))


def greedy(client, ids, n):
    return client.post("/generate", json={"prompt_ids": ids, "max_new_tokens": n, "temperature": 0})


def test_flags_select_the_cache_and_the_paged_attention_mode(monkeypatch):
    defaults = serve.build_parser().parse_args([])
    assert (defaults.cache, defaults.paged_attention, defaults.device) == ("contiguous", "auto", "cpu")
    for flags, cache_type, mode in (
        ((), KVCache, None),
        (("--cache", "paged"), PagedKVCache, "auto"),
        (("--cache", "paged", "--paged-attention", "gather"), PagedKVCache, "gather"),
    ):
        client, ledger = start(monkeypatch, *flags)
        assert greedy(client, [3, 1, 4], 2).status_code == 200
        (cache,) = ledger.opened
        assert type(cache) is cache_type and getattr(cache, "attention_mode", None) == mode
        if mode is not None:
            # One maximum-length request: ceil(48 / 16) blocks of 16, all back in the pool.
            assert (serve.allocator.num_blocks, serve.allocator.block_size) == (3, 16) and pool_is_full()
        assert ledger.balanced()
    with pytest.raises(SystemExit):
        serve.build_parser().parse_args(["--cache", "ring"])


def test_greedy_tokens_do_not_depend_on_the_cache(monkeypatch):
    ids = [17, 4, 999, 23, 5]
    answers = []
    for flags in ((), ("--cache", "paged", "--paged-attention", "gather"), ("--cache", "paged")):
        client, _ = start(monkeypatch, *flags)
        body = greedy(client, ids, 10).json()
        answers.append((body["token_ids"], body["finish_reason"]))
    assert answers[0] == answers[1] == answers[2]


def test_forced_direct_on_the_cpu_fails_before_touching_the_pool(monkeypatch):
    """'direct' needs the HIP kernel; on the CPU the request fails (500) and
    the pool is exactly as it was: no block was taken, the cache was handed
    back."""
    client, ledger = start(monkeypatch, "--cache", "paged", "--paged-attention", "direct")
    resp = greedy(client, [1, 2, 3], 4)
    assert resp.status_code == 500
    assert pool_is_full() and ledger.balanced() and len(ledger.opened) == 1
    assert ledger.opened[0].block_table == [] and ledger.opened[0].position == 0


@pytest.mark.parametrize("payload,status", [
    ({"max_new_tokens": 3}, 422),                                   # no prompt at all
    ({"prompt_ids": [], "prompt": ""}, 422),
    ({"prompt": "abc", "max_new_tokens": 0}, 422),
    ({"prompt": "abc", "temperature": -0.5}, 422),
    ({"prompt_ids": [50257]}, 400),                                  # one past the vocabulary
    ({"prompt_ids": [-1, 2]}, 400),
    ({"prompt_ids": [7] * 49}, 400),                                 # longer than the 48-token context
])
def test_rejected_requests_open_no_cache(monkeypatch, payload, status):
    client, ledger = start(monkeypatch, "--cache", "paged")
    resp = client.post("/generate", json=payload)
    assert resp.status_code == status, resp.text
    assert ledger.opened == [] and pool_is_full()


def test_a_failing_generation_still_returns_its_blocks(monkeypatch):
    client, ledger = start(monkeypatch, "--cache", "paged", "--paged-attention", "gather")
    real = serve.model.generate

    def fail_midway(token_ids, max_new_tokens, **kwargs):
        real(token_ids, max_new_tokens=2, temperature=0, cache=kwargs["cache"])  # takes a block
        assert not pool_is_full()
        raise MemoryError("out of memory in the middle of a request")

    monkeypatch.setattr(serve.model, "generate", fail_midway)
    assert greedy(client, [9, 8, 7], 5).status_code == 500
    assert ledger.balanced() and pool_is_full()


def test_finish_reasons_follow_the_generated_length(monkeypatch):
    client, _ = start(monkeypatch, "--cache", "paged")
    body = greedy(client, [5, 6, 7], 3).json()
    if body["finish_reason"] != "eos":
        assert body["finish_reason"] == "length" and body["new_tokens"] == 3
    # Asking for more than the context holds: the model stops at its context
    # (one token past the last position that fits), unless EOS comes first.
    body = greedy(client, [5, 6, 7], 500).json()
    assert body["new_tokens"] == len(body["token_ids"])
    if body["finish_reason"] != "eos":
        assert body["finish_reason"] == "context_limit" and 3 + body["new_tokens"] == SMALL["max_seq_length"] + 1


def test_the_pool_serves_one_request_at_a_time(monkeypatch):
    """Handshake, not timing: the first request parks inside generation until
    the test lets it go; meanwhile a second request must not get in.  Once
    released, the second one runs."""
    client, _ = start(monkeypatch, "--cache", "paged")
    inside = queue.Queue()
    release_first = threading.Event()

    def parked(token_ids, max_new_tokens, **kwargs):
        inside.put(token_ids.tolist())
        if len(token_ids) == 1:
            assert release_first.wait(timeout=30)
        return token_ids.unsqueeze(0)

    monkeypatch.setattr(serve.model, "generate", parked)
    results = {}
    first = threading.Thread(target=lambda: results.setdefault("first", greedy(client, [1], 2)))
    second = threading.Thread(target=lambda: results.setdefault("second", greedy(client, [2, 2], 2)))
    first.start()
    assert inside.get(timeout=30) == [1]
    second.start()
    with pytest.raises(queue.Empty):
        inside.get(timeout=0.5)  # the second request is held at the lock
    release_first.set()
    assert inside.get(timeout=30) == [2, 2]
    first.join(30)
    second.join(30)
    assert results["first"].status_code == results["second"].status_code == 200
    assert pool_is_full()


def test_byte_tokenizer_is_lossless_for_utf8():
    tok = serve.ByteTokenizer()
    text = "paged KV — ½ µs"
    assert tok.decode(tok.encode(text)) == text and max(tok.encode(text)) < 256
