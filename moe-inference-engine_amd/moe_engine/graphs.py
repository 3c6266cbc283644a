"""Whole decode steps captured as HIP graphs (paged-direct cache, greedy).

One greedy decode step is captured once and replayed for every later token:
the embedding (mie_embed), every layer's five launches (QKV into the pool,
paged decode, out_proj with the residual, the two MoE launches), and the head
(mie_lm_head: final norm, LM head, greedy pick).  Eagerly the host spends
longer issuing those launches than the GPU spends running them.

Everything that changes from step to step lives on the device: the token fed
in (the previous step's pick, which the graph writes into a fixed buffer), the
position of the new token and the context length (advanced by the graph's
last launch).  The paged cache is put in graph mode (PagedKVCache.graph_pos /
graph_ctx), so the append and the decode read those device values, and the
launches are planned for a bound on the position (FIRST_CONTEXT_BOUND and
its doublings, up to the model's capacity; partition_tokens 0 lets the
library choose the decode's form).  A step past the bound is captured
again.  The host keeps only the block bookkeeping: before each replay it
reserves the block the new token needs (one block id appended to the device
table every block_size tokens); the replay itself never allocates.

Only greedy decoding (temperature 0) over a PagedKVCache whose attention can
run the direct kernel, with the fused MoE (float32 or bfloat16), is captured; everything
else uses Model.generate.
"""

import torch

from moe_engine import paged_attention, projection
from moe_engine.model import _TENSOR_EPOCH, EOS_TOKEN_ID, PagedKVCache

# A captured step serves positions up to a bound: the smallest of 127, 255,
# 511, ... (contexts of 128, 256, 512, ... tokens) that holds the position it
# was captured at, capped by the model's context and the pool.  The launches are
# planned for that bound (the fused attention takes 4 waves per workgroup up to
# 128 tokens and 8 beyond), so a step past it is captured again for the next
# bound, and a sequence starting below it (a later request) is captured again
# for its own.
FIRST_CONTEXT_BOUND = 128


class GraphedDecoder:
    """Replays one greedy decode step of `model` over `cache` as a HIP graph.

    The cache must already hold the prompt (cache.position > 0).  prime(token)
    sets the token to decode next; each step() appends it, attends, and leaves
    the next greedy token in `next_token` (and the logits in `logits`).  Both
    are the decoder's buffers, overwritten by the next step: clone what must
    outlive it.
    """

    def __init__(self, model, cache, partition_tokens=0):
        if not isinstance(cache, PagedKVCache) or cache.attention_mode == "gather":
            raise ValueError("graph decode needs a paged cache whose attention mode is 'auto' or 'direct'")
        weight = model.token_embedding.weight
        if not paged_attention.is_supported(weight, model.config.head_dim):
            raise RuntimeError("graph decode needs the direct paged kernel (ROCm device, float32 or bfloat16)")
        for block in model.MoEBlocks:
            # The PyTorch MoE path selects rows with data-dependent shapes (a
            # host synchronization), which a graph cannot hold.
            moe = block.moe
            if moe.mode == "reference" or not moe.direct_configuration_supported(1):
                raise RuntimeError("graph decode needs the fused MoE decode kernel (mode 'auto' or 'direct', "
                                   "float32 or bfloat16)")
        if not projection.supported(model.config.hidden_dim, weight.dtype):
            raise RuntimeError("graph decode needs the HIP LM head for this width and dtype")
        if cache.position <= 0:
            raise ValueError("prefill the cache before building a graphed decoder")
        self.model = model
        self.cache = cache
        device = weight.device
        self.token = torch.zeros(1, 1, dtype=torch.long, device=device)
        # The new token's position and the context length, advanced together
        # by the pick's launch at the end of each step.
        self.counters = torch.zeros(2, dtype=torch.int32, device=device)
        self.pos = self.counters[0:1]
        self.ctx = self.counters[1:2]
        vocab = model.output_projection.weight.shape[0]
        self._logits = torch.empty(1, vocab, dtype=weight.dtype, device=device)
        self._head_ws = torch.empty(projection.head_workspace_bytes(vocab), dtype=torch.uint8, device=device)
        self.partition_tokens = partition_tokens
        self.bound = None  # the largest position the captured step serves
        self.captures = 0
        self.graph = None
        self._graph_out = None
        self._plans = None
        self._epoch = None  # _TENSOR_EPOCH at capture
        self.logits = None
        self.next_token = None
        self.replays = 0

    def position_bound(self, position):
        """The largest position a step captured at `position` serves: the
        context bound of FIRST_CONTEXT_BOUND doubled until it holds the
        position, at most the model's context or the pool's capacity."""
        c = self.cache
        limit = min(self.model.max_seq_length, c.allocator.num_blocks * c.allocator.block_size) - 1
        bound = FIRST_CONTEXT_BOUND
        while bound - 1 < position:
            bound *= 2
        return min(bound - 1, limit)

    def _graph_mode(self, on, bound=None):
        c = self.cache
        c.graph_pos = self.pos if on else None
        c.graph_ctx = self.ctx if on else None
        c.graph_partition_tokens = self.partition_tokens if on else 0
        c.graph_max_position = bound if on else None

    def _forward_body(self):
        """The captured step: embeddings and blocks (Model._hidden_states),
        then mie_lm_head - final norm, LM head and greedy pick, which writes
        the token the next step reads and advances the device position and
        context length.  The pick's merge is one workgroup with nothing to
        clear (torch.argmax over a row this wide reduces across workgroups
        behind a memset, which a graph must not hold)."""
        model = self.model
        x = model._hidden_states(self.token, self.cache)
        projection.lm_head(x[0, -1], model.final_norm, model.output_projection, out=self._logits,
                           token_out=self.token, workspace=self._head_ws, advance=self.counters)
        return self._logits

    @torch.no_grad()
    def prime(self, token):
        """Set the token to decode next (a [1, 1] or [1] integer tensor) and
        the device position from the cache."""
        self.token.copy_(token.reshape(1, 1))
        p = self.cache.position
        self.pos.fill_(p)
        self.ctx.fill_(p + 1)

    @torch.no_grad()
    def step(self):
        cache = self.cache
        if cache.position >= self.model.max_seq_length:
            raise RuntimeError("KV cache is full")
        cache._reserve(cache.position + 1)
        if self.graph is not None and (self._epoch != _TENSOR_EPOCH[0]
                                       or self.position_bound(cache.position) != self.bound):
            # A tensor the captured step reads was replaced (a conversion, an
            # assigning load, a parameter swapped with drop_decode_plan), or
            # the position left the captured step's bound: run eagerly and
            # capture again.
            self.graph = self._graph_out = self._plans = None
        if self.graph is None:
            # This step runs eagerly at the current position and the capture
            # serves the steps from the next one on.
            self.bound = self.position_bound(cache.position + 1)
        self._graph_mode(True, self.bound)
        try:
            if self.graph is None:
                # The first step runs eagerly on the stream the capture will use
                # (so every library handle it records exists already); its
                # results are returned.
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    self.logits = self._forward_body()
                torch.cuda.synchronize()
                position = cache.position
                if position < self.model.max_seq_length:
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=side):
                        self._graph_out = self._forward_body()
                    # Capture records the work without running it: restore the
                    # host position its forward advanced.
                    cache.position = position
                    self.graph = graph
                    # The replays use the blocks' launch plans' rows,
                    # accumulators and workspaces as captured; a block keeps
                    # one plan, which a decode on another cache (or a change
                    # of the block) replaces, so the decoder holds them.
                    self._plans = [block._one_token for block in self.model.MoEBlocks]
                    self._epoch = _TENSOR_EPOCH[0]
                    self.captures += 1
            else:
                self.graph.replay()
                cache.position += 1
                self.replays += 1
                self.logits = self._graph_out
            self.next_token = self.token
        finally:
            self._graph_mode(False)
        return self.next_token


@torch.no_grad()
def generate_graphed(model, token_ids, max_new_tokens, cache, partition_tokens=0):
    """Greedy generation with the same results and stopping rules as
    Model.generate(..., temperature=0, cache=cache) (model.py:567-621), with
    decode steps replayed from a HIP graph."""
    if max_new_tokens < 1:
        raise ValueError("max_new_tokens must be at least 1")
    if token_ids.dim() == 1:
        token_ids = token_ids.unsqueeze(0)
    token_ids = token_ids.to(model.token_embedding.weight.device).long()
    if token_ids.shape[0] != 1 or token_ids.shape[1] == 0:
        raise ValueError("generate_graphed() handles one non-empty sequence")
    if token_ids.shape[1] > model.max_seq_length:
        raise ValueError(f"prompt is {token_ids.shape[1]} tokens; max_seq_length is {model.max_seq_length}")
    if cache.position != 0:
        raise ValueError("generate_graphed() needs a fresh cache")
    out = [token_ids]
    logits = model(token_ids, cache)[:, -1, :]
    next_token = torch.argmax(logits, dim=-1, keepdim=True)
    decoder = None
    for step in range(max_new_tokens):
        if next_token.item() == EOS_TOKEN_ID:
            break
        out.append(next_token.clone())
        if step == max_new_tokens - 1 or cache.position >= model.max_seq_length:
            break  # the last token is never fed back (Model.generate does the same)
        if decoder is None:
            # Each step leaves the next token in the decoder's device buffer.
            decoder = GraphedDecoder(model, cache, partition_tokens)
            decoder.prime(next_token)
        next_token = decoder.step()
    return torch.cat(out, dim=1)


class GraphedGenerator:
    """generate_graphed for a sequence of requests on one cache object: the
    step graph is captured on the first request and replayed by every later
    one (the cache is freed after each request; its device block table, which
    the graph reads, stays).  Requests must not overlap."""

    def __init__(self, model, cache, partition_tokens=0):
        if not isinstance(cache, PagedKVCache):
            raise ValueError("graph decode needs a paged cache")
        self.model = model
        self.cache = cache
        self.partition_tokens = partition_tokens
        self.decoder = None

    @torch.no_grad()
    def generate(self, token_ids, max_new_tokens):
        """Greedy tokens as Model.generate(..., temperature=0) returns them."""
        model, cache = self.model, self.cache
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be at least 1")
        if token_ids.dim() == 1:
            token_ids = token_ids.unsqueeze(0)
        token_ids = token_ids.to(model.token_embedding.weight.device).long()
        if token_ids.shape[0] != 1 or token_ids.shape[1] == 0:
            raise ValueError("generate() handles one non-empty sequence")
        if token_ids.shape[1] > model.max_seq_length:
            raise ValueError(f"prompt is {token_ids.shape[1]} tokens; max_seq_length is {model.max_seq_length}")
        cache.free()
        try:
            out = [token_ids]
            logits = model(token_ids, cache)[:, -1, :]
            next_token = torch.argmax(logits, dim=-1, keepdim=True)
            for step in range(max_new_tokens):
                if next_token.item() == EOS_TOKEN_ID:
                    break
                out.append(next_token.clone())
                if step == max_new_tokens - 1 or cache.position >= model.max_seq_length:
                    break
                if step == 0:
                    if self.decoder is None:
                        self.decoder = GraphedDecoder(model, cache, self.partition_tokens)
                    self.decoder.prime(next_token)
                next_token = self.decoder.step()
            return torch.cat(out, dim=1)
        finally:
            cache.free()
