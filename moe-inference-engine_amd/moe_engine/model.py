"""miniMoE inference host with contiguous and paged KV caches.

Drop-in for the reference engine's src/moe_engine/model.py: the classes,
constructor arguments, attributes, state-dict names and error messages are the
reference's, so callers and checkpoints move over unchanged.  What differs is
underneath the paged cache on a ROCm device:

  * PagedKVCache.write  -> one mie_kv_append launch (K and V, decode or prefill)
  * PagedKVCache.read   -> one mie_kv_gather launch (K and V)
  * direct decode       -> mie_paged_decode (moe_engine.paged_attention)
  * one-token MoE       -> mie_moe_decode (moe_engine.fused_moe)
  * one decode token through a whole block (both halves fused) -> one
    mie_block_decode call into a stored launch plan (five launches)
  * at inference, the embedding, the one-token head and the greedy pick ->
    mie_embed, mie_lm_head, mie_argmax

A paged pool on a ROCm device requires the HIP library and raises at
construction without it.  Pools on the CPU use PyTorch indexing, which is the
reference's own CPU behaviour for this device.

Random initialisation consumes the RNG in the reference's module order
(token and positional embeddings, output projection, then per block:
attention out_proj, in_proj xavier, the experts' two linears each, router), so
a seeded model has the reference's weights.
"""

import collections
import ctypes
import math
import weakref
from dataclasses import dataclass
from typing import Optional

import torch
from torch import nn
from torch.nn import functional as F

from moe_engine import _native, embedding, fused_moe, kv_ops, paged_attention, projection

EOS_TOKEN_ID = 50256
ATTENTION_MODES = ("auto", "direct", "gather")
# Block ids one mie_block_table_append launch carries in its arguments.
_TABLE_APPEND_MAX = 16
MOE_MODES = ("auto", "direct", "reference")

# A block's one-token launch plan (TransformerMoEBlock._decode_one_token) and a
# captured decode step (moe_engine.graphs) hold raw device addresses of
# parameters, buffers and expert storages.  Every operation that can put a new
# tensor in their place inside the modules below - device / dtype conversion
# (_apply), assignment of a parameter, buffer or submodule (which
# load_state_dict(assign=True) and the expert repacking go through) - advances
# this epoch, and a plan or captured step made under an earlier epoch is made
# again before its next use.  Writing in place keeps the addresses, so it needs
# nothing.
_TENSOR_EPOCH = [0]

# One-token launch plans a block keeps (the most recently used): sequences
# decoded in turn each find theirs.
_KEPT_PLANS = 4


def _tensors_replaced() -> None:
    _TENSOR_EPOCH[0] += 1


# Plain attributes a launch plan is built from: a MoE layer's mode and a
# norm's eps.  Changing one advances _TENSOR_EPOCH like a tensor replacement.
_PLAN_SETTINGS = ("mode", "eps")


class _TracksReplacement:
    """Mixin for the modules a launch plan reads from: conversion or
    assignment of a tensor or submodule, or a change of a setting in
    _PLAN_SETTINGS, advances _TENSOR_EPOCH."""

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        _tensors_replaced()
        return result

    def __setattr__(self, name, value):
        changed = name in _PLAN_SETTINGS and getattr(self, name, None) != value
        super().__setattr__(name, value)
        if changed or isinstance(value, (torch.Tensor, nn.Module)):
            _tensors_replaced()

    def register_buffer(self, name, tensor, persistent=True):
        super().register_buffer(name, tensor, persistent)
        _tensors_replaced()

    def register_parameter(self, name, param):
        super().register_parameter(name, param)
        _tensors_replaced()


class Linear(_TracksReplacement, nn.Linear):
    """nn.Linear whose tensor replacements invalidate launch plans."""


class LayerNorm(_TracksReplacement, nn.LayerNorm):
    """nn.LayerNorm whose tensor replacements invalidate launch plans."""


class Embedding(_TracksReplacement, nn.Embedding):
    """nn.Embedding whose tensor replacements invalidate launch plans (the
    first block's plan reads both tables) and captured decode steps."""


@dataclass
class ModelConfig:
    """Reference fields (model.py:18-27) plus `ffn_dim`, the expert hidden size.

    ffn_dim None keeps the reference's hard-coded 4 * hidden_dim (model.py:489).
    """

    max_seq_length: int = 1024
    vocab_size: int = 50304
    num_layers: int = 6
    hidden_dim: int = 768
    moe_multiplier: float = 0.01  # checkpoint compatibility only
    num_experts: int = 8
    top_k: int = 2
    num_heads: int = 8
    ffn_dim: Optional[int] = None

    @property
    def head_dim(self) -> int:
        return self.hidden_dim // self.num_heads

    @property
    def expert_hidden_dim(self) -> int:
        return 4 * self.hidden_dim if self.ffn_dim is None else self.ffn_dim


class KVCache:
    """Contiguous K/V storage [layer, batch, head, max_seq, head_dim] (model.py:30-58).

    The comparator for the paged path: write is a slice store, read a view.
    """

    def __init__(self, config: ModelConfig, batch_size: int, device, dtype=torch.float32):
        shape = (config.num_layers, batch_size, config.num_heads, config.max_seq_length, config.head_dim)
        self.k = torch.zeros(shape, device=device, dtype=dtype)
        self.v = torch.zeros(shape, device=device, dtype=dtype)
        self.position = 0

    def write(self, layer_idx, position, k, v):
        end = position + k.shape[2]
        self.k[layer_idx, :, :, position:end] = k
        self.v[layer_idx, :, :, position:end] = v

    def read(self, layer_idx, length):
        return self.k[layer_idx, :, :, :length], self.v[layer_idx, :, :, :length]


class BlockAllocator:
    """Shared block pools and a LIFO free list (model.py:61-105).

    attention_mode chooses how caches from this pool attend while decoding:
      "gather" - rebuild contiguous K/V, then PyTorch attention (the oracle),
      "direct" - require the HIP kernel that reads blocks in place,
      "auto"   - direct when supported, else gather.
    """

    def __init__(
        self,
        config: ModelConfig,
        num_blocks: int,
        block_size: int,
        device,
        dtype=torch.float32,
        attention_mode: str = "auto",
    ):
        if attention_mode not in ATTENTION_MODES:
            raise ValueError(f"unknown attention_mode {attention_mode!r}")
        self.attention_mode = attention_mode
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_heads = config.num_heads
        self.head_dim = config.head_dim
        shape = (config.num_layers, num_blocks, config.num_heads, block_size, self.head_dim)
        self.k_pool = torch.zeros(shape, device=device, dtype=dtype)
        self.v_pool = torch.zeros(shape, device=device, dtype=dtype)
        # On a ROCm device every paged tensor operation is a HIP kernel; there
        # is no PyTorch substitute, so a missing library fails here, loudly.
        self.on_device = _native.is_rocm_device(self.k_pool)
        if self.on_device:
            _native.lib()
        # Launch constants shared by every call on this pool (element strides
        # inside one layer, dtype code); pointers are read per call.
        self._launch = None
        if self.on_device and dtype in _native.DTYPE_CODES:
            self._launch = (
                self.k_pool.stride(0) * self.k_pool.element_size(),  # layer stride, bytes
                self.k_pool.stride(1),  # block stride, elements
                self.k_pool.stride(2),  # head stride, elements
                _native.DTYPE_CODES[dtype],
            )
        # One-token decode projects QKV straight into the pools
        # (mie_qkv_append) when the model width and dtype are built; set to
        # False to run the reference's projection + append sequence instead.
        self.fuse_qkv = self._launch is not None and kv_ops.qkv_append_supported(
            config.num_heads * config.head_dim, dtype
        )
        self.free_blocks = list(range(num_blocks))

    def allocate(self) -> int:
        if not self.free_blocks:
            raise RuntimeError("no free KV cache blocks left")
        return self.free_blocks.pop()

    def free(self, block_ids: list) -> None:
        self.free_blocks.extend(block_ids)

    def new_cache(self) -> "PagedKVCache":
        return PagedKVCache(self)


class PagedKVCache:
    """One sequence's block table over a shared allocator (model.py:108-208)."""

    def __init__(self, allocator: BlockAllocator):
        self.allocator = allocator
        self.attention_mode = allocator.attention_mode
        self.block_table: list = []
        self.position = 0
        # Device mirror of block_table for the kernels.  Only the first
        # len(block_table) entries are meaningful; new entries are appended as
        # blocks are reserved (once per block_size tokens: on a ROCm device one
        # small launch carrying the ids, on the CPU an indexed copy), never
        # rebuilt.
        self.block_table_device = torch.zeros(
            allocator.num_blocks, dtype=torch.int32, device=allocator.k_pool.device
        )
        self._write_index_key = None  # (position, seq_len) of cached CPU indices
        # Graph mode (moe_engine.graphs): device int32 [1] tensors holding the
        # position of the token being decoded and the context length (adjacent
        # in memory: [position, length]); the kernels read them instead of host
        # ints, and blocks are reserved by the caller before each replay.
        # graph_max_position bounds the positions a replay can reach.  None in
        # ordinary use.
        self.graph_pos = None
        self.graph_ctx = None
        self.graph_partition_tokens = 0
        self.graph_max_position = None

    def _reserve(self, num_tokens: int) -> None:
        """Hold enough blocks for `num_tokens`, all or nothing (model.py:125-143)."""
        needed = -(-num_tokens // self.allocator.block_size)
        taken = []
        try:
            while len(self.block_table) + len(taken) < needed:
                taken.append(self.allocator.allocate())
        except RuntimeError:
            self.allocator.free(taken)
            raise
        if taken:
            start = len(self.block_table)
            self.block_table.extend(taken)
            if self.allocator.on_device and len(taken) <= _TABLE_APPEND_MAX:
                # The ids go in the arguments of one small launch on the
                # current stream: no staging copy for the host to wait on.
                ids = (ctypes.c_int32 * len(taken))(*taken)
                table = self.block_table_device
                _native.check(
                    _native.lib().mie_block_table_append(table.data_ptr(), table.numel(), start, ids, len(taken),
                                                         _native.stream_of(table)),
                    "mie_block_table_append",
                )
            else:
                self.block_table_device[start : start + len(taken)] = torch.tensor(
                    taken, dtype=torch.int32, device=self.block_table_device.device
                )

    def _block_for(self, token_pos: int):
        size = self.allocator.block_size
        return self.block_table[token_pos // size], token_pos % size

    def _write_indices(self, position, seq_len):
        """(physical block, slot) index tensors for a multi-token CPU write,
        built once per step and reused by every layer (model.py:149-165)."""
        if self._write_index_key != (position, seq_len):
            size = self.allocator.block_size
            pos = torch.arange(position, position + seq_len, device=self.block_table_device.device)
            self._write_index = (self.block_table_device[pos // size].long(), pos % size)
            self._write_index_key = (position, seq_len)
        return self._write_index

    def write(self, layer_idx, position, k, v):
        """Append k, v [1, H, S, D] at logical positions position..position+S-1."""
        if k.shape[0] != 1:
            raise ValueError("PagedKVCache holds one sequence; use batch size 1")
        seq_len = k.shape[2]
        alloc = self.allocator
        if self.graph_pos is not None:
            # Blocks were reserved before the replay; the position is on the device.
            if seq_len != 1:
                raise ValueError("graph mode appends one token per step")
            kv_ops.append(alloc.k_pool, alloc.v_pool, layer_idx, k, v, self.block_table_device[None],
                          positions=self.graph_pos)
            return
        self._reserve(position + seq_len)
        if alloc.on_device:
            ks = k.stride()
            if (
                alloc._launch is not None
                and ks == v.stride()
                and ks[3] == 1
                and k.dtype == alloc.k_pool.dtype
                and k.shape[1] == alloc.num_heads
                and k.shape[3] == alloc.head_dim
                and k.device == alloc.k_pool.device
                and 0 <= layer_idx < alloc.k_pool.shape[0]
            ):
                # Lean path for the engine's own calls: one C call, one launch.
                layer_bytes, sblk, shead, code = alloc._launch
                off = layer_idx * layer_bytes
                rc = _native.lib().mie_kv_append(
                    alloc.k_pool.data_ptr() + off, alloc.v_pool.data_ptr() + off, sblk, shead, alloc.num_blocks,
                    k.data_ptr(), v.data_ptr(), ks[0], ks[1], ks[2],
                    self.block_table_device.data_ptr(), 0, None, position,
                    1, seq_len, alloc.num_heads, alloc.head_dim, alloc.block_size, code, _native.stream_of(k),
                )
                if rc:
                    _native.check(rc, "mie_kv_append")
                return
            kv_ops.append(alloc.k_pool, alloc.v_pool, layer_idx, k, v, self.block_table_device, position=position)
            return
        if seq_len == 1:
            block_id, slot = self._block_for(position)
            alloc.k_pool[layer_idx, block_id, :, slot] = k[0, :, 0]
            alloc.v_pool[layer_idx, block_id, :, slot] = v[0, :, 0]
            return
        blocks, slots = self._write_indices(position, seq_len)
        alloc.k_pool[layer_idx, blocks, :, slots] = k[0].transpose(0, 1)
        alloc.v_pool[layer_idx, blocks, :, slots] = v[0].transpose(0, 1)

    def write_projected(self, layer_idx, position, x, in_proj_weight, in_proj_bias, norm=None):
        """One decode token: q, k, v = in_proj(norm(x)) with k, v stored at
        `position` (reference model.py:228-234 then :167-178) in one launch
        (mie_qkv_append).  Returns q [1, H, 1, D].  The caller has checked that
        the allocator's `fuse_qkv` applies and that x and the parameters share
        the pools' dtype and device."""
        alloc = self.allocator
        if self.graph_pos is None:
            self._reserve(position + 1)
        layer_bytes, sblk, shead, code = alloc._launch
        off = layer_idx * layer_bytes
        q = torch.empty((1, alloc.num_heads, 1, alloc.head_dim), dtype=alloc.k_pool.dtype, device=x.device)
        rc = _native.lib().mie_qkv_append(
            x.data_ptr(),
            None if norm is None else _native.ptr(norm.weight),
            None if norm is None else _native.ptr(norm.bias),
            1e-5 if norm is None else float(norm.eps),
            in_proj_weight.data_ptr(), _native.ptr(in_proj_bias), alloc.num_heads * alloc.head_dim,
            alloc.k_pool.data_ptr() + off, alloc.v_pool.data_ptr() + off, sblk, shead, alloc.num_blocks,
            self.block_table_device.data_ptr(), alloc.num_blocks, _native.ptr(self.graph_pos), position,
            q.data_ptr(), alloc.num_heads, alloc.head_dim, alloc.block_size, code, _native.stream_of(x),
        )
        if rc:
            _native.check(rc, "mie_qkv_append")
        return q

    def read(self, layer_idx, length):
        """Contiguous K, V [1, H, length, D] of logical positions 0..length-1."""
        alloc = self.allocator
        if alloc.on_device:
            return kv_ops.gather(alloc.k_pool, alloc.v_pool, layer_idx, self.block_table_device, length)
        ids = self.block_table[: -(-length // alloc.block_size)]

        def rebuild(pool):
            tiles = pool[layer_idx, ids]  # [nb, H, BS, D]
            return tiles.transpose(0, 1).reshape(alloc.num_heads, -1, alloc.head_dim)[:, :length].unsqueeze(0)

        return rebuild(alloc.k_pool), rebuild(alloc.v_pool)

    def free(self):
        """Return every block and reset; stale mirror entries are never read."""
        self.allocator.free(self.block_table)
        self.block_table = []
        self.position = 0
        self._write_index_key = None


class CachedAttention(_TracksReplacement, nn.Module):
    """Causal self-attention over an external cache (model.py:211-269)."""

    def __init__(self, dim: int, num_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.in_proj_weight = nn.Parameter(torch.empty(3 * dim, dim))
        self.in_proj_bias = nn.Parameter(torch.empty(3 * dim))
        self.out_proj = Linear(dim, dim)
        nn.init.xavier_uniform_(self.in_proj_weight)
        nn.init.zeros_(self.in_proj_bias)

    def fused_decode(self, x, norm, cache, layer_idx, position: int):
        """x + attention(norm(x)) for one decode token - the attention half of
        the block (reference model.py:495) - in three launches: the QKV
        projection stored straight into the paged pools (mie_qkv_append), the
        paged decode, and out_proj with the residual add (mie_linear_residual).
        Returns None when that path does not apply; the caller then runs
        x + forward(norm(x), ...).

        Applies to a paged cache on a ROCm device whose decode runs the direct
        kernel, a float32 / bfloat16 model of a built width, and a plain
        LayerNorm; results equal forward()'s to float32 rounding."""
        if position <= 0 or not self.fused_decode_supported(x, norm, cache):
            return None
        alloc = cache.allocator
        q = cache.write_projected(layer_idx, position, x, self.in_proj_weight, self.in_proj_bias, norm)
        attn = paged_attention.decode(q, cache, layer_idx, context_len=position + 1)  # [1, H, 1, D]: heads in order
        w, b = self.out_proj.weight, self.out_proj.bias
        out = torch.empty_like(x)
        rc = _native.lib().mie_linear_residual(
            attn.data_ptr(), w.data_ptr(), _native.ptr(b), x.data_ptr(), out.data_ptr(),
            w.shape[0], w.shape[1], alloc._launch[3], _native.stream_of(x),
        )
        if rc:
            _native.check(rc, "mie_linear_residual")
        return out

    def fused_decode_supported(self, x, norm, cache) -> bool:
        """Whether fused_decode's three launches apply to this token, cache
        and norm (everything but the position)."""
        alloc = getattr(cache, "allocator", None)
        return not (
            alloc is None
            or not getattr(alloc, "fuse_qkv", False)
            or cache.attention_mode == "gather"
            or x.shape[:2] != (1, 1)
            or not x.is_contiguous()
            or x.dtype != alloc.k_pool.dtype
            or x.device != alloc.k_pool.device
            or self.in_proj_weight.dtype != x.dtype
            or not isinstance(norm, nn.LayerNorm)
            or norm.weight is None
            or norm.weight.dtype != x.dtype
            or (norm.bias is not None and norm.bias.dtype != x.dtype)
            or tuple(norm.normalized_shape) != (x.shape[-1],)
            or self.out_proj.weight.dtype != x.dtype
            or not self.out_proj.weight.is_contiguous()
            or not paged_attention.is_supported(x, self.head_dim)
        )

    def forward(self, x, cache, layer_idx, position: int):
        batch, seq_len, dim = x.shape
        qkv = F.linear(x, self.in_proj_weight, self.in_proj_bias)
        # [batch, seq, 3*dim] -> three [batch, head, seq, head_dim] views
        q, k, v = (
            t.view(batch, seq_len, self.num_heads, self.head_dim).transpose(1, 2) for t in qkv.chunk(3, dim=-1)
        )

        mode = getattr(cache, "attention_mode", "gather")
        use_kernel = mode != "gather" and paged_attention.is_supported(x, self.head_dim)
        if mode == "direct" and not use_kernel:
            # Raised before the write below reserves blocks, so a rejected
            # forward leaves the cache untouched.
            raise RuntimeError(
                "attention_mode='direct' needs a ROCm device, the HIP paged-KV library, "
                "float32 or bfloat16 and a built head_dim; use 'auto' for automatic "
                "fallback or 'gather' for the oracle path"
            )

        cache.write(layer_idx, position, k, v)
        assert position == 0 or seq_len == 1, "prefill must start at position 0"

        if mode != "gather" and position == 0:
            # At position 0 the whole history is the K/V just projected.
            out = F.scaled_dot_product_attention(q, k, v, is_causal=seq_len > 1)
        elif use_kernel:
            out = paged_attention.decode(q, cache, layer_idx, context_len=position + 1)
        else:
            keys, values = cache.read(layer_idx, position + seq_len)
            out = F.scaled_dot_product_attention(q, keys, values, is_causal=seq_len > 1)

        out = out.transpose(1, 2).reshape(batch, seq_len, dim)
        return self.out_proj(out)


class Expert(_TracksReplacement, nn.Module):
    def __init__(self, dim, hidden_dim):
        super().__init__()
        self.net = nn.Sequential(Linear(dim, hidden_dim), nn.GELU(), Linear(hidden_dim, dim))

    def forward(self, x):
        return self.net(x)


class MoEFeedForward(_TracksReplacement, nn.Module):
    """Top-k mixture of experts (model.py:285-481).

    Mode 'reference' runs the reference's PyTorch path (model.py:443-461)
    everywhere.  In mode 'auto' or 'direct', one-token decode runs the fused
    HIP kernels (moe_engine.fused_moe) where they apply - a ROCm device, the
    HIP library, float32 or bfloat16, one token - and a float32 prefill of up to 512
    tokens on a ROCm device runs dense-masked (_forward_dense: the reference's
    result without its per-expert synchronisations).  'auto' falls back to the
    PyTorch path elsewhere; a forced 'direct' decode that cannot run raises
    before any cache mutation, through the model's decode preflight
    (model.py:408-441).

    The experts' parameters are views into four canonical contiguous storages
    (`_expert_storage`: w1 [E, hidden, dim], b1 [E, hidden], w2 [E, dim,
    hidden], b2 [E, dim]), so the kernels address a selected expert by offset;
    the views keep the checkpoint's parameter names, and the storages are
    rebuilt after load_state_dict and after device / dtype conversion
    (model.py:323-366).
    """

    def __init__(self, dim, hidden_dim, num_experts, top_k, mode="auto"):
        super().__init__()
        if mode not in MOE_MODES:
            raise ValueError(f"unknown MoE mode {mode!r}")
        self.mode = mode
        self.dim = dim
        self.hidden_dim = hidden_dim
        self.top_k = top_k
        self.num_experts = num_experts
        self.experts = nn.ModuleList(Expert(dim, hidden_dim) for _ in range(num_experts))
        self.router = Linear(dim, num_experts, bias=False)
        # Fixed per-layer decode workspaces; non-persistent, so checkpoints and
        # state-dict keys are unchanged (model.py:301-321).
        for name, shape, dtype in (
            ("_router_logits", (num_experts,), torch.float32),
            ("_expert_ids", (top_k,), torch.int32),
            ("_route_weights", (top_k,), torch.float32),
            ("_expert_hidden", (top_k, hidden_dim), torch.float32),
            ("_direct_out", (dim,), torch.float32),
        ):
            self.register_buffer(name, torch.empty(shape, dtype=dtype), persistent=False)
        self._pack_expert_parameters()
        self.register_load_state_dict_post_hook(self._repack_after_load)

    def _pack_group(self, layer_index: int, name: str) -> torch.Tensor:
        """One storage [E, *shape] whose slices become the experts' parameters."""
        params = [getattr(expert.net[layer_index], name) for expert in self.experts]
        if any(p.shape != params[0].shape for p in params):
            raise ValueError("all experts must have identical parameter shapes")
        storage = torch.empty((len(params), *params[0].shape), dtype=params[0].dtype, device=params[0].device)
        with torch.no_grad():
            for expert, src, dst in zip(self.experts, params, storage):
                dst.copy_(src)
                setattr(expert.net[layer_index], name, nn.Parameter(dst, requires_grad=src.requires_grad))
        return storage

    def _pack_expert_parameters(self) -> None:
        self._expert_storage = {
            "w1": self._pack_group(0, "weight"),
            "b1": self._pack_group(0, "bias"),
            "w2": self._pack_group(2, "weight"),
            "b2": self._pack_group(2, "bias"),
        }

    def _repack_after_load(self, _module, _incompatible_keys) -> None:
        # load_state_dict copies into the views; assign=True replaces them.
        self._pack_expert_parameters()

    def _apply(self, fn, recurse=True):
        # Device / dtype conversion replaces each parameter on its own.
        result = super()._apply(fn, recurse=recurse)
        self._pack_expert_parameters()
        # The routing workspaces stay float32 whatever the model's dtype (the
        # reference routes in float32); the others follow the conversion.
        for name in ("_router_logits", "_route_weights"):
            buf = getattr(self, name)
            if buf.dtype != torch.float32:
                setattr(self, name, buf.float())
        return result

    def set_mode(self, mode: str) -> None:
        if mode not in MOE_MODES:
            raise ValueError(f"unknown MoE mode {mode!r}")
        self.mode = mode

    def _has_direct_layout(self) -> bool:
        s = self._expert_storage
        return fused_moe.has_canonical_layout(
            self.router.weight, s["w1"], s["b1"], s["w2"], s["b2"],
            self._router_logits, self._expert_ids, self._route_weights, self._expert_hidden, self._direct_out,
        )

    def _direct_supported(self, x: torch.Tensor) -> bool:
        return (
            fused_moe.is_supported(
                x, num_experts=self.num_experts, top_k=self.top_k, expert_hidden_dim=self.hidden_dim
            )
            and self._has_direct_layout()
        )

    def direct_configuration_supported(self, batch_size: int = 1) -> bool:
        """Whether one-token decode of this layer can take the fused kernels
        (metadata only: no input needed)."""
        w = self.router.weight
        return (
            fused_moe.is_configuration_supported(
                device=w.device, dtype=w.dtype, batch_size=batch_size, hidden_dim=self.dim,
                num_experts=self.num_experts, top_k=self.top_k, expert_hidden_dim=self.hidden_dim,
            )
            and self._has_direct_layout()
        )

    @staticmethod
    def _raise_direct_unsupported() -> None:
        raise RuntimeError(
            "MoE mode 'direct' needs one-token batch-one float32 or bfloat16 decode on a ROCm device with the HIP "
            "library (at most 64 experts, top-k at most 8, dimensions multiples of 4); use 'auto' for "
            "automatic fallback or 'reference' for the PyTorch oracle"
        )

    def preflight_direct_decode(self, *, batch_size: int) -> None:
        """Reject an unsupported forced decode before any cache mutation."""
        if self.mode == "direct" and not self.direct_configuration_supported(batch_size):
            self._raise_direct_unsupported()

    def uses_direct(self, x: torch.Tensor, *, decode: bool) -> bool:
        """Resolve reference / direct / auto without reading device results."""
        if not decode or self.mode == "reference":
            return False
        supported = self._direct_supported(x)
        if self.mode == "direct" and not supported:
            self._raise_direct_unsupported()
        return supported

    def _forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        batch, seq_len, dim = x.shape
        flat = x.reshape(-1, dim)
        with torch.autocast(device_type=x.device.type, enabled=False):
            logits = F.linear(flat.float(), self.router.weight.float())
            top_logits, top_ids = torch.topk(logits, k=self.top_k, dim=-1)
            top_weights = F.softmax(top_logits, dim=-1)
        out = torch.zeros_like(flat)
        for expert_id, expert in enumerate(self.experts):
            rows, slot = torch.where(top_ids == expert_id)
            if rows.numel() == 0:
                continue
            weight = top_weights[rows, slot].unsqueeze(-1).to(flat.dtype)
            out.index_add_(0, rows, weight * expert(flat[rows]))
        return out.reshape(batch, seq_len, dim)

    def _forward_direct(self, x: torch.Tensor) -> torch.Tensor:
        s = self._expert_storage
        return fused_moe.decode(
            x, self.router.weight, s["w1"], s["b1"], s["w2"], s["b2"],
            router_logits=self._router_logits, expert_ids=self._expert_ids, route_weights=self._route_weights,
            hidden=self._expert_hidden, out=self._direct_out,
        )

    # Prefill of at most this many tokens runs dense-masked on the GPU.
    DENSE_PREFILL_MAX_TOKENS = 512

    def uses_dense_prefill(self, x: torch.Tensor, *, decode: bool) -> bool:
        """Multi-token (or mode 'auto'/'direct' prefill) float32 input on a
        ROCm device with the canonical layout takes _forward_dense; everything
        else keeps the reference path."""
        tokens = x.shape[0] * x.shape[1]
        return (
            self.mode != "reference"
            and not (decode and tokens == 1)
            and 1 <= tokens <= self.DENSE_PREFILL_MAX_TOKENS
            and _native.is_rocm_device(x)
            and x.dtype == torch.float32
            and self.router.weight.dtype == torch.float32
            and self._expert_storage["w1"].dtype == torch.float32
        )

    def _forward_dense(self, x: torch.Tensor) -> torch.Tensor:
        """The reference path's result (model.py:443-461) without its
        per-expert torch.where synchronisations: every expert runs on every
        token as one batched GEMM over the canonical storages, and the
        experts' weighted outputs are summed in increasing expert id, each
        product rounded before its add.  For a token's selected experts that is
        index_add_'s order and rounding; the unselected experts add exact zeros
        (routing weight 0).  Routing is the reference's: float32 logits,
        torch.topk, softmax over the top-k."""
        batch, seq_len, dim = x.shape
        flat = x.reshape(-1, dim)
        logits = F.linear(flat, self.router.weight)
        top_logits, top_ids = torch.topk(logits, k=self.top_k, dim=-1)
        dense_w = torch.zeros_like(logits).scatter_(1, top_ids, F.softmax(top_logits, dim=-1))
        s = self._expert_storage
        h = F.gelu(torch.matmul(flat, s["w1"].transpose(1, 2)) + s["b1"].unsqueeze(1))  # [E, T, hidden]
        y = torch.matmul(h, s["w2"].transpose(1, 2)) + s["b2"].unsqueeze(1)  # [E, T, dim]
        out = torch.zeros_like(flat)
        for e in range(self.num_experts):
            out = out + dense_w[:, e : e + 1] * y[e]
        return out.reshape(batch, seq_len, dim)

    def forward(self, x, *, decode=False):
        if self.uses_direct(x, decode=decode):
            return self._forward_direct(x)
        if self.uses_dense_prefill(x, decode=decode):
            return self._forward_dense(x)
        return self._forward_reference(x)

    def fused_block_supported(self, x, norm) -> bool:
        """Whether fused_block_decode's two launches apply to this token and norm."""
        return not (
            self.mode == "reference"
            or not isinstance(norm, nn.LayerNorm)
            or norm.weight is None
            or norm.weight.dtype != x.dtype
            or (norm.bias is not None and norm.bias.dtype != x.dtype)
            or tuple(norm.normalized_shape) != (self.dim,)
            or not self._direct_supported(x)
        )

    def fused_block_decode(self, x, norm):
        """x + self(norm(x), decode=True) for one token in two launches
        (mie_moe_decode_block: the norm and routing in the W1 launch, the
        residual add in the W2 launch), or None when the fused kernels do not
        apply - mode 'reference', an unsupported configuration, or a norm that
        is not a LayerNorm over the hidden size in x's dtype."""
        if not self.fused_block_supported(x, norm):
            return None
        s = self._expert_storage
        return fused_moe.decode_block(
            x, norm.weight, norm.bias, norm.eps, self.router.weight, s["w1"], s["b1"], s["w2"], s["b2"],
            router_logits=self._router_logits, expert_ids=self._expert_ids, route_weights=self._route_weights,
            hidden=self._expert_hidden, out=self._direct_out,
        )


class TransformerMoEBlock(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.attention = CachedAttention(config.hidden_dim, config.num_heads)
        self.moe = MoEFeedForward(config.hidden_dim, config.expert_hidden_dim, config.num_experts, config.top_k)
        self.attn_norm = LayerNorm(config.hidden_dim)
        self.moe_norm = LayerNorm(config.hidden_dim)
        self._one_token = None  # the last plan used: (key, cache weakref, launcher or None); see _decode_one_token
        self._plans = collections.OrderedDict()  # key -> plan, the most recently used last
        self._embed_row = None  # layer 0's embedding row for decode_token_ids
        self.register_load_state_dict_post_hook(TransformerMoEBlock._drop_plan_after_load)

    def __getstate__(self):
        # Copies and pickles leave the launch plans behind: a plan points at
        # this block's tensors, and a copy builds its own on first use.
        state = super().__getstate__().copy()
        state.update(_one_token=None, _plans=collections.OrderedDict(), _embed_row=None)
        return state

    def drop_decode_plan(self) -> None:
        """Forget the one-token launch plan; the next decode token builds a
        new one.  Conversions (.to(), .float(), ...), loads and assignments of
        tensors or submodules anywhere in the block invalidate the plan by
        themselves (_TENSOR_EPOCH); code that swaps a tensor's storage some
        other way (param.data = ...) calls this; it also advances the epoch, so
        every other plan and captured decode step built on the old tensors is
        rebuilt before its next use."""
        self._one_token = None
        self._plans.clear()
        _tensors_replaced()

    @staticmethod
    def _drop_plan_after_load(module, _incompatible_keys) -> None:
        # A load replaces the expert storage (MoEFeedForward repacks), and
        # assign=True replaces every parameter.
        module.drop_decode_plan()

    def _apply(self, fn, recurse=True):
        # Device / dtype conversion replaces the parameters.
        self.drop_decode_plan()
        return super()._apply(fn, recurse=recurse)

    def forward(self, x, cache, layer_idx, position):
        # One-token decode with both fused halves runs from a cached launch
        # plan (eagerly, or recorded into a graph with device positions);
        # otherwise each half takes its fused path where it applies (same
        # results to float32 rounding), else the reference's block
        # (model.py:494-498).
        if position > 0 and x.shape[1] == 1:
            out = self._decode_one_token(x, cache, layer_idx, position)
            if out is not None:
                return out
        h = self.attention.fused_decode(x, self.attn_norm, cache, layer_idx, position)
        if h is None:
            h = x + self.attention(self.attn_norm(x), cache, layer_idx, position)
        decode = position > 0 and h.shape[1] == 1
        out = self.moe.fused_block_decode(h, self.moe_norm) if decode else None
        if out is None:
            out = h + self.moe(self.moe_norm(h), decode=decode)
        return out

    def _one_token_key(self, x, cache, layer_idx):
        """What a plan is built for besides the block's own tensors: the
        cache (by identity; the plan also keeps a weak reference to it), its
        attention mode, the allocator's fuse_qkv switch, the MoE mode, the
        norms' eps, x's dtype, device and width, and the tensor epoch, which
        covers every replacement of a parameter, buffer or expert storage the
        plan points at.  Each token compares this short key only."""
        m = self._modules
        return (layer_idx, id(cache), cache.attention_mode, cache.allocator.fuse_qkv, m["moe"].mode,
                m["attn_norm"].eps, m["moe_norm"].eps, x.dtype, x.device, x.shape[-1], _TENSOR_EPOCH[0])

    def _decode_one_token(self, x, cache, layer_idx, position, embed=None):
        """The block for one decode token when both fused halves apply, from
        a launch plan (mie_block_decode): four launches for contexts the fused
        attention + output projection serves, else the five of fused_decode +
        fused_block_decode; the checks and the static launch arguments are
        computed once per plan key rather than per token.  In graph mode
        (cache.graph_pos set) the launches read the device position and
        length.  Returns None when the fused halves do not both apply."""
        if getattr(cache, "allocator", None) is None or x.dim() != 3 or x.shape[0] != 1 or not x.is_contiguous():
            return None
        graph_pos = getattr(cache, "graph_pos", None)
        if graph_pos is not None and (
                cache.graph_ctx is None or cache.graph_max_position is None
                or cache.graph_ctx.data_ptr() != graph_pos.data_ptr() + 4):
            return None  # the plan reads [position, length] as one device pair
        key = self._one_token_key(x, cache, layer_idx)
        if embed is not None:
            key = key + (embed[1].data_ptr(), embed[1].shape[0], embed[2].data_ptr(), embed[2].shape[0])
        plan = self._one_token
        # The weak reference rules out a new cache that reuses a dead one's id;
        # the plan itself holds no reference to the cache or its pools, so a
        # finished sequence's pools can be freed.  The last few plans are kept,
        # so sequences decoded in turn do not rebuild them every token.
        if plan is None or plan[0] != key or plan[1]() is not cache:
            plan = self._plans.get(key)
            if plan is None or plan[1]() is not cache:
                launcher = None
                if self.attention.fused_decode_supported(x, self.attn_norm, cache) and \
                        self.moe.fused_block_supported(x, self.moe_norm):
                    launcher = self._build_one_token(x, cache, layer_idx, embed)
                plan = (key, weakref.ref(cache), launcher)
                self._plans[key] = plan
                if len(self._plans) > _KEPT_PLANS:
                    self._plans.popitem(last=False)
            else:
                self._plans.move_to_end(key)
            self._one_token = plan
        if plan[2] is None:
            return None
        return plan[2](x, cache, position) if embed is None else plan[2].embed(embed[0], cache, position)

    def decode_token_ids(self, token_ids, cache, position, token_embedding, positional_embedding):
        """The embedding (model.py:558) and this block for one decode token,
        with the embedding folded into the block's QKV launch
        (mie_block_decode_embed): token_ids is an int64 [1, 1] device tensor.
        Returns None when the block's launch plan does not apply; the caller
        then embeds and calls the block itself."""
        w, pw = token_embedding.weight, positional_embedding.weight
        if not (token_ids.dtype == torch.int64 and token_ids.numel() == 1 and token_ids.is_contiguous()
                and token_ids.device == w.device and w.is_contiguous() and pw.is_contiguous() and pw.dtype == w.dtype
                and pw.device == w.device and w.shape[1] == pw.shape[1]):
            return None
        row = self._embed_row
        if row is None or row.dtype != w.dtype or row.device != w.device or row.shape[-1] != w.shape[1]:
            row = self._embed_row = torch.empty((1, 1, w.shape[1]), dtype=w.dtype, device=w.device)
        # The plan is keyed on the row it forms x in; the launcher then reads
        # the token id and the tables instead of x.
        return self._decode_one_token(row, cache, 0, position, embed=(token_ids, w, pw))


    def _build_one_token(self, x, cache, layer_idx, embed=None):
        """A launch plan of the block's launches (mie_block_plan_init): each
        token is then one call, mie_block_decode(plan, x, counters, position).
        The plan holds an accumulator row for the fused attention + output
        projection (zeros; each call leaves it zeroed)."""
        alloc = cache.allocator
        att, moe = self.attention, self.moe
        lib = _native.lib()
        ptr, check, stream_of, decode_plan = _native.ptr, _native.check, _native.stream_of, _native.decode_plan
        layer_bytes, sblk, shead, code = alloc._launch
        heads, head_dim, block_size, num_blocks = alloc.num_heads, alloc.head_dim, alloc.block_size, alloc.num_blocks
        dim = x.shape[-1]
        dtype, device = x.dtype, x.device
        off = layer_idx * layer_bytes
        # Addresses only: the launcher must not keep the cache or its pools alive.
        k_layer, v_layer = alloc.k_pool.data_ptr() + off, alloc.v_pool.data_ptr() + off
        table = cache.block_table_device.data_ptr()
        an, mn = self.attn_norm, self.moe_norm
        s = moe._expert_storage
        out = moe._direct_out.view(1, 1, dim)
        # The block's intermediates, reused by every token: q, the attention
        # output and the attention half's output are consumed within the call.
        q = torch.empty((1, heads, 1, head_dim), dtype=dtype, device=device)
        attn = torch.empty_like(q)
        h = torch.empty((1, 1, dim), dtype=dtype, device=device)
        acc = torch.zeros(dim + 1, dtype=torch.int64, device=device)
        plan = ctypes.create_string_buffer(lib.mie_block_plan_bytes())
        held = {}  # the split-context workspace the plan points at
        tables = None if embed is None else (embed[1], embed[2])  # token and positional tables

        def init(ws):
            held["ws"] = ws
            check(lib.mie_block_plan_init(
                plan, len(plan), dim, heads, head_dim, block_size, code,
                ptr(an.weight), ptr(an.bias), float(an.eps), att.in_proj_weight.data_ptr(), ptr(att.in_proj_bias),
                att.out_proj.weight.data_ptr(), ptr(att.out_proj.bias),
                k_layer, v_layer, sblk, shead, num_blocks, table, num_blocks, 1.0 / math.sqrt(head_dim),
                q.data_ptr(), attn.data_ptr(), h.data_ptr(), ptr(ws), 0 if ws is None else ws.numel(),
                ptr(mn.weight), ptr(mn.bias), float(mn.eps), moe.router.weight.data_ptr(),
                s["w1"].data_ptr(), s["b1"].data_ptr(), s["w2"].data_ptr(), s["b2"].data_ptr(),
                moe.router.weight.shape[0], moe._expert_ids.numel(), s["w1"].shape[1],
                moe._router_logits.data_ptr(), moe._expert_ids.data_ptr(), moe._route_weights.data_ptr(),
                moe._expert_hidden.data_ptr(), moe._direct_out.data_ptr(), acc.data_ptr(),
            ), "mie_block_plan_init")
            if tables is not None:
                # Layer 0 with the embedding in its QKV launch: x is formed in
                # the row `x` (the block's _embed_row) from the token id and
                # the tables.
                w, pw = tables
                check(lib.mie_block_plan_set_embedding(plan, w.data_ptr(), w.shape[0], pw.data_ptr(), pw.shape[0],
                                                       x.data_ptr()), "mie_block_plan_set_embedding")

        init(None)

        def run(fn, arg, cache, position, stream):
            """One call of the plan.  A longer context splits into partitions:
            the call then fails before launching anything, and the plan is set
            up again with a workspace at least twice the last one."""
            if cache.graph_pos is None:
                cache._reserve(position + 1)
                counters, bound = None, position
            else:
                # Blocks were reserved before the replay; the launches read the
                # device [position, length] pair, bounded by the capacity.
                counters, bound = cache.graph_pos.data_ptr(), cache.graph_max_position
            rc = fn(plan, arg, counters, bound, stream)
            if rc == _native.ERR_WORKSPACE:
                _, need = decode_plan(1, heads, head_dim, block_size, bound + 1, dtype, 0)
                old = held["ws"]
                init(torch.empty(max(need, 0 if old is None else 2 * old.numel()), dtype=torch.uint8, device=device))
                rc = fn(plan, arg, counters, bound, stream)
            if rc:
                check(rc, "mie_block_decode")
            return out

        decode, decode_embed = lib.mie_block_decode, lib.mie_block_decode_embed

        def launch(x, cache, position):
            return run(decode, x.data_ptr(), cache, position, stream_of(x))

        def launch_embed(token_ids, cache, position):
            return run(decode_embed, token_ids.data_ptr(), cache, position, stream_of(token_ids))

        if tables is not None:
            launch.embed = launch_embed
        launch.out = out
        launch.plan = plan
        launch.held = held
        launch.buffers = (q, attn, h, acc, plan, held)  # kept alive with the plan
        return launch


class Model(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.max_seq_length = config.max_seq_length
        self.token_embedding = Embedding(config.vocab_size, config.hidden_dim)
        self.positional_embedding = Embedding(config.max_seq_length, config.hidden_dim)
        self.output_projection = Linear(config.hidden_dim, config.vocab_size)
        self.MoEBlocks = nn.ModuleList(TransformerMoEBlock(config) for _ in range(config.num_layers))
        self.final_norm = LayerNorm(config.hidden_dim)
        self.output_projection.weight = self.token_embedding.weight  # tied
        # The embedding and every block for one decode token as one library
        # call over the blocks' launch plans (_run_decode_step): step key ->
        # (cache weakref, plan array, launchers), the most recently used last.
        self._steps = collections.OrderedDict()

    def new_cache(self, batch_size: int = 1) -> KVCache:
        weight = self.token_embedding.weight
        return KVCache(self.config, batch_size, weight.device, weight.dtype)

    def set_moe_mode(self, mode: str) -> "Model":
        for block in self.MoEBlocks:
            block.moe.set_mode(mode)
        return self

    def new_block_allocator(self, num_blocks: int, block_size: int = 16, attention_mode: str = "auto") -> BlockAllocator:
        """A block pool on the model's device and dtype (model.py:529-541)."""
        weight = self.token_embedding.weight
        return BlockAllocator(self.config, num_blocks, block_size, weight.device, weight.dtype, attention_mode)

    def forward(self, token_ids, cache):
        x = self._hidden_states(token_ids, cache)
        if x.shape[0] == 1 and x.shape[1] == 1 and not torch.is_grad_enabled() and self._head_on_device(x):
            # One decode token at inference: final norm and LM head in one
            # launch (no autograd graph; with gradients on, the modules run).
            # The head keeps its workgroups' picks, so a greedy pick of these
            # logits (projection.argmax) is one small merge launch.
            return projection.lm_head(x.view(-1), self.final_norm, self.output_projection,
                                      keep_pick=True).view(1, 1, -1)
        return self.output_projection(self.final_norm(x))

    def _head_on_device(self, x) -> bool:
        w = self.output_projection.weight
        return (_native.is_rocm_device(x) and x.is_contiguous() and x.dtype == w.dtype
                and projection.supported(x.shape[-1], x.dtype) and w.is_contiguous())

    def hidden_states(self, token_ids, cache):
        """The forward pass up to the final norm (model.py:543-562): the
        embeddings and every block, advancing cache.position.  The result is
        the caller's (as the reference's is), never a buffer a later step
        overwrites."""
        x = self._hidden_states(token_ids, cache)
        if x.shape[:2] == (1, 1) and x.data_ptr() == self.MoEBlocks[-1].moe._direct_out.data_ptr():
            x = x.clone()  # one-token decode leaves the last block's output in its MoE buffer
        return x

    def _hidden_states(self, token_ids, cache):
        """hidden_states without the copy: for one decode token the result
        may be the last block's MoE output buffer, which the next token
        overwrites (Model.forward and the captured step consume it at once)."""
        batch, seq_len = token_ids.shape
        position = cache.position
        assert position + seq_len <= self.max_seq_length, "KV cache is full"
        graph_pos = getattr(cache, "graph_pos", None)
        decode = position > 0 and seq_len == 1
        one_token = decode and batch == 1 and len(self.MoEBlocks) and not torch.is_grad_enabled()
        if one_token and graph_pos is None:
            x = self._run_decode_step(token_ids, cache, position)
            if x is not None:
                cache.position += seq_len
                return x
        if decode:
            self._preflight_decode(batch)
        if one_token:
            # One decode token: the embedding inside layer 0's QKV launch when
            # its launch plan applies.
            x = self.MoEBlocks[0].decode_token_ids(token_ids, cache, position, self.token_embedding,
                                                   self.positional_embedding)
            if x is not None:
                for i in range(1, len(self.MoEBlocks)):
                    x = self.MoEBlocks[i](x, cache, i, position)
                cache.position += seq_len
                if graph_pos is None:
                    self._build_decode_step(token_ids, cache)
                return x
        if graph_pos is not None:  # device-side position (HIP-graph decode, moe_engine.graphs)
            x = embedding.embed(token_ids, graph_pos, self.token_embedding, self.positional_embedding)
        elif (batch == 1 and seq_len <= 65535 and token_ids.dtype == torch.int64 and token_ids.is_contiguous()
              and not torch.is_grad_enabled() and embedding.supported(self.token_embedding, self.positional_embedding)):
            # At inference, one launch for the two lookups and the add
            # (bit-identical sum).
            x = embedding.embed(token_ids, position, self.token_embedding, self.positional_embedding)
        else:
            pos = torch.arange(position, position + seq_len, device=token_ids.device)
            x = self.token_embedding(token_ids) + self.positional_embedding(pos)
        for i, block in enumerate(self.MoEBlocks):
            x = block(x, cache, i, position)
        cache.position += seq_len
        return x

    def _apply(self, fn, recurse=True):
        # A conversion replaces the tensors the kept steps' plans point at.
        self._steps.clear()
        return super()._apply(fn, recurse=recurse)

    def __getstate__(self):
        # Copies and pickles leave the decode steps behind (they point at this
        # model's buffers); a copy builds its own on first use.
        state = super().__getstate__().copy()
        state["_steps"] = collections.OrderedDict()
        return state

    @staticmethod
    def _step_key(token_ids, cache):
        """What a decode step is built for besides the blocks' plans: the
        cache (by identity, with a weak reference beside it), its attention
        mode, the allocator's fuse_qkv switch, the token's device and the
        tensor epoch, which every conversion, replacement, MoE mode or norm
        eps change advances - so the blocks' own plan keys hold too.  None
        for a cache without a block pool."""
        alloc = getattr(cache, "allocator", None)
        if alloc is None:
            return None
        return id(cache), cache.attention_mode, alloc.fuse_qkv, token_ids.device, _TENSOR_EPOCH[0]

    def _build_decode_step(self, token_ids, cache):
        """After a decode token ran block by block from launch plans (layer 0
        with the embedding inside its QKV launch), keep those plans as one
        step for the cache's next tokens.  The step holds the plans'
        launchers, which own their buffers, and no reference to the cache or
        its pools; the last few steps are kept, so sequences decoded in turn
        each find theirs."""
        key = self._step_key(token_ids, cache)
        if key is None:
            return
        step = self._steps.get(key)
        if step is not None and step[0]() is cache:
            return
        launchers = []
        for block in self.MoEBlocks:
            plan = block._one_token
            if plan is None or plan[2] is None or plan[1]() is not cache:
                return
            launchers.append(plan[2])
        if not hasattr(launchers[0], "embed"):
            return
        plans = (ctypes.c_void_p * len(launchers))(*(ctypes.addressof(l.plan) for l in launchers))
        self._steps[key] = (weakref.ref(cache), plans, launchers)
        self._steps.move_to_end(key)
        if len(self._steps) > _KEPT_PLANS:
            self._steps.popitem(last=False)

    def _run_decode_step(self, token_ids, cache, position):
        """The embedding and every block for one decode token in one call
        (mie_blocks_decode): the launches the blocks' plans make one by one,
        in the same order, with the host's per-block work gone from the time
        before the first launch.  None when no step was built for this key,
        or when a split context outgrew a plan's workspace (nothing launched;
        the blocks one by one then grow it)."""
        if not self._steps:
            return None
        key = self._step_key(token_ids, cache)
        step = self._steps.get(key)
        if step is None or step[0]() is not cache:
            return None
        if not (token_ids.dtype == torch.int64 and token_ids.numel() == 1 and token_ids.is_contiguous()):
            return None
        _, plans, launchers = step
        cache._reserve(position + 1)
        rc = _native.lib().mie_blocks_decode(plans, len(launchers), token_ids.data_ptr(), None, position,
                                             _native.stream_of(token_ids))
        if rc == _native.ERR_WORKSPACE:
            del self._steps[key]
            return None
        _native.check(rc, "mie_blocks_decode")
        return launchers[-1].out

    def _preflight_decode(self, batch):
        """A forced-direct MoE must fail before layer 0 writes K/V or reserves
        a block (the embedding touches no cache).  Only mode 'direct' can
        fail, so the others are skipped without a call."""
        for block in self.MoEBlocks:
            moe = block._modules["moe"]
            if moe.mode == "direct":
                moe.preflight_direct_decode(batch_size=batch)

    @torch.no_grad()
    def generate(self, token_ids, max_new_tokens, temperature=1.0, top_k=None, cache=None):
        """Generate one sequence; the caller owns a supplied cache (model.py:567-621)."""
        if not math.isfinite(temperature) or temperature < 0:
            raise ValueError("temperature must be a finite non-negative number")
        if top_k is not None and top_k <= 0:
            raise ValueError("top_k must be positive")
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be at least 1")
        if token_ids.dim() == 1:
            token_ids = token_ids.unsqueeze(0)
        token_ids = token_ids.to(self.token_embedding.weight.device).long()
        if token_ids.shape[0] != 1:
            raise ValueError("generate() handles one sequence; use batch size 1")
        if token_ids.shape[1] == 0:
            raise ValueError("prompt must contain at least one token")
        if token_ids.shape[1] > self.max_seq_length:
            raise ValueError(f"prompt is {token_ids.shape[1]} tokens; max_seq_length is {self.max_seq_length}")
        if cache is None:
            cache = self.new_cache(batch_size=1)
        if cache.position != 0:
            raise ValueError("generate() needs a fresh cache")

        out = token_ids
        step_input = token_ids
        for _ in range(max_new_tokens):
            logits = self(step_input, cache)[:, -1, :]
            if temperature == 0:
                if projection.can_argmax(logits.view(-1)):
                    next_token = projection.argmax(logits.view(-1)).view(1, 1)  # one launch, same pick
                else:
                    next_token = torch.argmax(logits, dim=-1, keepdim=True)
            else:
                logits = logits / temperature
                if top_k is not None:
                    kth = torch.topk(logits, min(top_k, logits.size(-1))).values[:, [-1]]
                    logits[logits < kth] = -float("inf")
                next_token = torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)
            if next_token == EOS_TOKEN_ID:
                return out
            out = torch.cat((out, next_token), dim=1)
            step_input = next_token
            if cache.position >= self.max_seq_length:
                break  # the sampled token has not entered the cache
        return out
