"""CPU restatement of the reference's paged-KV decode path.  TEST INFRASTRUCTURE ONLY.

Each function cites the reference (maokner/moe-inference-engine) lines it
restates.  Pools are [layers, blocks, heads, block_size, head_dim] as in
BlockAllocator (src/moe_engine/model.py:85-93).  Byte work (append, gather)
runs on numpy arrays of any dtype, including integer views of bf16 bit
patterns, so equality is bit equality.  Attention runs in float64.
"""

import math

import numpy as np
import torch
import torch.nn.functional as F


def raw_bits(t: torch.Tensor) -> np.ndarray:
    """Integer view of a CPU tensor's bit patterns (bf16 -> int16, f32 -> int32, ...)."""
    int_dtype = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.detach().cpu().contiguous().view(int_dtype).numpy()


def to_f64(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


# ---- KV append / gather (model.py:145-201) ---------------------------------


def append_rows(k_pool, v_pool, layer, block_table, position, k_new, v_new):
    """PagedKVCache.write after _reserve (model.py:167-184), one sequence.

    k_new, v_new: [H, S, D].  Row s goes to logical position p = position + s,
    i.e. pool[layer, block_table[p // BS], :, p % BS, :] (model.py:145-147,
    175-177 for S == 1; 182-184 for S > 1).
    """
    bs = k_pool.shape[3]
    for s in range(k_new.shape[1]):
        p = position + s
        blk, slot = block_table[p // bs], p % bs
        k_pool[layer, blk, :, slot, :] = k_new[:, s, :]
        v_pool[layer, blk, :, slot, :] = v_new[:, s, :]


def gather_rows(pool, layer, block_table, length):
    """PagedKVCache.read for one pool (model.py:186-201), without the batch axis.

    Takes the first ceil(length / BS) table entries, stacks their
    [H, BS, D] tiles, moves heads first and keeps `length` tokens: [H, length, D].
    """
    bs = pool.shape[3]
    nb = -(-length // bs)
    ids = np.asarray(list(block_table[:nb]), dtype=np.int64)
    tiles = pool[layer, ids]  # [nb, H, BS, D]
    heads, dim = pool.shape[2], pool.shape[4]
    return tiles.transpose(1, 0, 2, 3).reshape(heads, nb * bs, dim)[:, :length]


# ---- attention (paged_attention.py:46-110; model.py:265-266) ----------------


def attention_fp64(q, k, v, scale=None):
    """softmax(scale * q . k^T) . v per head, in float64.

    q [H, D]; k, v [H, C, D]; scale defaults to 1/sqrt(D) as in the reference
    wrapper (paged_attention.py:140).  C == 0 gives zeros, as
    torch.nn.functional.scaled_dot_product_attention does for no keys.
    """
    q, k, v = to_f64(q), to_f64(k), to_f64(v)
    heads, ctx, dim = k.shape
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if ctx == 0:
        return np.zeros((heads, dim))
    scores = np.einsum("hd,hcd->hc", q, k) * scale
    scores -= scores.max(axis=1, keepdims=True)
    weights = np.exp(scores)
    weights /= weights.sum(axis=1, keepdims=True)
    return np.einsum("hc,hcd->hd", weights, v)


def split_attention_fp64(q, k, v, partition, scale=None):
    """attention_fp64 computed as independent partitions merged by log-sum-exp.

    Partition i over tokens [i*P, (i+1)*P) yields m_i = max score,
    l_i = sum exp(s - m_i), acc_i = sum exp(s - m_i) v; with M = max m_i the
    result is sum exp(m_i - M) acc_i / sum exp(m_i - M) l_i.  This is the
    flash-decoding split the HIP kernels implement; it equals the unsplit
    softmax exactly in real arithmetic.
    """
    q, k, v = to_f64(q), to_f64(k), to_f64(v)
    heads, ctx, dim = k.shape
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if ctx == 0:
        return np.zeros((heads, dim))
    ms, ls, accs = [], [], []
    for start in range(0, ctx, partition):
        s = np.einsum("hd,hcd->hc", q, k[:, start : start + partition]) * scale
        m = s.max(axis=1)
        e = np.exp(s - m[:, None])
        ms.append(m)
        ls.append(e.sum(axis=1))
        accs.append(np.einsum("hc,hcd->hd", e, v[:, start : start + partition]))
    ms, ls, accs = np.stack(ms), np.stack(ls), np.stack(accs)  # [P, H], [P, H], [P, H, D]
    big = ms.max(axis=0)
    w = np.exp(ms - big[None])
    return (w[:, :, None] * accs).sum(axis=0) / (w * ls).sum(axis=0)[:, None]


# ---- QKV projection of a decode token (model.py:228-234, 478-481) ----------


def qkv_project_fp64(x, in_proj_weight, in_proj_bias, heads, norm_weight=None, norm_bias=None, eps=1e-5,
                     round_norm=None):
    """q, k, v [H, D] of one token, in float64.

    The block normalises x (attn_norm, a LayerNorm: (x - mean) / sqrt(var + eps)
    * w + b with the biased variance) when norm_weight is given, then the
    attention projects it with the packed in_proj (model.py:228-229) and splits
    the 3*dim outputs into q, k, v in that order, each viewed [H, D]
    (model.py:230-234).  `round_norm`, when given, maps the normalised vector
    to the values the model feeds the projection (a bf16 model rounds the norm
    output to bf16).
    """
    y = to_f64(x).reshape(-1)
    dim = y.shape[0]
    if norm_weight is not None:
        mean = y.mean()
        var = ((y - mean) ** 2).mean()
        y = (y - mean) / math.sqrt(var + eps) * to_f64(norm_weight)
        if norm_bias is not None:
            y = y + to_f64(norm_bias)
    if round_norm is not None:
        y = round_norm(y)
    qkv = to_f64(in_proj_weight) @ y
    if in_proj_bias is not None:
        qkv = qkv + to_f64(in_proj_bias)
    q, k, v = (qkv[i * dim : (i + 1) * dim].reshape(heads, dim // heads) for i in range(3))
    return q, k, v


# ---- the attention half of a block for one decode token (model.py:260-269, :495)


def attention_half_fp64(q, k, v, out_proj_weight, out_proj_bias, x, scale=None):
    """x + out_proj(attention) for one token, in float64.

    q [H, D]; k, v [H, C, D]; out_proj_weight [dim, dim] with dim = H * D;
    out_proj_bias [dim] or None; x [dim] (the block's input, the residual).
    The per-head attention outputs are concatenated head by head - the
    [1, H, 1, D] -> [1, 1, dim] reshape of CachedAttention.forward
    (model.py:269) - and projected (model.py:269), then added to x
    (model.py:495).  Returns (out_proj output, x + it).
    """
    a = attention_fp64(q, k, v, scale).reshape(-1)
    o = to_f64(out_proj_weight) @ a
    if out_proj_bias is not None:
        o = o + to_f64(out_proj_bias)
    return o, to_f64(x).reshape(-1) + o


def gather_sdpa(q, k_pool, v_pool, layer, block_table, context_len):
    """The reference's gather decode path on the CPU: PagedKVCache.read
    (model.py:186-201) then scaled_dot_product_attention (model.py:265-266).

    q [1, H, 1, D] torch; pools torch [L, NB, H, BS, D]; returns [1, H, 1, D].
    """
    bs = k_pool.shape[3]
    ids = list(block_table[: -(-context_len // bs)])

    def rebuild(pool):
        tiles = pool[layer, ids]
        return tiles.transpose(0, 1).reshape(pool.shape[2], -1, pool.shape[4])[:, :context_len].unsqueeze(0)

    return F.scaled_dot_product_attention(q, rebuild(k_pool), rebuild(v_pool))


def batched_gather_sdpa(q, k_pool, v_pool, layer, block_tables, context_lens):
    """gather_sdpa for each sequence of a batch: q [B, H, D] -> [B, H, D]."""
    outs = []
    for b, (table, ctx) in enumerate(zip(block_tables, context_lens)):
        outs.append(gather_sdpa(q[b][None, :, None], k_pool, v_pool, layer, table, int(ctx))[0, :, 0])
    return torch.stack(outs)


# ---- allocator (model.py:94-143) --------------------------------------------


class LifoAllocator:
    """BlockAllocator's free list (model.py:94-105): pop from the end."""

    def __init__(self, num_blocks):
        self.free_blocks = list(range(num_blocks))

    def allocate(self):
        if not self.free_blocks:
            raise RuntimeError("no free KV cache blocks left")
        return self.free_blocks.pop()

    def free(self, ids):
        self.free_blocks.extend(ids)


def reserve(block_table, allocator, num_tokens, block_size):
    """PagedKVCache._reserve (model.py:125-143): all-or-nothing growth of
    `block_table` (a list, modified in place) to ceil(num_tokens / block_size)
    blocks; on exhaustion the blocks taken so far go back and the error is
    re-raised.  Returns the newly taken ids."""
    needed = -(-num_tokens // block_size)
    taken = []
    try:
        while len(block_table) + len(taken) < needed:
            taken.append(allocator.allocate())
    except RuntimeError:
        allocator.free(taken)
        raise
    block_table.extend(taken)
    return taken
