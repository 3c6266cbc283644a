"""Seeded synthetic paged-KV workloads for benchmarks and tests.

BASELINE configs 2-5 are kernel-level workloads: B sequences with given
context lengths in one shared pool [layers, blocks, heads, block_size,
head_dim].  Pools are filled with ATen advanced indexing following the
reference's prefill scatter (src/moe_engine/model.py:182-184), so building a
workload never runs the kernels being measured or tested.
"""

from dataclasses import dataclass

import torch


@dataclass
class Workload:
    k_pool: torch.Tensor  # [L, NB, H, BS, D]
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # int32 [B, max_blocks] on the device
    context_lens: torch.Tensor  # int32 [B] on the device
    lens: list  # host copy of context_lens
    tables: list  # host copy of the tables (lists of block ids)
    q: torch.Tensor  # [B, H, D]
    layer: int

    @property
    def max_len(self):
        return max(self.lens) if self.lens else 0

    @property
    def block_size(self):
        return self.k_pool.shape[3]


def scatter_tokens(pool, layer, table, k):
    """pool[layer, table[t // BS], :, t % BS] = k[:, t] for t < k.shape[1] (ATen indexing).

    k is [H, C, D]; the indexed store gives [C, H, D] rows, hence the transpose,
    as in the reference's prefill write (model.py:182-184).
    """
    bs = pool.shape[3]
    t = torch.arange(k.shape[1], device=pool.device)
    ids = torch.as_tensor(table, dtype=torch.long, device=pool.device)[t // bs]
    pool[layer, ids, :, t % bs] = k.transpose(0, 1)


def make_workload(
    lens,
    num_heads=12,
    head_dim=64,
    block_size=16,
    num_blocks=None,
    dtype=torch.bfloat16,
    seed=0,
    layers=1,
    layer=0,
    heavy_fraction=0.0,
    heavy_scale=20.0,
    device="cuda",
):
    """B sequences with the given context lengths sharing one pool.

    Block ids come from one random permutation of the pool dealt to the
    sequences in order, so each table is a random non-contiguous shuffle over
    the shared pool.  K, V, q ~ N(0, 1) from `seed`; a `heavy_fraction` of the
    keys is multiplied by `heavy_scale` to stress the online-softmax max.
    """
    lens = [int(c) for c in lens]
    need = [-(-c // block_size) for c in lens]
    if num_blocks is None:
        num_blocks = max(1, sum(need))
    if sum(need) > num_blocks:
        raise ValueError(f"{sum(need)} blocks needed, pool has {num_blocks}")
    gen = torch.Generator(device=device).manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    tables, start = [], 0
    for n in need:
        tables.append(perm[start : start + n])
        start += n
    shape = (layers, num_blocks, num_heads, block_size, head_dim)
    k_pool = torch.zeros(shape, dtype=dtype, device=device)
    v_pool = torch.zeros(shape, dtype=dtype, device=device)
    for table, ctx in zip(tables, lens):
        if ctx == 0:
            continue
        k = torch.randn(num_heads, ctx, head_dim, generator=gen, device=device)
        v = torch.randn(num_heads, ctx, head_dim, generator=gen, device=device)
        if heavy_fraction > 0:
            heavy = torch.rand(ctx, generator=gen, device=device) < heavy_fraction
            k[:, heavy] *= heavy_scale
        scatter_tokens(k_pool, layer, table, k.to(dtype))
        scatter_tokens(v_pool, layer, table, v.to(dtype))
    width = max([1] + need)
    bt = torch.zeros(len(lens), width, dtype=torch.int32)
    for b, table in enumerate(tables):
        bt[b, : len(table)] = torch.tensor(table, dtype=torch.int32)
    q = torch.randn(len(lens), num_heads, head_dim, generator=gen, device=device).to(dtype)
    return Workload(
        k_pool=k_pool,
        v_pool=v_pool,
        block_tables=bt.to(device),
        context_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        lens=lens,
        tables=tables,
        q=q,
        layer=layer,
    )


def sequence_kv(w: Workload, b: int):
    """Contiguous K, V [H, C, D] of sequence b, read with ATen indexing."""
    ctx = w.lens[b]
    bs = w.block_size
    t = torch.arange(ctx, device=w.k_pool.device)
    ids = torch.as_tensor(w.tables[b], dtype=torch.long, device=w.k_pool.device)[t // bs]
    return (
        w.k_pool[w.layer, ids, :, t % bs].transpose(0, 1),
        w.v_pool[w.layer, ids, :, t % bs].transpose(0, 1),
    )


def attention_bytes(lens, num_heads, head_dim, block_size, elt):
    """Algorithmic bytes of one decode-attention call: every K and V row once,
    q read and out written once, one 4-byte table entry per block."""
    kv = sum(lens) * num_heads * head_dim * 2 * elt
    qo = 2 * len(lens) * num_heads * head_dim * elt
    tables = sum(-(-c // block_size) for c in lens) * 4
    return kv + qo + tables


def append_bytes(batch, num_heads, head_dim, elt, layers=1):
    """Algorithmic bytes of appending one token per sequence: K and V rows read and written."""
    return layers * batch * 4 * num_heads * head_dim * elt


def gather_bytes(context, num_heads, head_dim, elt, layers=1):
    """Algorithmic bytes of gathering `context` tokens of K and V: read and write."""
    return layers * 4 * context * num_heads * head_dim * elt


def cfg4_lens(batch=64, low=512, high=8192, seed=2):
    """Context lengths of BASELINE config 4: U[low, high] from `seed`."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(low, high + 1, (batch,), generator=g).tolist()


def take_last_tokens(w: Workload):
    """Each sequence's last context token's K/V rows ([B, H, D] each), read
    from the pool and then zeroed there: a decode step that appends them
    (its new token is its last context token) restores the pool exactly."""
    heads, dim = w.k_pool.shape[2], w.k_pool.shape[4]
    bs = w.block_size
    k_new = torch.zeros(len(w.lens), heads, dim, dtype=w.k_pool.dtype, device=w.k_pool.device)
    v_new = torch.zeros_like(k_new)
    for b, ctx in enumerate(w.lens):
        if ctx == 0:
            continue
        blk, slot = w.tables[b][(ctx - 1) // bs], (ctx - 1) % bs
        k_new[b] = w.k_pool[w.layer, blk, :, slot]
        v_new[b] = w.v_pool[w.layer, blk, :, slot]
        w.k_pool[w.layer, blk, :, slot] = 0
        w.v_pool[w.layer, blk, :, slot] = 0
    return k_new, v_new


@dataclass
class DecodeStep:
    """One decode step of one layer over a batch: every sequence's new token
    (its last context token, rows k_new / v_new [B, H, D]) is appended
    through its block table and attended to together with the rest of its
    context.  `fused()` is one mie_paged_decode_append call; `append()` then
    `attend()` is the same step as the append launch and the decode launch.
    bench.py times exactly these calls."""

    w: Workload
    k_new: torch.Tensor
    v_new: torch.Tensor
    out: torch.Tensor
    partition_tokens: int = 0

    def __post_init__(self):
        # Position of each new token: its sequence's last slot (an empty
        # sequence gets -1, which the append skips).
        self.positions = (self.w.context_lens - 1).contiguous()

    def fused(self):
        from moe_engine import paged_attention

        w = self.w
        return paged_attention.decode_batched(
            w.q, w.k_pool, w.v_pool, w.layer, w.block_tables, w.context_lens, w.max_len,
            out=self.out, partition_tokens=self.partition_tokens, context_lens_host=w.lens,
            k_new=self.k_new, v_new=self.v_new,
        )

    def append(self):
        from moe_engine import kv_ops

        w = self.w
        kv_ops.append(w.k_pool, w.v_pool, w.layer, self.k_new[:, :, None], self.v_new[:, :, None],
                      w.block_tables, positions=self.positions)

    def attend(self):
        from moe_engine import paged_attention

        w = self.w
        return paged_attention.decode_batched(
            w.q, w.k_pool, w.v_pool, w.layer, w.block_tables, w.context_lens, w.max_len,
            out=self.out, partition_tokens=self.partition_tokens, context_lens_host=w.lens,
        )


def config4_step(out_dtype=torch.bfloat16, partition_tokens=0, device="cuda"):
    """BASELINE config 4's decode step: 64 sequences, contexts U[512, 8192]
    (seed 2), 12 x 64, block 16, bf16, tables shuffled over a shared
    40000-block pool; the new rows are the sequences' last tokens, taken out
    of the pool (take_last_tokens).  Output [64, 12, 64] in out_dtype."""
    lens = cfg4_lens()
    w = make_workload(lens, block_size=16, num_blocks=40000, dtype=torch.bfloat16, seed=2, device=device)
    k_new, v_new = take_last_tokens(w)
    out = torch.empty(len(lens), 12, 64, dtype=out_dtype, device=device)
    return DecodeStep(w, k_new, v_new, out, partition_tokens)


NORTH_STAR_BATCH, NORTH_STAR_CONTEXT = 64, 8192


def north_star_step(out_dtype=torch.bfloat16, partition_tokens=0, device="cuda"):
    """The north star's literal target shape: 64 sequences of 8192 tokens
    each, 12 x 64, block 16, bf16, tables shuffled over a shared 40000-block
    pool (32768 blocks used), seed 3; the decode step as config4_step builds
    it (new rows taken out of the pool).  Output [64, 12, 64] in out_dtype."""
    lens = [NORTH_STAR_CONTEXT] * NORTH_STAR_BATCH
    w = make_workload(lens, block_size=16, num_blocks=40000, dtype=torch.bfloat16, seed=3, device=device)
    k_new, v_new = take_last_tokens(w)
    out = torch.empty(len(lens), 12, 64, dtype=out_dtype, device=device)
    return DecodeStep(w, k_new, v_new, out, partition_tokens)
