"""HIP KV append and gather on the GPU: bit-exact against the oracle.

Append is checked by comparing the WHOLE pool (bit patterns) with the oracle's
append_rows applied to a CPU copy of the initial pool, so rows that must not
change are covered too.  Gather is checked against the oracle's gather_rows
and, at BASELINE config 3's full size, by the size-independent round trip
(ATen scatter of contiguous K/V -> HIP append of the new token -> HIP gather
returns the contiguous K/V, bit for bit).
"""

import random

import numpy as np
import pytest
import torch

from conftest import print_case
from moe_engine import kv_ops
from moe_engine.model import BlockAllocator, ModelConfig
from oracle import paged_ref as ref
from paged_cases import scatter_tokens

pytestmark = pytest.mark.gpu

CFG = dict(max_seq_length=256, vocab_size=96, num_layers=2, hidden_dim=48, num_heads=3)


def randn(shape, dtype, gen):
    return torch.randn(shape, generator=gen).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("block_size", [1, 3, 4, 16, 32])
def test_paged_cache_write_read_bit_exact(dtype, block_size):
    """Prefill then decode writes through PagedKVCache on the GPU, against the
    oracle on a CPU copy of the pool; then the gather of every prefix length."""
    print_case("kv write/read", dtype, block_size)
    cfg = ModelConfig(**CFG)
    gen = torch.Generator().manual_seed(block_size)
    num_blocks = -(-cfg.max_seq_length // block_size)
    allocator = BlockAllocator(cfg, num_blocks, block_size, "cuda", dtype)
    random.Random(block_size).shuffle(allocator.free_blocks)
    # Non-zero initial pools so a stray or missing write cannot hide.
    allocator.k_pool.copy_(randn(allocator.k_pool.shape, dtype, gen))
    allocator.v_pool.copy_(randn(allocator.v_pool.shape, dtype, gen))
    want_k, want_v = ref.raw_bits(allocator.k_pool).copy(), ref.raw_bits(allocator.v_pool).copy()
    cache = allocator.new_cache()
    H, D = cfg.num_heads, cfg.head_dim
    ctx = 3 * block_size + 7
    k = randn((1, H, ctx, D), dtype, gen)
    v = randn((1, H, ctx, D), dtype, gen)
    prefill = ctx - 4
    for layer in range(cfg.num_layers):
        cache.write(layer, 0, k[:, :, :prefill].cuda(), v[:, :, :prefill].cuda())
    for p in range(prefill, ctx):
        for layer in range(cfg.num_layers):
            cache.write(layer, p, k[:, :, p : p + 1].cuda(), v[:, :, p : p + 1].cuda())
    for layer in range(cfg.num_layers):
        ref.append_rows(want_k, want_v, layer, cache.block_table, 0, ref.raw_bits(k[0]), ref.raw_bits(v[0]))
    assert np.array_equal(ref.raw_bits(allocator.k_pool), want_k)
    assert np.array_equal(ref.raw_bits(allocator.v_pool), want_v)
    for length in sorted({0, 1, block_size, block_size + 1, ctx}):
        for layer in range(cfg.num_layers):
            rk, rv = cache.read(layer, length)
            assert rk.shape == (1, H, length, D) and rk.dtype == dtype
            assert np.array_equal(ref.raw_bits(rk[0]), ref.gather_rows(want_k, layer, cache.block_table, length))
            assert np.array_equal(ref.raw_bits(rv[0]), ref.gather_rows(want_v, layer, cache.block_table, length))


def test_append_reads_strided_qkv_views():
    """CachedAttention hands the append views of the fused QKV projection
    ([B, S, 3*dim] chunked); they are read in place, no copy."""
    gen = torch.Generator().manual_seed(3)
    H, D, S = 4, 16, 5
    qkv = randn((1, S, 3 * H * D), torch.float32, gen).cuda()
    q, k, v = (t.view(1, S, H, D).transpose(1, 2) for t in qkv.chunk(3, dim=-1))
    assert not k.is_contiguous()
    k_pool = torch.zeros(1, 4, H, 2, D, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    table = torch.tensor([3, 0, 2, 1], dtype=torch.int32, device="cuda")
    kv_ops.append(k_pool, v_pool, 0, k, v, table, position=1)
    wk, wv = np.zeros((1, 4, H, 2, D), np.float32), np.zeros((1, 4, H, 2, D), np.float32)
    ref.append_rows(wk, wv, 0, [3, 0, 2, 1], 1, k[0].cpu().numpy(), v[0].cpu().numpy())
    assert np.array_equal(k_pool.cpu().numpy(), wk) and np.array_equal(v_pool.cpu().numpy(), wv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_batched_append_with_device_positions(dtype):
    """One launch appends a token to each of B sequences at their own positions."""
    gen = torch.Generator().manual_seed(5)
    B, H, D, BS, NB = 6, 12, 64, 16, 64
    positions = [0, 15, 16, 17, 100, 127]  # rows hold 8 blocks = 128 tokens
    perm = torch.randperm(NB, generator=gen)
    tables = perm[: B * 8].view(B, 8).to(torch.int32)
    k_pool = randn((2, NB, H, BS, D), dtype, gen).cuda()
    v_pool = randn((2, NB, H, BS, D), dtype, gen).cuda()
    want_k, want_v = ref.raw_bits(k_pool).copy(), ref.raw_bits(v_pool).copy()
    k_new = randn((B, H, 1, D), dtype, gen)
    v_new = randn((B, H, 1, D), dtype, gen)
    pos_dev = torch.tensor(positions, dtype=torch.int32, device="cuda")
    kv_ops.append(k_pool, v_pool, 1, k_new.cuda(), v_new.cuda(), tables.cuda(), positions=pos_dev)
    for b in range(B):
        ref.append_rows(want_k, want_v, 1, tables[b].tolist(), positions[b], ref.raw_bits(k_new[b]), ref.raw_bits(v_new[b]))
    assert np.array_equal(ref.raw_bits(k_pool), want_k) and np.array_equal(ref.raw_bits(v_pool), want_v)


def test_append_skips_out_of_range_block_ids():
    """A table entry past the pool, or a position past the table row, is
    bounds-checked in the kernel: that row is not written, every other row is."""
    k_pool = torch.zeros(1, 4, 2, 4, 8, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    tables = torch.tensor([[1], [99], [2]], dtype=torch.int32, device="cuda")
    k_new = torch.ones(3, 2, 1, 8, device="cuda")
    positions = torch.tensor([2, 2, 4], dtype=torch.int32, device="cuda")  # 4 // 4 = block 1: past the row
    kv_ops.append(k_pool, v_pool, 0, k_new, -k_new, tables, positions=positions)
    assert k_pool[0, 1, :, 2].eq(1).all() and v_pool[0, 1, :, 2].eq(-1).all()
    assert k_pool.sum().item() == 16 and v_pool.sum().item() == -16


def test_gather_leaves_rows_of_out_of_pool_blocks_unwritten():
    """Table entries of -1 or past the pool are never read: the gather leaves
    those tokens' output rows as they were, and copies every other token
    exactly (the oracle's gather over the valid blocks)."""
    NB, H, BS, D = 6, 3, 4, 8
    gen = torch.Generator().manual_seed(11)
    k_pool = torch.randn(2, NB, H, BS, D, generator=gen)
    v_pool = torch.randn(2, NB, H, BS, D, generator=gen)
    table = [4, -1, NB, 0, 2]  # blocks 1 and 2 of the sequence are outside the pool
    length = 4 * BS + 3  # the last block is partial
    sentinel = 7.0
    out_k = torch.full((1, H, length, D), sentinel, device="cuda")
    out_v = torch.full((1, H, length, D), -sentinel, device="cuda")
    kv_ops.gather(k_pool.cuda(), v_pool.cuda(), 1, torch.tensor(table, dtype=torch.int32, device="cuda"), length,
                  out_k, out_v)
    got_k, got_v = out_k[0].cpu(), out_v[0].cpu()
    for j, blk in enumerate(table):
        rows = slice(j * BS, min(length, (j + 1) * BS))
        if 0 <= blk < NB:
            n = rows.stop - rows.start
            assert torch.equal(got_k[:, rows], k_pool[1, blk, :, :n])
            assert torch.equal(got_v[:, rows], v_pool[1, blk, :, :n])
        else:
            assert got_k[:, rows].eq(sentinel).all() and got_v[:, rows].eq(-sentinel).all()
    # Against the oracle wherever the table is valid: substitute a valid id and
    # compare only the valid blocks' rows.
    want_k = ref.gather_rows(ref.raw_bits(k_pool), 1, [b if 0 <= b < NB else 0 for b in table], length)
    valid = np.concatenate([np.full(min(length, (j + 1) * BS) - j * BS, 0 <= b < NB) for j, b in enumerate(table)])
    assert np.array_equal(ref.raw_bits(got_k)[:, valid], want_k[:, valid])


@pytest.mark.parametrize("context", [128, 1024, 8192])
def test_config3_append_and_gather_round_trip(context):
    """12 layers, 12 x 64, bf16, block 16, random tables
    over a 65536-block pool; append one token per layer, then gather the full
    context of every layer back to contiguous, bit for bit."""
    print_case("config3", context)
    L, NB, H, BS, D = 12, 65536, 12, 16, 64
    dtype = torch.bfloat16
    gen = torch.Generator(device="cuda").manual_seed(context)
    k_pool = torch.zeros(L, NB, H, BS, D, dtype=dtype, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    nblk = -(-(context + 1) // BS)
    table = torch.randperm(NB, generator=torch.Generator().manual_seed(context))[:nblk].tolist()
    table_dev = torch.zeros(NB, dtype=torch.int32, device="cuda")
    table_dev[:nblk] = torch.tensor(table, dtype=torch.int32)
    truth_k = torch.randn(L, H, context + 1, D, generator=gen, device="cuda").to(dtype)
    truth_v = torch.randn(L, H, context + 1, D, generator=gen, device="cuda").to(dtype)
    for layer in range(L):
        scatter_tokens(k_pool, layer, table, truth_k[layer, :, :context])
        scatter_tokens(v_pool, layer, table, truth_v[layer, :, :context])
    for layer in range(L):  # decode step: one new token per layer
        kv_ops.append(
            k_pool, v_pool, layer,
            truth_k[layer, None, :, context : context + 1], truth_v[layer, None, :, context : context + 1],
            table_dev, position=context,
        )
    for layer in range(L):
        gk, gv = kv_ops.gather(k_pool, v_pool, layer, table_dev, context + 1)
        assert torch.equal(gk[0].view(torch.int16), truth_k[layer].view(torch.int16))
        assert torch.equal(gv[0].view(torch.int16), truth_v[layer].view(torch.int16))
