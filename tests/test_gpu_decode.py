"""Direct paged decode attention on the GPU against the CPU oracle.

Tolerances: float32 inputs within 1e-5 absolute of the
float64 oracle; bf16 inputs with float32 output within 2e-3 absolute of the
float64 oracle on the same bf16 values; bf16 output within 2e-3 + 2^-8 |ref|
(one bf16 ULP above |o| = 0.25 exceeds 2e-3, so the bf16-rounded output gets a
relative term; see paged_cases.bf16_close).

Cases follow the reference's kernel tests (tests/test_paged_attention.py:64-124)
at its production shape (8 heads x 96, float32) and BASELINE configs 2, 4, 5
at 12 heads x 64.
"""

import math

import numpy as np
import pytest
import torch

from conftest import print_case
from moe_engine import _native, paged_attention
from moe_engine.model import BlockAllocator, ModelConfig
from oracle import paged_ref as ref
from paged_cases import bf16_close, cfg4_lens, make_workload, oracle_outputs, sequence_kv, take_last_tokens

pytestmark = pytest.mark.gpu

PROD = dict(max_seq_length=1024, vocab_size=96, num_layers=1, hidden_dim=768, num_heads=8)
TINY = dict(max_seq_length=128, vocab_size=96, num_layers=2, hidden_dim=32, num_experts=4, top_k=2)


def filled_cache(config, context_len, block_size, shuffle=False, seed=0, dtype=torch.float32):
    """A paged cache whose every layer holds `context_len` random tokens,
    written through the product's PagedKVCache.write (the HIP append).
    Returns the cache and the per-layer contiguous K/V that were written."""
    cfg = ModelConfig(**config)
    num_blocks = -(-cfg.max_seq_length // block_size)
    allocator = BlockAllocator(cfg, num_blocks, block_size, "cuda", dtype)
    if shuffle:
        import random

        random.Random(seed).shuffle(allocator.free_blocks)
    cache = allocator.new_cache()
    g = torch.Generator().manual_seed(seed)
    shape = (1, cfg.num_heads, context_len, cfg.head_dim)
    written = []
    for layer in range(cfg.num_layers):
        k = torch.randn(shape, generator=g).to(dtype)
        v = torch.randn(shape, generator=g).to(dtype)
        cache.write(layer, 0, k.cuda(), v.cuda())
        written.append((k[0], v[0]))
    cache.position = context_len
    return cache, written


def oracle(q, kv):
    k, v = kv
    return ref.attention_fp64(ref.to_f64(q[0, :, 0]), ref.to_f64(k), ref.to_f64(v))


@pytest.mark.parametrize("context_len", [1, 15, 16, 17, 31, 32, 63, 64, 190, 1024])
def test_kernel_matches_oracle_production_shape(context_len):
    print_case("prod-shape fp32", context_len)
    cache, written = filled_cache(PROD, context_len, 16)
    q = torch.randn(1, 8, 1, 96, generator=torch.Generator().manual_seed(context_len))
    got = paged_attention.decode(q.cuda(), cache, 0, context_len)
    assert got.shape == (1, 8, 1, 96) and got.dtype == torch.float32
    np.testing.assert_allclose(got[0, :, 0].cpu().numpy(), oracle(q, written[0]), rtol=0, atol=1e-5)


@pytest.mark.parametrize("context_len", [17, 190])
def test_kernel_handles_noncontiguous_blocks(context_len):
    print_case("noncontiguous", context_len)
    cache, written = filled_cache(PROD, context_len, 16, shuffle=True, seed=5)
    table = cache.block_table
    # The shuffled pool must really scatter the context: some two logical
    # neighbours are not neighbours in the pool.
    assert any(abs(b - a) != 1 for a, b in zip(table, table[1:]))
    q = torch.randn(1, 8, 1, 96, generator=torch.Generator().manual_seed(1))
    got = paged_attention.decode(q.cuda(), cache, 0, context_len)
    np.testing.assert_allclose(got[0, :, 0].cpu().numpy(), oracle(q, written[0]), rtol=0, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("block_size", [4, 16, 32])
def test_kernel_handles_other_block_sizes(block_size, dtype):
    """Partial final blocks at several block sizes, 8 heads of dim 4."""
    for context_len in [1, block_size - 1, block_size, block_size + 1, 3 * block_size + 2]:
        if context_len == 0:
            continue
        print_case("tiny", block_size, dtype, context_len)
        cache, written = filled_cache(TINY, context_len, block_size, dtype=dtype)
        q = torch.randn(1, 8, 1, 4, generator=torch.Generator().manual_seed(context_len)).to(dtype)
        got = paged_attention.decode_layer(
            q[:, :, 0].cuda(), cache.allocator.k_pool[0], cache.allocator.v_pool[0], cache.block_table_device,
            context_len=context_len, out_dtype=torch.float32,
        )
        atol = 1e-5 if dtype == torch.float32 else 2e-3
        np.testing.assert_allclose(got[0].cpu().numpy(), oracle(q, written[0]), rtol=0, atol=atol)


def test_kernel_matches_oracle_on_every_layer():
    """Distinct K/V per layer: reading the wrong layer cannot pass."""
    cache, written = filled_cache(dict(PROD, num_layers=3), 40, 16, seed=3)
    q = torch.randn(1, 8, 1, 96, generator=torch.Generator().manual_seed(3))
    oracles = [oracle(q, written[layer]) for layer in range(3)]
    assert not np.allclose(oracles[0], oracles[1])
    for layer in range(3):
        got = paged_attention.decode(q.cuda(), cache, layer, 40)[0, :, 0].cpu().numpy()
        np.testing.assert_allclose(got, oracles[layer], rtol=0, atol=1e-5)
        for other in range(3):
            if other != layer:
                assert not np.allclose(got, oracles[other], atol=1e-3, rtol=1e-3)


def check_workload(w, out_f32_atol=2e-3, partition_tokens=0, batches=None):
    """float32 output from a launch sized by max_context_len (surplus
    workgroups exit), then output in the input dtype from a launch sized
    exactly from host lengths; both against the float64 oracle."""
    want = oracle_outputs(w, batches)
    sel = slice(None) if batches is None else list(batches)
    dt = w.q.dtype
    got32 = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, w.layer, w.block_tables, w.context_lens, w.max_len,
        out_dtype=torch.float32, partition_tokens=partition_tokens,
    )
    np.testing.assert_allclose(got32.cpu().numpy()[sel], want, rtol=0, atol=out_f32_atol)
    got = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, w.layer, w.block_tables, w.context_lens, w.max_len,
        partition_tokens=partition_tokens, context_lens_host=w.lens,
    )
    assert got.dtype == dt
    if dt == torch.float32:
        np.testing.assert_allclose(got.cpu().numpy()[sel], want, rtol=0, atol=out_f32_atol)
    else:
        assert bf16_close(got.float().cpu().numpy()[sel], want)
    return got32


def test_config2_single_layer_bf16():
    """batch 1, 12 x 64, context 2048 (the new token is the
    2048th), block 16, bf16, table = random permutation over 4096 blocks; the
    new token's K/V is appended with the HIP append before attention."""
    print_case("config2")
    w = make_workload([2047], block_size=16, num_blocks=4096, dtype=torch.bfloat16, seed=1)
    g = torch.Generator(device="cuda").manual_seed(11)
    k_new = torch.randn(1, 12, 1, 64, generator=g, device="cuda").to(torch.bfloat16)
    v_new = torch.randn(1, 12, 1, 64, generator=g, device="cuda").to(torch.bfloat16)
    table = w.tables[0]  # 128 blocks: position 2047 is slot 15 of the last one
    assert len(table) == 128
    full_table = torch.zeros(4096, dtype=torch.int32, device="cuda")
    full_table[: len(table)] = torch.tensor(table, dtype=torch.int32)
    from moe_engine import kv_ops

    kv_ops.append(w.k_pool, w.v_pool, 0, k_new, v_new, full_table, position=2047)
    w.lens[0] = 2048
    w.context_lens.fill_(2048)
    w.block_tables = full_table[None, :128].contiguous()
    check_workload(w)
    # The single-sequence reference API on the same data.
    k, v = sequence_kv(w, 0)
    want = ref.attention_fp64(ref.to_f64(w.q[0]), ref.to_f64(k), ref.to_f64(v))
    got = paged_attention.decode_layer(
        w.q[0:1], w.k_pool[0], w.v_pool[0], full_table, context_len=2048, out_dtype=torch.float32
    )
    np.testing.assert_allclose(got[0].cpu().numpy(), want, rtol=0, atol=2e-3)


def test_config4_batched_64_sequences_bf16():
    """64 sequences, contexts U[512, 8192] (seed 2),
    12 x 64, block 16, bf16, shuffled tables over a shared 40000-block pool."""
    lens = cfg4_lens()
    print_case("config4", sum(lens))
    w = make_workload(lens, block_size=16, num_blocks=40000, dtype=torch.bfloat16, seed=2)
    check_workload(w)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_config4_timed_step(out_dtype):
    """The step bench.py times, through the same object (workloads.config4_step):
    one mie_paged_decode_append call over config 4 with the new rows passed in,
    host lengths (longest-first order) and the automatic plan.  The new rows
    were taken out of the pool, so only the launch's stores can put them back:
    afterwards both pools are bit-identical to the workload as built, and
    every sequence's output is the oracle's attention over its full context.
    A second call (the bench repeats the step) gives the same bits."""
    from moe_engine import workloads

    print_case("config4 timed step", out_dtype)
    lens = cfg4_lens()
    built = make_workload(lens, block_size=16, num_blocks=40000, dtype=torch.bfloat16, seed=2)
    step = workloads.config4_step(out_dtype=out_dtype)
    w = step.w
    assert w.lens == built.lens and w.tables == built.tables
    assert not torch.equal(w.k_pool, built.k_pool), "the new rows must be missing before the step"
    want = oracle_outputs(built)
    got = step.fused().clone()
    assert torch.equal(w.k_pool.view(torch.int16), built.k_pool.view(torch.int16))
    assert torch.equal(w.v_pool.view(torch.int16), built.v_pool.view(torch.int16))
    assert got.dtype == out_dtype and got.shape == (64, 12, 64)
    if out_dtype == torch.float32:
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=0, atol=2e-3)
    else:
        assert bf16_close(got.float().cpu().numpy(), want)
    again = step.fused()
    assert np.array_equal(ref.raw_bits(got.cpu()), ref.raw_bits(again.cpu()))


def test_north_star_64_sequences_of_8192_tokens():
    """The north star's literal shape, 64 x 8192 uniform (bench.py's
    north_star_64x8192 figure times exactly this step object): one
    mie_paged_decode_append call puts the missing new rows back bit for bit,
    and every sequence's float32 output is the oracle's attention over its
    full 8192-token context within 2e-3; the bf16-output step as well."""
    from moe_engine import workloads

    print_case("north star 64 x 8192")
    step = workloads.north_star_step(out_dtype=torch.float32)
    w = step.w
    assert w.lens == [8192] * 64 and sum(len(t) for t in w.tables) == 64 * 512
    part, ws = _native.decode_plan(64, 12, 64, 16, 8192, torch.bfloat16, 0)
    assert ws == 0 and part >= 8192  # the workgroup form, one launch
    k_missing, v_missing = w.k_pool.clone(), w.v_pool.clone()
    got = step.fused().clone()
    k_full, v_full = w.k_pool.clone(), w.v_pool.clone()
    for b, table in enumerate(w.tables):  # the step wrote exactly the new rows
        blk = table[-1]
        assert torch.equal(k_full[0, blk, :, 15].view(torch.int16), step.k_new[b].view(torch.int16))
        assert torch.equal(v_full[0, blk, :, 15].view(torch.int16), step.v_new[b].view(torch.int16))
        k_missing[0, blk, :, 15] = k_full[0, blk, :, 15]
        v_missing[0, blk, :, 15] = v_full[0, blk, :, 15]
    assert torch.equal(k_missing.view(torch.int16), k_full.view(torch.int16))
    assert torch.equal(v_missing.view(torch.int16), v_full.view(torch.int16))
    del k_missing, v_missing, k_full, v_full
    want = oracle_outputs(w)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=0, atol=2e-3)
    step.out = torch.empty(64, 12, 64, dtype=torch.bfloat16, device="cuda")
    assert bf16_close(step.fused().float().cpu().numpy(), want)


def test_config4_unfused_step():
    """bench.py --unfused: the append launch, then the decode launch, leave
    the pools the fused step leaves, and both outputs are the oracle's (the
    fused launch scores the new token from registers, so the two may differ
    in the last bits)."""
    from moe_engine import workloads

    print_case("config4 unfused step")
    step = workloads.config4_step(out_dtype=torch.float32)
    k_missing, v_missing = step.w.k_pool.clone(), step.w.v_pool.clone()
    step.append()
    got = step.attend().clone()
    k_after, v_after = step.w.k_pool.clone(), step.w.v_pool.clone()
    step.w.k_pool.copy_(k_missing)
    step.w.v_pool.copy_(v_missing)
    fused = step.fused()
    assert torch.equal(step.w.k_pool.view(torch.int16), k_after.view(torch.int16))
    assert torch.equal(step.w.v_pool.view(torch.int16), v_after.view(torch.int16))
    want = oracle_outputs(step.w)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=0, atol=2e-3)
    np.testing.assert_allclose(fused.cpu().numpy(), want, rtol=0, atol=2e-3)


CONFIG5_CELLS = [
    (batch, ctx, block_size, dtype)
    for dtype in (torch.bfloat16, torch.float32)
    for batch in (1, 8)
    for ctx in (32768, 131072)
    for block_size in (16, 32)
]


@pytest.mark.parametrize(
    "batch,ctx,block_size,dtype", CONFIG5_CELLS,
    ids=[f"{'bf16' if d == torch.bfloat16 else 'f32'}-b{b}-c{c}-bs{bs}" for b, c, bs, d in CONFIG5_CELLS],
)
def test_config5_long_context_split(batch, ctx, block_size, dtype):
    """BASELINE config 5, every cell bench.py times (the same workload: seed 5,
    1 % of keys x20): split-context partitions merged by the reduce launch,
    every sequence against the float64 oracle, through the call bench.py
    makes (host lengths, output in the input dtype) and a float32-output
    launch sized from max_context_len."""
    print_case("config5", batch, ctx, block_size, dtype)
    w = make_workload([ctx] * batch, block_size=block_size, dtype=dtype, seed=5, heavy_fraction=0.01)
    part, ws = _native.decode_plan(batch, 12, 64, block_size, ctx, dtype, 0)
    assert ws > 0 and part < ctx, "long contexts must take the split path"
    atol = 1e-5 if dtype == torch.float32 else 2e-3
    check_workload(w, out_f32_atol=atol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_partition_sizes_agree(dtype):
    """Every partition size, from one tile to a single partition, gives the
    oracle's answer: the log-sum-exp merge is exact up to rounding."""
    lens = [1, 31, 32, 33, 1000, 4095, 4096]
    w = make_workload(lens, block_size=16, dtype=dtype, seed=7, heavy_fraction=0.01)
    tile, _ = _native.decode_plan(len(lens), 12, 64, 16, 1, dtype, 0)
    atol = 1e-5 if dtype == torch.float32 else 2e-3
    sizes = []
    p = tile
    while p <= 8192:
        sizes.append(p)
        p *= 4
    for part in sizes + [0, -1]:  # -1: one workgroup per (sequence, head)
        print_case("partition", dtype, part)
        check_workload(w, out_f32_atol=atol, partition_tokens=part)


def test_ragged_batch_with_empty_sequence_and_block_size_3():
    """A zero-length sequence yields zeros (as SDPA does with no keys); a
    block size that is not a power of two goes through the fast division."""
    lens = [0, 5, 48, 700]
    w = make_workload(lens, block_size=3, dtype=torch.float32, seed=9)
    got = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, w.max_len, partition_tokens=64
    )
    assert torch.equal(got[0], torch.zeros_like(got[0]))
    want = oracle_outputs(w, [1, 2, 3])
    np.testing.assert_allclose(got[1:].cpu().numpy(), want, rtol=0, atol=1e-5)


@pytest.mark.parametrize("block_size", [3, 16])
def test_workgroup_form_ragged_batch_with_empty_sequence(block_size):
    """The workgroup form (one workgroup of 16 waves per (sequence, head),
    merged in LDS): empty, single-token and ragged contexts, through the fast
    block-id path (block 16) and the per-row division (block 3)."""
    lens = [0, 1, 5, 17, 48, 700, 4096]
    w = make_workload(lens, block_size=block_size, dtype=torch.float32, seed=12, heavy_fraction=0.01)
    got = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, w.max_len, partition_tokens=-1
    )
    assert torch.equal(got[0], torch.zeros_like(got[0]))
    np.testing.assert_allclose(got[1:].cpu().numpy(), oracle_outputs(w, range(1, len(lens))), rtol=0, atol=1e-5)


def test_automatic_plan_chooses_the_form():
    """The automatic plan takes the workgroup form (one launch, no workspace)
    for few (sequence, head) rows with contexts up to 4096 tokens."""
    for batch, ctx in ((1, 96), (1, 1024), (21, 1000), (12, 4096), (64, 8192)):
        part, ws = _native.decode_plan(batch, 12, 64, 16, ctx, torch.bfloat16, 0)
        assert ws == 0 and part >= ctx, (batch, ctx)
    # Few rows of longer contexts split into partitions across many waves.
    for batch, ctx in ((1, 2048), (4, 4096), (64, 16384), (128, 8192)):
        part, ws = _native.decode_plan(batch, 12, 64, 16, ctx, torch.bfloat16, 0)
        assert ws > 0 and part < ctx, (batch, ctx)


def test_out_of_range_block_id_yields_nan_without_touching_memory():
    """The kernel bounds-checks table entries: an id past the pool is never
    dereferenced and the affected sequence reports NaN; the others are exact."""
    w = make_workload([40, 40], block_size=16, dtype=torch.float32, seed=4)
    w.block_tables[1, 1] = w.k_pool.shape[1] + 5
    for part in (0, -1, 16):  # automatic (the workgroup form here), forced, and split partitions
        got = paged_attention.decode_batched(
            w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, 40, partition_tokens=part
        )
        assert torch.isnan(got[1]).all(), part
        np.testing.assert_allclose(got[0].cpu().numpy(), oracle_outputs(w, [0])[0], rtol=0, atol=1e-5)


def test_decode_is_deterministic_and_leaves_pools_untouched():
    w = make_workload([3000, 17], block_size=16, dtype=torch.bfloat16, seed=12)
    k_before, v_before = w.k_pool.clone(), w.v_pool.clone()
    runs = [
        paged_attention.decode_batched(w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, 3000)
        for _ in range(3)
    ]
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    assert torch.equal(w.k_pool, k_before) and torch.equal(w.v_pool, v_before)


def test_explicit_scale():
    w = make_workload([300], block_size=16, dtype=torch.float32, seed=13)
    got = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, 300, scale=0.05
    )
    k, v = sequence_kv(w, 0)
    want = ref.attention_fp64(ref.to_f64(w.q[0]), ref.to_f64(k), ref.to_f64(v), scale=0.05)
    np.testing.assert_allclose(got[0].cpu().numpy(), want, rtol=0, atol=1e-5)
    assert math.isfinite(float(got.abs().max()))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("partition", [0, -1, 64])
@pytest.mark.parametrize("host_lens", [False, True])
def test_fused_append_decode_matches_append_then_decode(dtype, partition, host_lens):
    """mie_paged_decode_append: the pools end bit-identical to appending the
    new tokens (mie_kv_append's closed form), and the output is the oracle's
    attention over the full contexts - in the workgroup form (one launch) and
    in the partition form (append launch, then decode)."""
    print_case("fused append", dtype, partition, host_lens)
    lens = [0, 1, 2, 17, 300, 1000, 3000]
    w = make_workload(lens, block_size=16, dtype=dtype, seed=21, heavy_fraction=0.01)
    want = oracle_outputs(w)
    k_before, v_before = w.k_pool.clone(), w.v_pool.clone()
    k_new, v_new = take_last_tokens(w)
    got = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, w.max_len, out_dtype=torch.float32,
        partition_tokens=partition, context_lens_host=w.lens if host_lens else None, k_new=k_new, v_new=v_new,
    )
    assert np.array_equal(ref.raw_bits(w.k_pool.cpu()), ref.raw_bits(k_before.cpu()))
    assert np.array_equal(ref.raw_bits(w.v_pool.cpu()), ref.raw_bits(v_before.cpu()))
    assert torch.equal(got[0], torch.zeros_like(got[0]))
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=0, atol=1e-5 if dtype == torch.float32 else 2e-3)


def test_fused_append_to_an_unmapped_block_is_skipped_and_reported():
    """A new token whose block id lies outside the pool is not stored and its
    (sequence, head) outputs are NaN; the other sequences are exact."""
    w = make_workload([33, 40], block_size=16, dtype=torch.float32, seed=22)
    want = oracle_outputs(w, [0])
    k_new, v_new = take_last_tokens(w)
    w.block_tables[1, (40 - 1) // 16] = w.k_pool.shape[1] + 3
    k_before = w.k_pool.clone()
    got = paged_attention.decode_batched(
        w.q, w.k_pool, w.v_pool, 0, w.block_tables, w.context_lens, w.max_len, partition_tokens=-1,
        k_new=k_new[:, :, :].contiguous(), v_new=v_new,
    )
    assert torch.isnan(got[1]).all()
    np.testing.assert_allclose(got[0].cpu().numpy(), want[0], rtol=0, atol=1e-5)
    # Only sequence 0's new token was stored.
    diff = (w.k_pool != k_before).nonzero()
    assert diff.numel() > 0 and all(int(i) == w.tables[0][(33 - 1) // 16] for i in diff[:, 1])
