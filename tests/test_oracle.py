"""Pins for the CPU oracle (oracle/paged_ref.py).

The reference commits no golden vectors for this path, so each oracle function
is pinned by checks that do not restate its own formula: the reference Triton
kernel's flat-offset addressing (a second statement of the pool layout, in a
different file from the one the oracle restates), round trips against
contiguous storage, closed-form attention answers, torch's SDPA in float64,
and the log-sum-exp identity.  Every pin is also run against deliberately
broken oracle variants (planted on the CPU) to show it would catch that
mistake.
"""

import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_ref as ref


def lifo_table(num_blocks, needed, seed):
    """A block table the reference allocator hands out after shuffling its
    free list (tests/test_paged_attention.py:46-48 does the same shuffle)."""
    alloc = ref.LifoAllocator(num_blocks)
    random.Random(seed).shuffle(alloc.free_blocks)
    table = []
    ref.reserve(table, alloc, needed, 1)
    return table


def flat_offsets(pool, layer, table, length):
    """Element offsets of logical tokens [0, length) for every (h, t, d), from
    the reference Triton kernel's addressing (paged_attention.py:86-94):
    phys * stride_kb + head * stride_kh + slot * stride_ks + d inside k_pool[layer]."""
    L, NB, H, BS, D = pool.shape
    layer_base = layer * NB * H * BS * D
    stride_kb, stride_kh, stride_ks = H * BS * D, BS * D, D
    t = np.arange(length)
    phys = np.asarray(table, dtype=np.int64)[t // BS]
    slot = t % BS
    h = np.arange(H)[:, None, None]
    d = np.arange(D)[None, None, :]
    return layer_base + phys[None, :, None] * stride_kb + h * stride_kh + slot[None, :, None] * stride_ks + d


def check_gather_layout(gather_fn, seed):
    """True iff gather_fn reproduces the flat-offset addressing on a pool whose
    every element holds its own flat index."""
    rng = np.random.default_rng(seed)
    L, NB, H, BS, D = 3, 11, 3, 4, 5
    pool = np.arange(L * NB * H * BS * D, dtype=np.int64).reshape(L, NB, H, BS, D)
    layer = int(rng.integers(L))
    length = 4 * BS + 3
    table = lifo_table(NB, 5, seed)
    got = gather_fn(pool, layer, table, length)
    return got.shape == (H, length, D) and np.array_equal(got, flat_offsets(pool, layer, table, length))


# ---- append / gather ----------------------------------------------------------


@pytest.mark.parametrize("seed", range(4))
def test_gather_matches_reference_kernel_addressing(seed):
    assert check_gather_layout(ref.gather_rows, seed)


def _gather_slot_block_swapped(pool, layer, table, length):
    L, NB, H, BS, D = pool.shape
    out = np.empty((H, length, D), dtype=pool.dtype)
    for t in range(length):
        out[:, t] = pool[layer, table[t % BS], :, (t // BS) % BS]
    return out


def _gather_ignores_table(pool, layer, table, length):
    return ref.gather_rows(pool, layer, list(range(len(table))), length)


def _gather_reshape_without_transpose(pool, layer, table, length):
    L, NB, H, BS, D = pool.shape
    nb = -(-length // BS)
    tiles = pool[layer, np.asarray(table[:nb])]  # [nb, H, BS, D], heads not moved first
    return tiles.reshape(H, nb * BS, D)[:, :length]


@pytest.mark.parametrize(
    "broken", [_gather_slot_block_swapped, _gather_ignores_table, _gather_reshape_without_transpose]
)
def test_layout_pin_rejects_planted_mistakes(broken):
    assert not check_gather_layout(broken, seed=0)


@pytest.mark.parametrize("block_size", [1, 3, 4, 16, 32])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_append_then_gather_round_trips(block_size, dtype):
    """Prefill + decode appends through a shuffled table read back as the
    contiguous sequence, bit for bit, and touch nothing else."""
    g = torch.Generator().manual_seed(block_size)
    L, H, D, ctx = 2, 3, 8, 3 * block_size + 2
    NB = -(-ctx // block_size) + 4
    pools = [ref.raw_bits(torch.randn(L, NB, H, block_size, D, generator=g).to(dtype)) for _ in range(2)]
    before = [p.copy() for p in pools]
    k = ref.raw_bits(torch.randn(H, ctx, D, generator=g).to(dtype))
    v = ref.raw_bits(torch.randn(H, ctx, D, generator=g).to(dtype))
    table = lifo_table(NB, -(-ctx // block_size), seed=block_size)
    layer = 1
    prefill = ctx - 3
    ref.append_rows(pools[0], pools[1], layer, table, 0, k[:, :prefill], v[:, :prefill])
    for p in range(prefill, ctx):
        ref.append_rows(pools[0], pools[1], layer, table, p, k[:, p : p + 1], v[:, p : p + 1])
    assert np.array_equal(ref.gather_rows(pools[0], layer, table, ctx), k)
    assert np.array_equal(ref.gather_rows(pools[1], layer, table, ctx), v)
    # Elements outside the addressed rows are unchanged.
    touched = np.zeros(pools[0].size, dtype=bool)
    touched[flat_offsets(pools[0], layer, table, ctx).ravel()] = True
    for p, b in zip(pools, before):
        assert np.array_equal(p.ravel()[~touched], b.ravel()[~touched])


def test_append_brute_force_tiny():
    """Every element of a 1-layer, 2-block pool after appending 3 tokens at
    block size 2 with table [1, 0], written out by hand."""
    pool_k = np.zeros((1, 2, 1, 2, 1), dtype=np.int64)
    pool_v = np.zeros_like(pool_k)
    k = np.array([[[10], [11], [12]]])  # [H=1, S=3, D=1]
    ref.append_rows(pool_k, pool_v, 0, [1, 0], 0, k, -k)
    # token 0 -> block 1 slot 0, token 1 -> block 1 slot 1, token 2 -> block 0 slot 0
    assert pool_k[0, :, 0, :, 0].tolist() == [[12, 0], [10, 11]]
    assert pool_v[0, :, 0, :, 0].tolist() == [[-12, 0], [-10, -11]]


# ---- attention ----------------------------------------------------------------


def rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def test_attention_single_key_returns_its_value():
    q, k, v = rand((3, 8), 0), rand((3, 1, 8), 1), rand((3, 1, 8), 2)
    assert np.array_equal(ref.attention_fp64(q, k, v), v[:, 0])


def test_attention_equal_keys_and_zero_query_average_values():
    k = np.repeat(rand((2, 1, 4), 3), 7, axis=1)
    v = rand((2, 7, 4), 4)
    np.testing.assert_allclose(ref.attention_fp64(rand((2, 4), 5), k, v), v.mean(axis=1), rtol=0, atol=1e-14)
    np.testing.assert_allclose(
        ref.attention_fp64(np.zeros((2, 4)), rand((2, 7, 4), 6), v), v.mean(axis=1), rtol=0, atol=1e-14
    )


def test_attention_two_keys_by_hand():
    q, k1, k2, v1, v2, scale = 0.7, -1.3, 2.1, 5.0, -3.0, 0.37
    s1, s2 = q * k1 * scale, q * k2 * scale
    want = (math.exp(s1) * v1 + math.exp(s2) * v2) / (math.exp(s1) + math.exp(s2))
    got = ref.attention_fp64(np.array([[q]]), np.array([[[k1], [k2]]]), np.array([[[v1], [v2]]]), scale)
    assert abs(got[0, 0] - want) < 1e-15


def test_attention_empty_context_is_zero_like_sdpa():
    q = torch.randn(1, 2, 1, 4, dtype=torch.float64)
    empty = torch.zeros(1, 2, 0, 4, dtype=torch.float64)
    sdpa = F.scaled_dot_product_attention(q, empty, empty)[0, :, 0].numpy()
    assert np.array_equal(ref.attention_fp64(q[0, :, 0], empty[0], empty[0]), sdpa)


def sdpa64(q, k, v, scale=None):
    t = [torch.from_numpy(np.ascontiguousarray(x)) for x in (q[:, None], k, v)]
    return F.scaled_dot_product_attention(t[0][None], t[1][None], t[2][None], scale=scale)[0, :, 0].numpy()


@pytest.mark.parametrize("ctx,dim", [(1, 4), (17, 64), (190, 96), (1024, 64)])
def test_attention_matches_torch_sdpa_float64(ctx, dim):
    q, k, v = rand((5, dim), ctx), rand((5, ctx, dim), ctx + 1), rand((5, ctx, dim), ctx + 2)
    np.testing.assert_allclose(ref.attention_fp64(q, k, v), sdpa64(q, k, v), rtol=0, atol=1e-12)
    np.testing.assert_allclose(ref.attention_fp64(q, k, v, 0.3), sdpa64(q, k, v, 0.3), rtol=0, atol=1e-12)


def _attention_no_scale(q, k, v, scale=None):
    return ref.attention_fp64(q, k, v, scale=1.0)


def _attention_softmax_over_heads(q, k, v, scale=None):
    s = np.einsum("hd,hcd->hc", q, k) / math.sqrt(q.shape[1])
    w = np.exp(s - s.max(axis=0, keepdims=True))
    return np.einsum("hc,hcd->hd", w / w.sum(axis=0, keepdims=True), v)


def _attention_values_transposed(q, k, v, scale=None):
    return ref.attention_fp64(q, k, v[:, ::-1])


@pytest.mark.parametrize("broken", [_attention_no_scale, _attention_softmax_over_heads, _attention_values_transposed])
def test_sdpa_pin_rejects_planted_mistakes(broken):
    q, k, v = rand((5, 16), 10), rand((5, 33, 16), 11), rand((5, 33, 16), 12)
    assert not np.allclose(broken(q, k, v), sdpa64(q, k, v), rtol=0, atol=1e-6)


@pytest.mark.parametrize("partition", [1, 2, 3, 7, 16, 99, 100, 256])
def test_split_attention_equals_unsplit(partition):
    """Log-sum-exp merging of partitions is exact; 1 % of keys x20 stresses the max."""
    ctx = 100
    k = rand((4, ctx, 16), 20)
    k[:, ::100] *= 20.0
    q, v = rand((4, 16), 21), rand((4, ctx, 16), 22)
    np.testing.assert_allclose(
        ref.split_attention_fp64(q, k, v, partition), ref.attention_fp64(q, k, v), rtol=0, atol=1e-12
    )


def test_split_pin_rejects_merge_without_rescale():
    q, k, v = rand((2, 8), 30), rand((2, 40, 8), 31, 3.0), rand((2, 40, 8), 32)

    def merged_without_rescale(partition):
        outs = [ref.attention_fp64(q, k[:, s : s + partition], v[:, s : s + partition]) for s in range(0, 40, partition)]
        return np.mean(outs, axis=0)

    assert not np.allclose(merged_without_rescale(8), ref.attention_fp64(q, k, v), atol=1e-6)


@pytest.mark.parametrize("ctx,block_size", [(1, 16), (17, 16), (64, 4), (190, 32)])
def test_gather_sdpa_matches_float64_attention(ctx, block_size):
    g = torch.Generator().manual_seed(ctx)
    L, H, D = 2, 4, 32
    NB = -(-ctx // block_size) + 3
    k_pool, v_pool = torch.randn(L, NB, H, block_size, D, generator=g), torch.randn(L, NB, H, block_size, D, generator=g)
    table = lifo_table(NB, -(-ctx // block_size), seed=ctx)
    q = torch.randn(1, H, 1, D, generator=g)
    got = ref.gather_sdpa(q, k_pool, v_pool, 1, table, ctx)[0, :, 0].numpy()
    k = ref.gather_rows(k_pool.numpy(), 1, table, ctx)
    v = ref.gather_rows(v_pool.numpy(), 1, table, ctx)
    np.testing.assert_allclose(got, ref.attention_fp64(q[0, :, 0], k, v), rtol=0, atol=1e-5)
    batched = ref.batched_gather_sdpa(q[:, :, 0].repeat(2, 1, 1), k_pool, v_pool, 1, [table, table], [ctx, ctx])
    assert torch.equal(batched[0], batched[1]) and torch.allclose(batched[0], torch.from_numpy(got).float())


# ---- allocator ------------------------------------------------------------------


def test_lifo_allocation_order_and_exhaustion():
    alloc = ref.LifoAllocator(3)
    assert [alloc.allocate() for _ in range(3)] == [2, 1, 0]
    with pytest.raises(RuntimeError, match="no free KV cache blocks left"):
        alloc.allocate()
    alloc.free([1])
    assert alloc.allocate() == 1


def test_reserve_rolls_back_on_exhaustion():
    """tests/test_parity.py:100-115: a prefill needing two blocks from a
    one-block pool leaves the pool and the table as they were."""
    alloc = ref.LifoAllocator(1)
    table = []
    with pytest.raises(RuntimeError, match="no free KV cache blocks left"):
        ref.reserve(table, alloc, 8, 4)
    assert table == [] and alloc.free_blocks == [0]
    assert ref.reserve(table, alloc, 4, 4) == [0]


# ---- qkv_project_fp64 (model.py:228-234, the block's attn_norm) -------------


def torch_qkv64(x, w, b, heads, nw, nb, eps=1e-5):
    """torch's own LayerNorm and linear in float64, split as CachedAttention does."""
    x = torch.from_numpy(np.asarray(x, dtype=np.float64))
    dim = x.numel()
    y = F.layer_norm(x, (dim,), torch.from_numpy(nw), torch.from_numpy(nb), eps) if nw is not None else x
    qkv = F.linear(y, torch.from_numpy(w), torch.from_numpy(b) if b is not None else None)
    return tuple(t.view(heads, dim // heads).numpy() for t in qkv.chunk(3))


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("heads,head_dim", [(2, 8), (12, 64), (3, 5)])
def test_qkv_projection_matches_torch_float64(norm, heads, head_dim):
    dim = heads * head_dim
    x, w, b = rand((dim,), 30) * 3 + 0.5, rand((3 * dim, dim), 31), rand((3 * dim,), 32)
    nw, nb = (rand((dim,), 33) + 1.0, rand((dim,), 34)) if norm else (None, None)
    got = ref.qkv_project_fp64(x, w, b, heads, nw, nb)
    for g, want in zip(got, torch_qkv64(x, w, b, heads, nw, nb)):
        np.testing.assert_allclose(g, want, rtol=0, atol=1e-12)


def test_qkv_projection_known_answers():
    heads, head_dim = 3, 4
    dim = heads * head_dim
    x = np.arange(dim, dtype=np.float64) - 2.5
    eye = np.eye(dim)
    # Stacked [I; 2I; 3I] and no bias: q = x, k = 2x, v = 3x, head h = x[h*D:(h+1)*D].
    q, k, v = ref.qkv_project_fp64(x, np.concatenate([eye, 2 * eye, 3 * eye]), None, heads)
    np.testing.assert_array_equal(q, x.reshape(heads, head_dim))
    np.testing.assert_array_equal(k, 2 * x.reshape(heads, head_dim))
    np.testing.assert_array_equal(v, 3 * x.reshape(heads, head_dim))
    # A constant x normalises to the norm bias alone.
    nb = np.linspace(-1, 1, dim)
    q, _, _ = ref.qkv_project_fp64(np.full(dim, 7.0), np.concatenate([eye] * 3), None, heads, np.full(dim, 5.0), nb)
    np.testing.assert_allclose(q.reshape(-1), nb, rtol=0, atol=1e-12)


def _qkv_unbiased_variance(x, w, b, heads, nw, nb):
    y = (x - x.mean()) / math.sqrt(x.var(ddof=1) + 1e-5) * nw + nb
    return ref.qkv_project_fp64(y, w, b, heads)


def _qkv_k_v_swapped(x, w, b, heads, nw, nb):
    q, k, v = ref.qkv_project_fp64(x, w, b, heads, nw, nb)
    return q, v, k


def _qkv_heads_transposed(x, w, b, heads, nw, nb):
    q, k, v = ref.qkv_project_fp64(x, w, b, heads, nw, nb)
    d = q.shape[1]
    return tuple(t.reshape(-1).reshape(d, heads).T for t in (q, k, v))


@pytest.mark.parametrize("broken", [_qkv_unbiased_variance, _qkv_k_v_swapped, _qkv_heads_transposed])
def test_qkv_pin_rejects_planted_mistakes(broken):
    heads, dim = 4, 32
    x, w, b = rand((dim,), 40), rand((3 * dim, dim), 41), rand((3 * dim,), 42)
    nw, nb = rand((dim,), 43) + 1.0, rand((dim,), 44)
    want = torch_qkv64(x, w, b, heads, nw, nb)
    got = broken(x, w, b, heads, nw, nb)
    assert not all(np.allclose(g, t, rtol=0, atol=1e-6) for g, t in zip(got, want))


# ---- attention half: attention, head concatenation, out_proj, residual -------


def test_attention_half_matches_torch_multihead_layout():
    """attention_half_fp64 against torch in float64: SDPA over [1, H, C, D],
    the [1, H, 1, D] -> [1, 1, dim] transpose/reshape CachedAttention.forward
    does (model.py:267), F.linear with out_proj, plus x."""
    g = torch.Generator().manual_seed(11)
    H, C, D = 3, 9, 8
    q, k, v = torch.randn(H, D, generator=g), torch.randn(H, C, D, generator=g), torch.randn(H, C, D, generator=g)
    w, b, x = torch.randn(H * D, H * D, generator=g), torch.randn(H * D, generator=g), torch.randn(H * D, generator=g)
    a = F.scaled_dot_product_attention(q.double()[None, :, None], k.double()[None], v.double()[None])
    o = F.linear(a.transpose(1, 2).reshape(1, 1, H * D), w.double(), b.double())[0, 0]
    got_o, got_h = ref.attention_half_fp64(q, k, v, w, b, x)
    np.testing.assert_allclose(got_o, o.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got_h, (x.double() + o).numpy(), rtol=1e-12, atol=1e-12)


def test_attention_half_known_answer():
    """One key per head: the attention is each head's value row, so with
    W = I the output is the concatenated values, head 0 first."""
    H, D = 2, 3
    q = torch.ones(H, D)
    k = torch.ones(H, 1, D)
    v = torch.arange(H * D, dtype=torch.float64).reshape(H, 1, D)
    o, h = ref.attention_half_fp64(q, k, v, torch.eye(H * D), None, torch.full((H * D,), 10.0))
    np.testing.assert_array_equal(o, np.arange(H * D))
    np.testing.assert_array_equal(h, 10 + np.arange(H * D))


def test_attention_half_pin_rejects_a_transposed_projection():
    g = torch.Generator().manual_seed(12)
    H, C, D = 2, 5, 4
    q, k, v = torch.randn(H, D, generator=g), torch.randn(H, C, D, generator=g), torch.randn(H, C, D, generator=g)
    w, x = torch.randn(H * D, H * D, generator=g), torch.zeros(H * D)
    a = torch.from_numpy(ref.attention_fp64(q, k, v).reshape(-1))
    o, _ = ref.attention_half_fp64(q, k, v, w, None, x)
    assert not np.allclose(o, (w.double().T @ a).numpy())  # a transposed operand would fail the pin
    np.testing.assert_allclose(o, (w.double() @ a).numpy(), rtol=1e-12)
