"""Randomized bit-exact sweep of the HIP KV append and gather.

Each seeded case (32 by default; MIE_RANDOM_KV_CASES=N for more) draws the
element type (float32, bfloat16, float16, float64), head count, head_dim
(odd sizes included, so rows of 2, 4, 8 and 16-byte vectors are all taken),
block size (powers of two and not), layer count and layer, batch, one shuffled
block table per sequence over a shared pool with non-zero contents, each
sequence's start position and the number of rows appended (prefill or one
token), and whether positions come from the host or the device.  The append
must leave the WHOLE pool equal, bit for bit, to oracle.paged_ref.append_rows
applied to a CPU copy; the gather of every sequence's first `length` tokens
must equal oracle.paged_ref.gather_rows bit for bit.
"""

import os
import random

import numpy as np
import pytest
import torch

from conftest import print_case
from moe_engine import kv_ops
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float64)
CASES = int(os.environ.get("MIE_RANDOM_KV_CASES", "32"))


def draw(seed):
    rng = random.Random(seed)
    c = dict(
        dtype=rng.choice(DTYPES),
        heads=rng.choice((1, 2, 3, 12)),
        head_dim=rng.choice((1, 3, 4, 8, 13, 32, 64, 96, 128)),
        block_size=rng.choice((1, 2, 3, 5, 16, 32)),
        layers=rng.choice((1, 3)),
        batch=rng.randint(1, 6),
        rows=rng.choice((1, 1, 7, 40)),
        device_positions=rng.random() < 0.5,
    )
    c["layer"] = rng.randrange(c["layers"])
    c["starts"] = [rng.randint(0, 60) for _ in range(c["batch"])]
    return c


@pytest.mark.parametrize("seed", range(CASES))
def test_random_append_and_gather_bit_exact(seed):
    c = draw(seed)
    print_case("random kv", seed, c)
    rng = random.Random(seed + 1000)
    gen = torch.Generator().manual_seed(seed)
    dt, H, D, BS, B, S = c["dtype"], c["heads"], c["head_dim"], c["block_size"], c["batch"], c["rows"]
    ends = [p + S for p in c["starts"]]
    need = [-(-e // BS) for e in ends]
    max_blocks = max(need)
    num_blocks = sum(need) + 3
    ids = list(range(num_blocks))
    rng.shuffle(ids)
    tables, at = [], 0
    for n in need:
        tables.append(ids[at : at + n] + [0] * (max_blocks - n))
        at += n
    shape = (c["layers"], num_blocks, H, BS, D)
    k_pool = torch.randn(shape, generator=gen).to(dt)
    v_pool = torch.randn(shape, generator=gen).to(dt)
    want_k, want_v = ref.raw_bits(k_pool).copy(), ref.raw_bits(v_pool).copy()
    k_new = torch.randn((B, H, S, D), generator=gen).to(dt)
    v_new = torch.randn((B, H, S, D), generator=gen).to(dt)
    kp, vp = k_pool.cuda(), v_pool.cuda()
    table_dev = torch.tensor(tables, dtype=torch.int32, device="cuda")
    if c["device_positions"]:
        pos = torch.tensor(c["starts"], dtype=torch.int32, device="cuda")
        kv_ops.append(kp, vp, c["layer"], k_new.cuda(), v_new.cuda(), table_dev, positions=pos)
    else:
        # Host positions: one launch per sequence.
        for b in range(B):
            kv_ops.append(kp, vp, c["layer"], k_new[b : b + 1].cuda(), v_new[b : b + 1].cuda(),
                          table_dev[b : b + 1], position=c["starts"][b])
    for b in range(B):
        ref.append_rows(want_k, want_v, c["layer"], tables[b], c["starts"][b], ref.raw_bits(k_new[b]),
                        ref.raw_bits(v_new[b]))
    assert np.array_equal(ref.raw_bits(kp.cpu()), want_k)
    assert np.array_equal(ref.raw_bits(vp.cpu()), want_v)
    for b in range(B):
        length = rng.randint(0, ends[b])
        got_k, got_v = kv_ops.gather(kp, vp, c["layer"], table_dev[b].contiguous(), length)
        assert np.array_equal(ref.raw_bits(got_k[0].cpu()), ref.gather_rows(want_k, c["layer"], tables[b], length))
        assert np.array_equal(ref.raw_bits(got_v[0].cpu()), ref.gather_rows(want_v, c["layer"], tables[b], length))
