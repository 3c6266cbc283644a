"""The four-launch decoder block's two new entry points, through the C ABI.

mie_attn_out_acc: the attention of one decode token fused with out_proj,
every head's share of every output row added into an int64 accumulator as
round(y * 2^32).  Checked against the float64 oracle
(paged_ref.attention_half_fp64: attention per head, the heads concatenated in
order, W_out, + b_out), per output row i within

    |got_i - want_i| <= 2e-5 * scale_i + 1e-6,   scale_i = sum_j |W_ij a_j| + |b_i|

(float32 softmax and float32 dot products of D terms per head; the fixed-point
sum adds at most 2^-33 per head).  The accumulator must be bit-identical
between runs, whatever order the workgroups finished in.

mie_moe_decode_block_acc: h_out = x + (acc * 2^-32 + b_out) in float32, then
the MoE half exactly as mie_moe_decode_block computes it on h_out - both
compared bit for bit - and the accumulator cleared for the next token.
"""

import math

import numpy as np
import pytest
import torch

from conftest import print_case
from moe_engine import _native
from moe_engine.workloads import make_workload, sequence_kv
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

FIX = 2.0 ** -32


def stream():
    return torch.cuda.current_stream().cuda_stream


def attn_out(w, b, w_out, acc, ctx=None, ctx_dev=None, max_ctx=None, dtype=0):
    kp, vp = w.k_pool[w.layer], w.v_pool[w.layer]
    heads, bs, head_dim = kp.shape[1], kp.shape[2], kp.shape[3]
    table = w.block_tables[b]
    ctx = w.lens[b] if ctx is None else ctx
    max_ctx = ctx if max_ctx is None else max_ctx
    rc = _native.lib().mie_attn_out_acc(
        w.q[b].data_ptr(), kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.shape[0],
        table.data_ptr(), table.numel(), None if ctx_dev is None else ctx_dev.data_ptr(), ctx, max_ctx,
        heads, head_dim, bs, 1.0 / math.sqrt(head_dim), w_out.data_ptr(), acc.data_ptr(), dtype, stream())
    _native.check(rc, "mie_attn_out_acc")


def oracle_rows(w, b, w_out, ctx=None):
    """Expected out_proj output (no bias) and the per-row error scale."""
    k, v = sequence_kv(w, b)
    ctx = w.lens[b] if ctx is None else ctx
    k, v = k[:, :ctx], v[:, :ctx]
    a = ref.attention_fp64(ref.to_f64(w.q[b]), ref.to_f64(k), ref.to_f64(v)).reshape(-1)
    o, _ = ref.attention_half_fp64(w.q[b], k, v, w_out, None, torch.zeros(w_out.shape[0]))
    scale = np.abs(ref.to_f64(w_out)) @ np.abs(a)
    return o, scale


def check_rows(acc, want, scale):
    dim = want.shape[0]
    got = acc[:dim].cpu().numpy().astype(np.float64) * FIX
    assert int(acc[dim]) == 0, "the overflow / NaN flag is set"
    err = np.abs(got - want)
    bound = 2e-5 * scale + 1e-6
    assert (err <= bound).all(), f"max error {err.max():.3e} at row {err.argmax()} (bound {bound[err.argmax()]:.3e})"


CASES = [
    # (heads, head_dim, block_size, context lengths)
    (12, 64, 16, [1, 2, 33, 96, 97]),  # config 1's shape and contexts
    (12, 64, 16, [1024, 2048]),
    (12, 64, 16, [128, 129]),  # either side of the switch from 4 to 8 waves per workgroup
    (12, 64, 1, [1, 40]),
    (12, 64, 5, [7, 130]),  # a block size that is not a power of two
    (12, 64, 64, [63, 64, 65, 700]),
    (4, 32, 16, [1, 17, 300]),
    (24, 32, 8, [55]),
    (6, 128, 16, [1, 90, 513]),
    (1, 64, 16, [3, 1500]),
    (20, 64, 32, [250]),  # 20 heads: a second group of 8 heads runs partly idle
]


@pytest.mark.parametrize("heads,head_dim,block_size,lens", CASES)
def test_attn_out_matches_float64_attention_half(heads, head_dim, block_size, lens):
    print_case("attn_out", heads, head_dim, block_size, lens)
    w = make_workload(lens, num_heads=heads, head_dim=head_dim, block_size=block_size, dtype=torch.float32,
                      seed=heads + head_dim + block_size, heavy_fraction=0.02)
    dim = heads * head_dim
    g = torch.Generator(device="cuda").manual_seed(7)
    w_out = torch.randn(dim, dim, generator=g, device="cuda") / math.sqrt(dim)
    for b in range(len(lens)):
        acc = torch.zeros(dim + 1, dtype=torch.int64, device="cuda")
        attn_out(w, b, w_out, acc)
        want, scale = oracle_rows(w, b, w_out)
        check_rows(acc, want, scale)
        again = torch.zeros_like(acc)
        attn_out(w, b, w_out, again)
        assert torch.equal(acc, again), "the fixed-point sums differ between runs"


def test_attn_out_reads_the_context_length_on_the_device_and_clamps_it():
    print_case("attn_out device ctx")
    w = make_workload([300], num_heads=12, head_dim=64, block_size=16, dtype=torch.float32, seed=3)
    w_out = torch.randn(768, 768, device="cuda") / math.sqrt(768)
    for live, bound in ((200, 256), (300, 300), (299, 120)):
        ctx_dev = torch.tensor([live], dtype=torch.int32, device="cuda")
        acc = torch.zeros(769, dtype=torch.int64, device="cuda")
        attn_out(w, 0, w_out, acc, ctx=0, ctx_dev=ctx_dev, max_ctx=bound)
        want, scale = oracle_rows(w, 0, w_out, ctx=min(live, bound))
        check_rows(acc, want, scale)


def test_attn_out_adds_into_the_accumulator_and_flags_blocks_outside_the_pool():
    """Two calls add (integer sums); a context block id outside the pool is
    never read and sets the flag entry acc[dim]; an empty context adds zeros."""
    print_case("attn_out accumulate / flag")
    w = make_workload([50], num_heads=12, head_dim=64, block_size=16, dtype=torch.float32, seed=4)
    w_out = torch.randn(768, 768, device="cuda") / math.sqrt(768)
    once = torch.zeros(769, dtype=torch.int64, device="cuda")
    attn_out(w, 0, w_out, once)
    twice = torch.zeros_like(once)
    attn_out(w, 0, w_out, twice)
    attn_out(w, 0, w_out, twice)
    assert torch.equal(twice, 2 * once)
    empty = torch.zeros_like(once)
    attn_out(w, 0, w_out, empty, ctx=0, max_ctx=0)
    assert not empty.any()
    w.block_tables[0, 2] = w.k_pool.shape[1]  # one past the pool
    flagged = torch.zeros_like(once)
    attn_out(w, 0, w_out, flagged)
    assert int(flagged[768]) != 0


def test_attn_out_flags_partials_whose_head_sum_could_leave_int64():
    """Each of the H heads adds one partial per row, so a partial is added
    only below 2^31 / H in magnitude (the sum of H of them, times 2^32, stays
    inside int64).  With V all ones every head's attention output is 1, so
    y = W_out[i, h*D : (h+1)*D] . 1 = 64 w for a constant W_out = w: at
    w = 5e6 (y = 3.2e8, above 2^31 / 12 = 1.8e8, below 2^31) the flag is set
    - twelve such partials would wrap the sum - and at w = 5e5 the rows hold
    12 * round(y * 2^32) exactly."""
    print_case("attn_out int64 bound")
    w = make_workload([40], num_heads=12, head_dim=64, block_size=16, dtype=torch.float32, seed=5)
    w.v_pool.fill_(1.0)
    for value, flagged in ((5e6, True), (5e5, False)):
        w_out = torch.full((768, 768), value, device="cuda")
        acc = torch.zeros(769, dtype=torch.int64, device="cuda")
        attn_out(w, 0, w_out, acc)
        torch.cuda.synchronize()
        assert (int(acc[768]) != 0) == flagged
        if not flagged:
            got = acc[:768].double() * FIX
            assert torch.allclose(got, torch.full_like(got, 12 * 64 * value), rtol=1e-6)


def moe_inputs(dim, hidden, experts, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *shape, s=1.0: torch.randn(*shape, generator=g, device="cuda") * s  # noqa: E731
    return dict(
        x=r(dim), o=r(dim, s=0.5), b_out=r(dim, s=0.1), ln_w=1 + r(dim, s=0.1), ln_b=r(dim, s=0.1),
        router=r(experts, dim, s=dim ** -0.5), w1=r(experts, hidden, dim, s=dim ** -0.5), b1=r(experts, hidden, s=0.1),
        w2=r(experts, dim, hidden, s=hidden ** -0.5), b2=r(experts, dim, s=0.1),
    )


def moe_scratch(dim, hidden, experts, top_k):
    z = lambda *shape, dtype=torch.float32: torch.zeros(*shape, dtype=dtype, device="cuda")  # noqa: E731
    return z(experts), z(top_k, dtype=torch.int32), z(top_k), z(top_k, hidden), z(dim)


@pytest.mark.parametrize("dim,hidden,experts,top_k", [(768, 2048, 8, 2), (256, 512, 4, 1), (512, 1024, 16, 4)])
def test_moe_block_acc_forms_the_residual_and_clears_the_accumulator(dim, hidden, experts, top_k):
    print_case("moe_decode_block_acc", dim, hidden, experts, top_k)
    lib = _native.lib()
    t = moe_inputs(dim, hidden, experts, seed=dim + experts)
    acc = torch.zeros(dim + 1, dtype=torch.int64, device="cuda")
    acc[:dim] = torch.round(t["o"].double() / FIX).long()
    # h as the kernel forms it: int64 -> float32 (one rounding), the exact 2^-32
    # scale, + b_out, then + x, each in float32.
    h_want = t["x"] + ((acc[:dim].float() * FIX) + t["b_out"])
    h_out = torch.empty(dim, device="cuda")
    logits, ids, weights, hid, out = moe_scratch(dim, hidden, experts, top_k)
    rc = lib.mie_moe_decode_block_acc(
        t["x"].data_ptr(), acc.data_ptr(), t["b_out"].data_ptr(), h_out.data_ptr(), t["ln_w"].data_ptr(),
        t["ln_b"].data_ptr(), 1e-5, t["router"].data_ptr(), t["w1"].data_ptr(), t["b1"].data_ptr(),
        t["w2"].data_ptr(), t["b2"].data_ptr(), experts, top_k, dim, hidden, logits.data_ptr(), ids.data_ptr(),
        weights.data_ptr(), hid.data_ptr(), out.data_ptr(), 0, stream())
    _native.check(rc, "mie_moe_decode_block_acc")
    torch.cuda.synchronize()
    assert torch.equal(h_out, h_want)
    assert not acc.any(), "the accumulator is not cleared"
    logits2, ids2, weights2, hid2, out2 = moe_scratch(dim, hidden, experts, top_k)
    rc = lib.mie_moe_decode_block(
        h_want.data_ptr(), t["ln_w"].data_ptr(), t["ln_b"].data_ptr(), 1e-5, t["router"].data_ptr(),
        t["w1"].data_ptr(), t["b1"].data_ptr(), t["w2"].data_ptr(), t["b2"].data_ptr(), experts, top_k, dim, hidden,
        logits2.data_ptr(), ids2.data_ptr(), weights2.data_ptr(), hid2.data_ptr(), out2.data_ptr(), 0, stream())
    _native.check(rc, "mie_moe_decode_block")
    assert torch.equal(ids, ids2) and torch.equal(weights, weights2) and torch.equal(hid, hid2)
    assert torch.equal(out, out2)


def test_moe_block_acc_writes_nan_when_the_flag_is_set():
    print_case("moe_decode_block_acc flag")
    lib = _native.lib()
    dim, hidden, experts, top_k = 256, 512, 4, 2
    t = moe_inputs(dim, hidden, experts, seed=1)
    acc = torch.zeros(dim + 1, dtype=torch.int64, device="cuda")
    acc[dim] = 1
    h_out = torch.empty(dim, device="cuda")
    logits, ids, weights, hid, out = moe_scratch(dim, hidden, experts, top_k)
    rc = lib.mie_moe_decode_block_acc(
        t["x"].data_ptr(), acc.data_ptr(), t["b_out"].data_ptr(), h_out.data_ptr(), t["ln_w"].data_ptr(),
        t["ln_b"].data_ptr(), 1e-5, t["router"].data_ptr(), t["w1"].data_ptr(), t["b1"].data_ptr(),
        t["w2"].data_ptr(), t["b2"].data_ptr(), experts, top_k, dim, hidden, logits.data_ptr(), ids.data_ptr(),
        weights.data_ptr(), hid.data_ptr(), out.data_ptr(), 0, stream())
    _native.check(rc, "mie_moe_decode_block_acc")
    torch.cuda.synchronize()
    assert torch.isnan(h_out).all() and torch.isnan(out).all()
    assert not acc.any()


@pytest.mark.parametrize("heads,head_dim,block_size,lens", [CASES[0], CASES[3], CASES[5]])
def test_attn_out_bf16_matches_float64_on_rounded_head_outputs(heads, head_dim, block_size, lens):
    """bfloat16 q, pools and W_out: each head's attention output is rounded
    to bfloat16 before the projection (as the decode kernels store it), then
    projected and summed in fixed point.  Against float64 attention on the
    same bfloat16 values, rounded the same way: a float32 softmax can put a
    head output on the other side of a bfloat16 rounding boundary, so at
    least 98 % of rows meet the float32 bound and every row a bound one
    bfloat16 ulp of the row's scale wider."""
    print_case("attn_out bf16", heads, head_dim, block_size, lens)
    w = make_workload(lens, num_heads=heads, head_dim=head_dim, block_size=block_size, dtype=torch.bfloat16,
                      seed=heads + head_dim + block_size, heavy_fraction=0.02)
    dim = heads * head_dim
    g = torch.Generator(device="cuda").manual_seed(7)
    w_out = (torch.randn(dim, dim, generator=g, device="cuda") / math.sqrt(dim)).to(torch.bfloat16)
    w64 = ref.to_f64(w_out)
    for b in range(len(lens)):
        acc = torch.zeros(dim + 1, dtype=torch.int64, device="cuda")
        attn_out(w, b, w_out, acc, dtype=1)
        k, v = sequence_kv(w, b)
        a = ref.attention_fp64(ref.to_f64(w.q[b]), ref.to_f64(k), ref.to_f64(v)).reshape(-1)
        a = torch.from_numpy(a).to(torch.bfloat16).double().numpy()
        want, scale = w64 @ a, np.abs(w64) @ np.abs(a)
        got = acc[:dim].cpu().numpy().astype(np.float64) * FIX
        assert int(acc[dim]) == 0
        err = np.abs(got - want)
        tight = err <= 2e-5 * scale + 1e-6
        assert tight.mean() >= 0.98, f"only {tight.mean():.1%} of rows within the float32 bound"
        assert (err <= (2e-5 + 2.0 ** -7) * scale + 1e-6).all(), f"max error {err.max():.3e}"
        again = torch.zeros_like(acc)
        attn_out(w, b, w_out, again, dtype=1)
        assert torch.equal(acc, again), "the fixed-point sums differ between runs"


def test_moe_block_acc_bf16_forms_the_rounded_residual():
    """bfloat16: h_out = round(x + round(acc * 2^-32 + b_out)) - the
    projection's output, then the residual, each rounded to bfloat16 as
    mie_linear_residual stores them - bit for bit against torch's float32
    arithmetic and rounding, then the MoE half exactly as mie_moe_decode_block
    computes it on h_out."""
    print_case("moe_decode_block_acc bf16")
    lib = _native.lib()
    dim, hidden, experts, top_k = 768, 2048, 8, 2
    t = {k: v.to(torch.bfloat16) for k, v in moe_inputs(dim, hidden, experts, seed=11).items()}
    acc = torch.zeros(dim + 1, dtype=torch.int64, device="cuda")
    acc[:dim] = torch.round(t["o"].double() / FIX).long()
    proj = (acc[:dim].float() * FIX + t["b_out"].float()).to(torch.bfloat16)
    h_want = (t["x"].float() + proj.float()).to(torch.bfloat16)
    h_out = torch.empty(dim, dtype=torch.bfloat16, device="cuda")
    z = lambda *shape, dtype=torch.float32: torch.zeros(*shape, dtype=dtype, device="cuda")  # noqa: E731

    def scratch():
        return z(experts), z(top_k, dtype=torch.int32), z(top_k), z(top_k, hidden, dtype=torch.bfloat16), \
            z(dim, dtype=torch.bfloat16)

    logits, ids, weights, hid, out = scratch()
    rc = lib.mie_moe_decode_block_acc(
        t["x"].data_ptr(), acc.data_ptr(), t["b_out"].data_ptr(), h_out.data_ptr(), t["ln_w"].data_ptr(),
        t["ln_b"].data_ptr(), 1e-5, t["router"].data_ptr(), t["w1"].data_ptr(), t["b1"].data_ptr(),
        t["w2"].data_ptr(), t["b2"].data_ptr(), experts, top_k, dim, hidden, logits.data_ptr(), ids.data_ptr(),
        weights.data_ptr(), hid.data_ptr(), out.data_ptr(), 1, stream())
    _native.check(rc, "mie_moe_decode_block_acc")
    torch.cuda.synchronize()
    assert torch.equal(h_out, h_want)
    assert not acc.any(), "the accumulator is not cleared"
    logits2, ids2, weights2, hid2, out2 = scratch()
    rc = lib.mie_moe_decode_block(
        h_want.data_ptr(), t["ln_w"].data_ptr(), t["ln_b"].data_ptr(), 1e-5, t["router"].data_ptr(),
        t["w1"].data_ptr(), t["b1"].data_ptr(), t["w2"].data_ptr(), t["b2"].data_ptr(), experts, top_k, dim, hidden,
        logits2.data_ptr(), ids2.data_ptr(), weights2.data_ptr(), hid2.data_ptr(), out2.data_ptr(), 1, stream())
    _native.check(rc, "mie_moe_decode_block")
    assert torch.equal(ids, ids2) and torch.equal(weights, weights2) and torch.equal(hid, hid2)
    assert torch.equal(out, out2)

