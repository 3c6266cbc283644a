"""mie_qkv_append: one decode token's QKV projection with K and V stored
straight into the paged pools, against the oracle (qkv_project_fp64, then
append_rows for the placement).

Tolerances, per output element r with scale_r = sum_j |W_rj y_j| + |b_r|
(float64, from the oracle's inputs):
  float32: |got - want| <= 1e-5 * scale_r + 1e-6   (float32 accumulation of
           `dim` products; the kernel and torch's GEMM order them differently)
  bf16:    |got - want| <= 2^-7 * |want| + 1e-4 * scale_r   (one rounding of
           the output to bf16, plus norm outputs that round to neighbouring
           bf16 values when the float32 and float64 norms straddle a tie)
Every pool element other than the token's K and V rows must keep its bits.
"""

import math

import numpy as np
import pytest
import torch

from conftest import print_case
from moe_engine import kv_ops
from moe_engine.model import Model, ModelConfig
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu


def round_to(dtype):
    return lambda y: torch.from_numpy(np.asarray(y)).to(dtype).double().numpy()


def make_inputs(heads, head_dim, dtype, norm, bias, seed):
    dim = heads * head_dim
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(dim, generator=g) * 2 + 0.3).to(dtype)
    w = (torch.randn(3 * dim, dim, generator=g) / math.sqrt(dim)).to(dtype)
    b = (torch.randn(3 * dim, generator=g) * 0.1).to(dtype) if bias else None
    nw = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype) if norm else None
    nb = (0.1 * torch.randn(dim, generator=g)).to(dtype) if norm else None
    return x, w, b, nw, nb


def expected(x, w, b, nw, nb, heads, dtype):
    q, k, v = ref.qkv_project_fp64(x, w, b, heads, nw, nb, 1e-5, round_to(dtype))
    y = ref.to_f64(x)
    if nw is not None:
        y = round_to(dtype)(
            (y - y.mean()) / math.sqrt(((y - y.mean()) ** 2).mean() + 1e-5) * ref.to_f64(nw) + ref.to_f64(nb)
        )
    else:
        y = round_to(dtype)(y)
    scale = np.abs(ref.to_f64(w)) @ np.abs(y) + (np.abs(ref.to_f64(b)) if b is not None else 0.0)
    dim = y.shape[0]
    return (q, k, v), [scale[i * dim : (i + 1) * dim].reshape(q.shape) for i in range(3)]


def assert_close(got, want, scale, dtype, what):
    got = ref.to_f64(got).reshape(want.shape)
    err = np.abs(got - want)
    if dtype == torch.float32:
        bound = 1e-5 * scale + 1e-6
    else:
        bound = 2.0**-7 * np.abs(want) + 1e-4 * scale
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert (err <= bound).all(), f"{what}: error {err[worst]:.3e} > bound {bound[worst]:.3e} at {worst}"


def pools(layers, num_blocks, heads, block_size, head_dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    shape = (layers, num_blocks, heads, block_size, head_dim)
    return torch.randn(shape, generator=g).to(dtype).cuda(), torch.randn(shape, generator=g).to(dtype).cuda()


CASES = [
    # dtype, heads, head_dim, block_size, norm, bias, position
    (torch.float32, 12, 64, 16, True, True, 37),  # config 1
    (torch.bfloat16, 12, 64, 16, True, True, 37),
    (torch.float32, 8, 96, 16, True, True, 0),  # production attention dims
    (torch.bfloat16, 8, 96, 16, False, True, 15),
    (torch.float32, 2, 16, 5, False, False, 23),
    (torch.bfloat16, 4, 32, 1, True, False, 9),
    (torch.float32, 32, 64, 16, True, True, 100),  # dim 2048, the float32 maximum
    (torch.bfloat16, 32, 128, 16, True, True, 100),  # dim 4096, the bf16 maximum
]


@pytest.mark.parametrize("dtype,heads,head_dim,block_size,norm,bias,position", CASES)
@pytest.mark.parametrize("device_position", [False, True])
def test_qkv_append_matches_oracle(dtype, heads, head_dim, block_size, norm, bias, position, device_position):
    print_case("qkv_append", dtype, heads, head_dim, block_size, norm, bias, position, device_position)
    x, w, b, nw, nb = make_inputs(heads, head_dim, dtype, norm, bias, seed=heads * 7 + head_dim)
    num_blocks = -(-(position + 1) // block_size) + 6
    kp, vp = pools(2, num_blocks, heads, block_size, head_dim, dtype, seed=5)
    k0, v0 = kp.cpu(), vp.cpu()
    table = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(9)).int()
    dev = lambda t: None if t is None else t.cuda()
    pos_dev = torch.tensor([position], dtype=torch.int32, device="cuda") if device_position else None
    q = kv_ops.qkv_append(dev(x), dev(w), dev(b), kp, vp, 1, table.cuda(), position=0 if device_position else position,
                          position_dev=pos_dev, norm_weight=dev(nw), norm_bias=dev(nb))
    (wq, wk, wv), (sq, sk, sv) = expected(x, w, b, nw, nb, heads, dtype)
    assert q.shape == (1, heads, 1, head_dim) and q.dtype == dtype
    assert_close(q.cpu()[0, :, 0], wq, sq, dtype, "q")
    blk, slot = int(table[position // block_size]), position % block_size
    assert_close(kp.cpu()[1, blk, :, slot], wk, sk, dtype, "k row")
    assert_close(vp.cpu()[1, blk, :, slot], wv, sv, dtype, "v row")
    # Everything else keeps its bits: restore the written rows, compare whole pools.
    for got, before in ((kp.cpu(), k0), (vp.cpu(), v0)):
        got[1, blk, :, slot] = before[1, blk, :, slot]
        assert np.array_equal(ref.raw_bits(got), ref.raw_bits(before))


def draw_qkv(seed):
    """A random supported case: dtype, heads, head_dim (widths up to 2048),
    block size, norm and bias present or not, position, host or device."""
    import random

    rng = random.Random(seed)
    while True:
        dtype = rng.choice((torch.float32, torch.bfloat16))
        heads = rng.choice((1, 2, 3, 5, 8, 12, 16))
        head_dim = rng.choice((4, 8, 12, 16, 24, 32, 40, 64, 96, 128))
        if heads * head_dim <= 2048 and kv_ops.qkv_append_supported(heads * head_dim, dtype):
            break
    return (dtype, heads, head_dim, rng.choice((1, 3, 4, 16, 32)), rng.random() < 0.7, rng.random() < 0.7,
            rng.randint(0, 300), rng.random() < 0.5)


@pytest.mark.parametrize("seed", range(24))
def test_random_qkv_append_matches_oracle(seed):
    """Drawn cases through the same checks as the fixed ones above."""
    test_qkv_append_matches_oracle(*draw_qkv(seed))


def test_rows_land_where_append_rows_puts_them():
    """Placement against the oracle's append: the pool after the fused call
    equals append_rows of the kernel's own K/V values at every position."""
    heads, head_dim, bs, nb = 4, 16, 4, 8
    x, w, b, nw, nbias = make_inputs(heads, head_dim, torch.float32, True, True, seed=3)
    kp, vp = pools(1, nb, heads, bs, head_dim, torch.float32, seed=4)
    table = torch.tensor([5, 2, 7, 0, 1, 3, 6, 4], dtype=torch.int32)
    want_k, want_v = kp.cpu().numpy(), vp.cpu().numpy()
    for position in range(nb * bs):
        xt = x + 0.01 * position
        q = kv_ops.qkv_append(xt.cuda(), w.cuda(), b.cuda(), kp, vp, 0, table.cuda(), position=position,
                              norm_weight=nw.cuda(), norm_bias=nbias.cuda())
        torch.cuda.synchronize()
        blk, slot = int(table[position // bs]), position % bs
        k_new = kp.cpu()[0, blk, :, slot].numpy()[:, None, :]
        v_new = vp.cpu()[0, blk, :, slot].numpy()[:, None, :]
        ref.append_rows(want_k, want_v, 0, table.tolist(), position, k_new, v_new)
        (wq, wk, _), (sq, sk, _) = expected(xt, w, b, nw, nbias, heads, torch.float32)
        assert_close(k_new[:, 0], wk, sk, torch.float32, f"k at {position}")
    assert np.array_equal(kp.cpu().numpy(), want_k)
    assert np.array_equal(vp.cpu().numpy(), want_v)


def test_unmapped_blocks_are_skipped():
    """A table entry outside [0, num_blocks), or a device position past the
    table, stores no K/V (as mie_kv_append skips such rows); q is still written."""
    heads, head_dim, bs, nb = 2, 16, 4, 4
    x, w, b, _, _ = make_inputs(heads, head_dim, torch.float32, False, True, seed=8)
    kp, vp = pools(1, nb, heads, bs, head_dim, torch.float32, seed=6)
    k0, v0 = kp.clone(), vp.clone()
    for table, position in (([0, nb, 1, 2], 5), ([0, -1, 1, 2], 6), ([0, 1], 9)):
        t = torch.tensor(table, dtype=torch.int32, device="cuda")
        pos_dev = torch.tensor([position], dtype=torch.int32, device="cuda")
        q = kv_ops.qkv_append(x.cuda(), w.cuda(), b.cuda(), kp, vp, 0, t, position_dev=pos_dev)
        torch.cuda.synchronize()
        assert torch.equal(kp, k0) and torch.equal(vp, v0)
        (wq, _, _), (sq, _, _) = expected(x, w, b, None, None, heads, torch.float32)
        assert_close(q.cpu()[0, :, 0], wq, sq, torch.float32, "q")


def test_wrapper_validates_before_launch():
    x, w, b, nw, nb = make_inputs(2, 16, torch.float32, True, True, seed=1)
    kp, vp = pools(1, 4, 2, 4, 16, torch.float32, seed=2)
    t = torch.arange(4, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="in_proj_weight"):
        kv_ops.qkv_append(x.cuda(), w[:-1].cuda(), b.cuda(), kp, vp, 0, t, position=1)
    with pytest.raises(ValueError, match="position"):
        kv_ops.qkv_append(x.cuda(), w.cuda(), b.cuda(), kp, vp, 0, t, position=16)
    with pytest.raises(ValueError, match="dtype"):
        kv_ops.qkv_append(x.double().cuda(), w.cuda(), b.cuda(), kp, vp, 0, t, position=1)
    with pytest.raises(ValueError, match="norm bias"):
        kv_ops.qkv_append(x.cuda(), w.cuda(), b.cuda(), kp, vp, 0, t, position=1, norm_bias=nb.cuda())
    assert not kv_ops.qkv_append_supported(4100, torch.float32)
    assert not kv_ops.qkv_append_supported(770, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_model_decode_with_and_without_fused_projection(dtype):
    """Decode logits with the fused projection agree with the reference's
    projection + append sequence (float32: 1e-4, as the reference's
    direct-vs-gather model test; bf16: 1 % relative), tokens identical."""
    print_case("model fused qkv", dtype)
    torch.manual_seed(0)
    model = Model(ModelConfig(max_seq_length=256, num_layers=2)).to("cuda", dtype).eval()
    ids = torch.randint(0, 1000, (1, 40), device="cuda")
    logits = {}
    for fuse in (False, True):
        allocator = model.new_block_allocator(num_blocks=16, block_size=16, attention_mode="direct")
        assert allocator.fuse_qkv
        allocator.fuse_qkv = fuse
        cache = allocator.new_cache()
        with torch.no_grad():
            steps = [model(ids[:, :30], cache)[:, -1]]
            steps += [model(ids[:, t : t + 1], cache)[:, -1] for t in range(30, 40)]
        logits[fuse] = torch.stack(steps, 1).float()
    if dtype == torch.float32:
        torch.testing.assert_close(logits[True], logits[False], atol=1e-4, rtol=1e-4)
    else:
        rel = ((logits[True] - logits[False]).norm() / logits[False].norm()).item()
        assert rel < 1e-2, rel


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols,residual,bias", [(768, 768, True, True), (96, 2048, False, True),
                                                       (50, 64, True, False), (3, 8, False, False)])
def test_linear_residual_matches_float64(dtype, rows, cols, residual, bias):
    """out = residual + round(W x + b) (the attention's out_proj plus the
    block's residual add) against float64 on the same inputs, with the
    projection's output rounding to the model dtype."""
    from moe_engine import projection

    if not projection.supported(cols, dtype):
        pytest.skip(f"width {cols} not built for {dtype}")
    print_case("linear_residual", dtype, rows, cols, residual, bias)
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(cols, generator=g).to(dtype)
    w = (torch.randn(rows, cols, generator=g) / math.sqrt(cols)).to(dtype)
    b = (torch.randn(rows, generator=g) * 0.1).to(dtype) if bias else None
    r = torch.randn(rows, generator=g).to(dtype) if residual else None
    got = projection.linear_residual(x.cuda(), w.cuda(), None if b is None else b.cuda(),
                                     None if r is None else r.cuda())
    proj = ref.to_f64(w) @ ref.to_f64(x) + (ref.to_f64(b) if b is not None else 0.0)
    scale = np.abs(ref.to_f64(w)) @ np.abs(ref.to_f64(x)) + (np.abs(ref.to_f64(b)) if b is not None else 0.0)
    if residual:
        proj_rounded = round_to(dtype)(proj)
        want = ref.to_f64(r) + proj_rounded
        got_f = ref.to_f64(got.cpu())
        # the projection's error, then one more rounding of the sum
        bound = (1e-5 * scale + 1e-6) if dtype == torch.float32 else (2.0**-7 * (np.abs(want) + np.abs(proj)) + 1e-4 * scale)
        assert (np.abs(got_f - want) <= bound).all()
    else:
        assert_close(got.cpu(), proj, scale, dtype, "linear")


def test_linear_residual_may_write_over_its_residual():
    from moe_engine import projection

    x = torch.randn(64, device="cuda")
    w = torch.randn(32, 64, device="cuda") / 8
    r = torch.randn(32, device="cuda")
    want = r + w @ x
    projection.linear_residual(x, w, None, r, out=r)
    torch.testing.assert_close(r, want, atol=1e-5, rtol=1e-5)
    with pytest.raises(ValueError, match="alias"):
        projection.linear_residual(x[:32].contiguous(), torch.eye(32, device="cuda"), out=x[:32])
