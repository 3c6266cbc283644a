"""The decode step's two ends on the GPU: mie_embed (token plus positional
embedding, reference src/moe_engine/model.py:558) and mie_lm_head (final_norm
+ output_projection, model.py:564-565, with generate's greedy torch.argmax,
model.py:603).

The head's logits are checked against float64 LayerNorm + linear on the same
inputs (float32 within 1e-5 of the row's absolute-value scale; bfloat16
within one bf16 rounding plus 1e-4 of the scale); its pick must equal
torch.argmax over the logits it stored, bit for bit, including ties (the first
index wins) and NaN (the first NaN wins).  The embedding must equal PyTorch's
sum of the two rows exactly.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from conftest import print_case
from moe_engine import embedding, projection

pytestmark = pytest.mark.gpu


def make_head(vocab, dim, dtype, norm, bias, seed):
    g = torch.Generator().manual_seed(seed)
    linear = nn.Linear(dim, vocab, bias=bias)
    with torch.no_grad():
        linear.weight.copy_(torch.randn(vocab, dim, generator=g))
        if bias:
            linear.bias.copy_(torch.rand(vocab, generator=g) - 0.5)
    ln = None
    if norm:
        ln = nn.LayerNorm(dim)
        with torch.no_grad():
            ln.weight.copy_(1 + 0.1 * torch.randn(dim, generator=g))
            ln.bias.copy_(0.1 * torch.randn(dim, generator=g))
        ln = ln.to("cuda", dtype)
    x = (torch.randn(dim, generator=g) * 2 + 0.3).to(dtype)
    return x.cuda(), ln, linear.to("cuda", dtype)


@torch.no_grad()
def head_f64(x, ln, linear):
    """float64 LayerNorm + linear; the norm output rounded to the model dtype
    as the model feeds it to the projection."""
    y = x.double().cpu()
    if ln is not None:
        y = F.layer_norm(y, y.shape, ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    y = y.to(x.dtype).double()
    w = linear.weight.double().cpu()
    out = w @ y
    scale = w.abs() @ y.abs()
    if linear.bias is not None:
        out = out + linear.bias.double().cpu()
        scale = scale + linear.bias.double().cpu().abs()
    return out.numpy(), scale.numpy()


def pick(logits):
    return int(torch.argmax(logits))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("vocab,dim", [(50257, 768), (1, 64), (17, 128), (1000, 2048), (4099, 96)])
@pytest.mark.parametrize("norm,bias", [(True, True), (False, False), (True, False)])
def test_lm_head_logits_and_pick(dtype, vocab, dim, norm, bias):
    if not projection.supported(dim, dtype):
        pytest.skip(f"width {dim} not built for {dtype}")
    print_case("lm_head", dtype, vocab, dim, norm, bias)
    x, ln, linear = make_head(vocab, dim, dtype, norm, bias, seed=vocab + dim)
    token = torch.full((1,), -7, dtype=torch.int64, device="cuda")
    logits = projection.lm_head(x, ln, linear, token_out=token)
    want, scale = head_f64(x, ln, linear)
    got = logits.double().cpu().numpy()
    if dtype == torch.float32:
        bound = 1e-5 * scale + 1e-6
    else:
        bound = 2.0**-7 * np.abs(want) + 1e-4 * scale
    err = np.abs(got - want)
    worst = int(np.argmax(err - bound))
    assert (err <= bound).all(), f"row {worst}: error {err[worst]:.3e} > {bound[worst]:.3e}"
    assert int(token) == pick(logits)
    # The logits alone: same values, the token untouched.
    token.fill_(-7)
    again = projection.lm_head(x, ln, linear)
    assert torch.equal(again, logits) and int(token) == -7


def test_lm_head_pick_keeps_argmax_ties_and_nan_rules():
    """Equal logits: the lowest index wins, also across workgroups; NaN
    logits: the first NaN wins over every number."""
    vocab, dim = 5000, 64
    x, _, linear = make_head(vocab, dim, torch.float32, False, False, seed=5)
    token = torch.zeros(1, dtype=torch.int64, device="cuda")
    with torch.no_grad():
        w = linear.weight
        w.mul_(0.01)
        w[4321] = x * 0.5  # a clear maximum, then copies of it before and after
        w[77] = w[4321]
        w[4999] = w[4321]
        w[3] = w[4321]
    logits = projection.lm_head(x, None, linear, token_out=token)
    assert logits[3] == logits[77] == logits[4321] == logits.max()
    assert int(token) == 3 == pick(logits)
    with torch.no_grad():
        linear.weight[2500, 0] = float("nan")
        linear.weight[4000, 0] = float("nan")
    logits = projection.lm_head(x, None, linear, token_out=token)
    assert int(token) == 2500 == pick(logits)
    with torch.no_grad():
        linear.weight.fill_(0)
    logits = projection.lm_head(x, None, linear, token_out=token)
    assert int(token) == 0 == pick(logits)


class _Counted:
    """Counts calls of two library entry points (the full pick and the merge
    of kept picks) while forwarding them."""

    def __init__(self, monkeypatch):
        from moe_engine import _native

        lib = _native.lib()
        self.calls = {"mie_argmax": 0, "mie_argmax_pairs": 0}
        for name in self.calls:
            real = getattr(lib, name)

            def counted(*args, _real=real, _name=name):
                self.calls[_name] += 1
                return _real(*args)

            monkeypatch.setattr(lib, name, counted)


@torch.no_grad()
def test_argmax_of_fresh_head_logits_merges_the_kept_picks(monkeypatch):
    """lm_head(keep_pick=True) leaves its workgroups' picks; argmax of those
    logits, or of a view of them, merges the picks (one small launch) and
    returns torch.argmax's index, ties and NaN included.  Logits written
    since - in place, by a later head call into the same buffer, or replaced
    by a newer keep_pick call - are read in full instead."""
    counted = _Counted(monkeypatch)
    vocab, dim = 5000, 64
    x, ln, linear = make_head(vocab, dim, torch.float32, True, True, seed=9)
    logits = projection.lm_head(x, ln, linear, keep_pick=True)
    assert int(projection.argmax(logits)) == pick(logits)
    assert int(projection.argmax(logits.view(1, 1, -1)[:, -1, :].reshape(-1))) == pick(logits)
    assert counted.calls == {"mie_argmax": 0, "mie_argmax_pairs": 2}

    # Ties across workgroups (the lowest index wins) and NaN (the first wins).
    x2, _, tied = make_head(vocab, dim, torch.float32, False, False, seed=5)
    tied.weight.mul_(0.01)
    for row in (3, 77, 4321, 4999):
        tied.weight[row] = x2 * 0.5
    logits = projection.lm_head(x2, None, tied, keep_pick=True)
    assert int(projection.argmax(logits)) == 3 == pick(logits)
    tied.weight[2500, 0] = float("nan")
    tied.weight[4000, 0] = float("nan")
    logits = projection.lm_head(x2, None, tied, keep_pick=True)
    assert int(projection.argmax(logits)) == 2500 == pick(logits)
    assert counted.calls["mie_argmax"] == 0

    # Written in place after the head: a full pick of the new values.
    logits = projection.lm_head(x, ln, linear, keep_pick=True)
    logits[4990] = 1e30
    assert int(projection.argmax(logits)) == 4990
    assert counted.calls["mie_argmax"] == 1
    # A newer keep_pick call replaces the picks: the older logits are read in full.
    old = projection.lm_head(x, ln, linear, keep_pick=True)
    new = projection.lm_head(x2, None, tied, keep_pick=True)
    assert int(projection.argmax(old)) == pick(old) and counted.calls["mie_argmax"] == 2
    assert int(projection.argmax(new)) == pick(new) and counted.calls["mie_argmax"] == 2
    # A head call without keep_pick rewriting the recorded logits drops the picks.
    kept = projection.lm_head(x2, None, tied, keep_pick=True)
    projection.lm_head(x, ln, linear, out=kept)
    assert int(projection.argmax(kept)) == pick(kept) and counted.calls["mie_argmax"] == 3

    # Each host thread keeps its own picks: another thread's head (same device
    # and vocabulary) neither replaces nor overwrites this thread's.
    import threading

    mine = projection.lm_head(x, ln, linear, keep_pick=True)
    theirs = {}
    worker = threading.Thread(target=lambda: theirs.update(
        logits=projection.lm_head(x2, None, tied, keep_pick=True)))
    worker.start()
    worker.join()
    torch.cuda.synchronize()
    merges = counted.calls["mie_argmax_pairs"]
    assert int(projection.argmax(mine)) == pick(mine)
    assert counted.calls["mie_argmax_pairs"] == merges + 1 and counted.calls["mie_argmax"] == 3
    assert not projection.can_argmax(theirs["logits"].bfloat16())  # not this thread's logits, not float32


def test_lm_head_advances_counters_after_the_pick():
    x, ln, linear = make_head(700, 64, torch.float32, True, True, seed=2)
    token = torch.zeros(1, dtype=torch.int64, device="cuda")
    counters = torch.tensor([5, 6, -1], dtype=torch.int32, device="cuda")
    for step in range(3):
        logits = projection.lm_head(x, ln, linear, token_out=token, advance=counters)
    assert counters.tolist() == [8, 9, 2]
    assert int(token) == pick(logits)
    with pytest.raises(ValueError, match="token_out"):
        projection.lm_head(x, ln, linear, advance=counters)


def test_lm_head_validates_before_launch():
    x, ln, linear = make_head(300, 64, torch.float32, True, True, seed=1)
    token = torch.zeros(1, dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError, match="workspace"):
        projection.lm_head(x, ln, linear, token_out=token, workspace=torch.empty(8, dtype=torch.uint8, device="cuda"))
    with pytest.raises(ValueError, match="int64"):
        projection.lm_head(x, ln, linear, token_out=token.int())
    with pytest.raises(ValueError, match="contiguous"):
        projection.lm_head(torch.randn(128, device="cuda")[::2], ln, linear)
    assert projection.head_workspace_bytes(300) >= 8 * math.ceil(300 / 64)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_embed_equals_torch_sum(dtype):
    print_case("embed", dtype)
    torch.manual_seed(3)
    tok = nn.Embedding(50257, 768).to("cuda", dtype)
    pos = nn.Embedding(1024, 768).to("cuda", dtype)
    ids = torch.tensor([[0, 50256, 17, 17, 40000]], device="cuda")
    positions = torch.tensor([0, 1023, 5, 6, 511], dtype=torch.int32, device="cuda")
    got = embedding.embed(ids, positions, tok, pos)
    want = tok(ids) + pos(positions.long())
    assert got.shape == want.shape and torch.equal(got, want)


def test_embed_out_of_range_gives_nan_rows():
    tok = nn.Embedding(10, 32).cuda()
    pos = nn.Embedding(8, 32).cuda()
    ids = torch.tensor([[3, 10, -1, 4]], device="cuda")
    positions = torch.tensor([0, 1, 2, 8], dtype=torch.int32, device="cuda")
    got = embedding.embed(ids, positions, tok, pos)[0]
    assert torch.equal(got[0], tok.weight[3] + pos.weight[0])
    assert torch.isnan(got[1:]).all()
