"""Host-side argument checks of every compute entry point, on the CPU.

Each check runs before anything is launched, so a call with one bad argument
must return its status and message here, with no GPU: a missing check would
instead reach the launch and come back as MIE_ERR_LAUNCH (4).  Pointers are
aligned stand-ins (never dereferenced by the checks); each case changes one
argument of a call that is otherwise valid.
"""

import ctypes

import pytest

from moe_engine import _native

INVALID, UNSUPPORTED, WORKSPACE = 1, 2, 3
F32, BF16 = 0, 1
_addr = iter(range(1 << 24, 1 << 40, 1 << 20))


def ptr():
    """A fresh 1 MiB-aligned stand-in address."""
    return next(_addr)


def call(name, args):
    lib = _native.lib()
    return getattr(lib, name)(*args), lib.mie_last_error()


def argmax_args(**over):
    a = dict(x=ptr(), n=50257, out=ptr(), dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def argmax_pairs_args(**over):
    a = dict(ws=ptr(), ws_bytes=_native.lib().mie_lm_head_workspace(50257), vocab=50257, out=ptr(), stream=None)
    a.update(over)
    return list(a.values())


def embed_args(**over):
    a = dict(ids=ptr(), positions=ptr(), position=0, n=1, tok=ptr(), vocab=1000, pos_table=ptr(), max_pos=128,
             dim=64, out=ptr(), dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def linear_args(**over):
    a = dict(x=ptr(), w=ptr(), b=ptr(), res=ptr(), out=ptr(), rows=768, cols=768, dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def lm_head_args(**over):
    ws = _native.lib().mie_lm_head_workspace(1000)
    a = dict(x=ptr(), ln_w=ptr(), ln_b=ptr(), eps=1e-5, w=ptr(), b=ptr(), vocab=1000, dim=64, logits=ptr(),
             token=ptr(), ws=ptr(), ws_bytes=ws, advance=ptr(), n_advance=2, dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def qkv_args(**over):
    a = dict(x=ptr(), ln_w=ptr(), ln_b=ptr(), eps=1e-5, w_in=ptr(), b_in=ptr(), dim=64, k=ptr(), v=ptr(),
             sblk=2 * 16 * 32, shead=16 * 32, num_blocks=8, table=ptr(), table_len=8, pos_dev=None, position=3,
             q=ptr(), heads=2, head_dim=32, block_size=16, dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def route_args(**over):
    a = dict(x=ptr(), router=ptr(), experts=8, top_k=2, dim=64, logits=ptr(), ids=ptr(), weights=ptr(), dtype=F32,
             stream=None)
    a.update(over)
    return list(a.values())


def moe_args(**over):
    a = dict(x=ptr(), router=ptr(), w1=ptr(), b1=ptr(), w2=ptr(), b2=ptr(), experts=8, top_k=2, dim=64, hidden=128,
             logits=ptr(), ids=ptr(), weights=ptr(), hid=ptr(), out=ptr(), dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def moe_block_args(**over):
    a = dict(x=ptr(), ln_w=ptr(), ln_b=ptr(), eps=1e-5, router=ptr(), w1=ptr(), b1=ptr(), w2=ptr(), b2=ptr(),
             experts=8, top_k=2, dim=64, hidden=128, logits=ptr(), ids=ptr(), weights=ptr(), hid=ptr(), out=ptr(),
             dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def moe_block_acc_args(**over):
    a = dict(x=ptr(), acc=ptr(), b_out=ptr(), h_out=ptr(), ln_w=ptr(), ln_b=ptr(), eps=1e-5, router=ptr(), w1=ptr(),
             b1=ptr(), w2=ptr(), b2=ptr(), experts=8, top_k=2, dim=64, hidden=128, logits=ptr(), ids=ptr(),
             weights=ptr(), hid=ptr(), out=ptr(), dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


def decode_args(append=False, noalloc=False, **over):
    a = dict(q=ptr(), q_sb=128, q_sh=64, k=ptr(), v=ptr(), sblk=2 * 16 * 64, shead=16 * 64, num_blocks=8,
             tables=ptr(), table_stride=8, ctx_dev=None, ctx_host=None, ctx=20, max_ctx=20, batch=1, heads=2,
             head_dim=64, block_size=16, scale=0.125, out=ptr(), o_sb=128, o_sh=64, out_dtype=F32)
    if not noalloc:
        a.update(ws=None, ws_bytes=0)
    a.update(partition=-1)
    if append:
        a.update(k_new=ptr(), v_new=ptr(), new_sb=128, new_sh=64)
    a.update(dtype=F32, stream=None)
    a.update(over)
    return list(a.values())


CASES = [
    # (entry point, arguments, status, message)
    ("mie_argmax", argmax_args(dtype=BF16), UNSUPPORTED, b"float32 only"),
    ("mie_argmax", argmax_args(n=0), INVALID, b"n=0"),
    ("mie_argmax", argmax_args(x=None), INVALID, b"null pointer"),
    ("mie_argmax_pairs", argmax_pairs_args(vocab=0), INVALID, b"vocab 0"),
    ("mie_argmax_pairs", argmax_pairs_args(ws=None), INVALID, b"null pointer"),
    ("mie_argmax_pairs", argmax_pairs_args(out=None), INVALID, b"null pointer"),
    ("mie_argmax_pairs", argmax_pairs_args(ws_bytes=64), INVALID, b"take"),
    ("mie_argmax_pairs", argmax_pairs_args(ws=ptr() + 2), INVALID, b"misaligned"),
    ("mie_argmax_pairs", argmax_pairs_args(out=ptr() + 4), INVALID, b"misaligned"),
    ("mie_embed", embed_args(dtype=3), UNSUPPORTED, b"dtype 3"),
    ("mie_embed", embed_args(n=-1), INVALID, b"n -1"),
    ("mie_embed", embed_args(vocab=0), INVALID, b"vocab 0"),
    ("mie_embed", embed_args(positions=None, position=-1), INVALID, b"position -1"),
    ("mie_embed", embed_args(tok=None), INVALID, b"null pointer"),
    ("mie_linear_residual", linear_args(cols=6), UNSUPPORTED, b"not built"),
    ("mie_linear_residual", linear_args(rows=0), INVALID, b"rows 0"),
    ("mie_linear_residual", linear_args(out=None), INVALID, b"null pointer"),
    ("mie_linear_residual", linear_args(w=ptr() + 4), INVALID, b"16-byte aligned"),
    ("mie_lm_head", lm_head_args(dim=6), UNSUPPORTED, b"not built"),
    ("mie_lm_head", lm_head_args(vocab=0), INVALID, b"vocab 0"),
    ("mie_lm_head", lm_head_args(logits=None), INVALID, b"null pointer"),
    ("mie_lm_head", lm_head_args(ln_w=None), INVALID, b"norm bias needs a norm weight"),
    ("mie_lm_head", lm_head_args(ws_bytes=8), INVALID, b"workspace"),
    ("mie_lm_head", lm_head_args(token=None, advance=None, n_advance=0, ws_bytes=8), INVALID, b"workspace"),
    ("mie_lm_head", lm_head_args(token=None, advance=None, n_advance=0, ws=ptr() + 2), INVALID, b"misaligned"),
    ("mie_lm_head", lm_head_args(n_advance=65), INVALID, b"counters to advance"),
    ("mie_lm_head", lm_head_args(token=ptr() + 4), INVALID, b"misaligned"),
    ("mie_qkv_append", qkv_args(dim=6, heads=1, head_dim=6), UNSUPPORTED, b"not built"),
    ("mie_qkv_append", qkv_args(heads=3), INVALID, b"!= dim"),
    ("mie_qkv_append", qkv_args(block_size=0), INVALID, b"block_size 0"),
    ("mie_qkv_append", qkv_args(q=None), INVALID, b"null pointer"),
    ("mie_qkv_append", qkv_args(ln_w=None), INVALID, b"norm bias needs a norm weight"),
    ("mie_qkv_append", qkv_args(x=ptr() + 8), INVALID, b"16-byte aligned"),
    ("mie_qkv_append", qkv_args(shead=16), INVALID, b"overlap"),
    ("mie_qkv_append", qkv_args(position=-1), INVALID, b"position -1"),
    ("mie_moe_route", route_args(dtype=3), UNSUPPORTED, b"float32 or bfloat16 only"),
    ("mie_moe_route", route_args(top_k=9), INVALID, b"top_k=9"),
    ("mie_moe_route", route_args(dim=66), INVALID, b"multiple of 4"),
    ("mie_moe_route", route_args(ids=None), INVALID, b"null pointer"),
    ("mie_moe_route", route_args(router=ptr() + 4), INVALID, b"16-byte aligned"),
    ("mie_moe_decode", moe_args(hidden=130), INVALID, b"hidden=130"),
    ("mie_moe_decode", moe_args(dim=2052), UNSUPPORTED, b"above 2048"),
    ("mie_moe_decode", moe_args(b2=None), INVALID, b"null pointer"),
    ("mie_moe_decode", moe_args(w2=ptr() + 4), INVALID, b"16-byte aligned"),
    ("mie_moe_decode", moe_args(experts=65), INVALID, b"experts=65"),
    ("mie_moe_decode_block", moe_block_args(ln_w=None), INVALID, b"needs a weight"),
    ("mie_moe_decode_block", moe_block_args(dtype=3), UNSUPPORTED, b"float32 or bfloat16 only"),
    ("mie_moe_decode_block_acc", moe_block_acc_args(dtype=3), UNSUPPORTED, b"float32 or bfloat16 only"),
    ("mie_moe_decode_block_acc", moe_block_acc_args(acc=None), INVALID, b"16-byte aligned"),
    ("mie_paged_decode", decode_args(head_dim=48, q_sh=48), UNSUPPORTED, b"not built"),
    ("mie_paged_decode", decode_args(partition=3), INVALID, b"partition_tokens 3"),
    ("mie_paged_decode", decode_args(ctx=30), INVALID, b"outside"),
    ("mie_paged_decode", decode_args(out=None), INVALID, b"null pointer"),
    ("mie_paged_decode", decode_args(shead=16), INVALID, b"pool strides overlap"),
    ("mie_paged_decode", decode_args(out_dtype=2), UNSUPPORTED, b"out_dtype 2"),
    ("mie_paged_decode", decode_args(q=ptr() + 8), INVALID, b"misaligned"),
    ("mie_paged_decode", decode_args(partition=16, ctx=400, max_ctx=400), WORKSPACE, b"workspace"),
    ("mie_paged_decode_append", decode_args(append=True, k_new=None), INVALID, b"null new rows"),
    ("mie_paged_decode_append", decode_args(append=True, ctx=0), INVALID, b"no slot for the new token"),
    ("mie_paged_decode_append", decode_args(append=True, v_new=ptr() + 2), INVALID, b"misaligned new rows"),
]


@pytest.mark.parametrize("name,args,status,message", CASES, ids=[f"{c[0]}-{i}" for i, c in enumerate(CASES)])
def test_a_bad_argument_fails_on_the_host(name, args, status, message):
    rc, err = call(name, args)
    assert rc == status, err
    assert message in err, err


def test_embed_of_no_tokens_is_a_no_op():
    """n = 0 is valid and launches nothing (so it succeeds without a GPU)."""
    rc, err = call("mie_embed", embed_args(n=0))
    assert rc == 0, err


def test_moe_decode_block_acc_refuses_h_out_aliasing_x():
    x = ptr()
    rc, err = call("mie_moe_decode_block_acc", moe_block_acc_args(x=x, h_out=x))
    assert rc == INVALID and b"must not alias x" in err


def test_support_queries_answer_on_the_host():
    lib = _native.lib()
    assert lib.mie_qkv_append_supported(768, F32) == 1
    assert lib.mie_qkv_append_supported(2048, F32) == 1
    assert lib.mie_qkv_append_supported(2052, F32) == 0  # above the 8 x 64 x 4 elements a wave holds
    assert lib.mie_qkv_append_supported(6, F32) == 0  # not a multiple of 4
    assert lib.mie_qkv_append_supported(4096, BF16) == 1 and lib.mie_qkv_append_supported(4, BF16) == 0
    assert lib.mie_qkv_append_supported(768, 3) == 0
    for head_dim in (4, 8, 16, 32, 64, 96, 128, 256):
        assert lib.mie_paged_decode_supported(head_dim, F32) == 1
        assert lib.mie_paged_decode_supported(head_dim, BF16) == 1
    assert lib.mie_paged_decode_supported(48, F32) == 0
    assert lib.mie_paged_decode_supported(64, 2) == 0


def test_embedding_plan_entries_fail_on_the_host():
    lib = _native.lib()
    size = lib.mie_block_plan_bytes()
    raw = ctypes.create_string_buffer(size)
    rc = lib.mie_block_plan_set_embedding(None, ptr(), 100, ptr(), 64, ptr())
    assert rc == INVALID and b"null plan" in lib.mie_last_error()
    rc = lib.mie_block_plan_set_embedding(raw, ptr(), 100, ptr(), 64, ptr())
    assert rc == INVALID and b"not initialised" in lib.mie_last_error()
    rc = lib.mie_block_decode_embed(raw, None, None, 3, None)
    assert rc == INVALID and b"null token id" in lib.mie_last_error()
    rc = lib.mie_block_decode_embed(raw, ptr(), None, 3, None)
    assert rc == INVALID and b"not initialised" in lib.mie_last_error()


def test_block_table_append_and_empty_launch_fail_on_the_host():
    lib = _native.lib()
    ids = (ctypes.c_int32 * 17)(*range(17))
    rc = lib.mie_block_table_append(ptr(), 64, 0, ids, 17, None)
    assert rc == INVALID and b"count 17" in lib.mie_last_error()
    rc = lib.mie_block_table_append(ptr(), 64, -1, ids, 1, None)
    assert rc == INVALID and b"outside a table" in lib.mie_last_error()
    rc = lib.mie_block_table_append(ptr(), 64, 60, ids, 5, None)
    assert rc == INVALID and b"outside a table" in lib.mie_last_error()
    rc = lib.mie_block_table_append(None, 64, 0, ids, 1, None)
    assert rc == INVALID and b"null pointer" in lib.mie_last_error()
    assert lib.mie_block_table_append(None, 0, 0, ids, 0, None) == 0  # nothing to append: no launch
    rc = lib.mie_empty_launch(0, None)
    assert rc == INVALID and b"workgroups 0" in lib.mie_last_error()
