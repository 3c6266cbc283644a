"""ctypes binding of libmie_paged.so, the C ABI in include/mie_paged_kv.h.

torch is imported before the library is opened: torch's bundled HIP runtime and
the system one share the SONAME libamdhip64.so.7, so opening the library after
torch makes the dynamic linker reuse torch's runtime and the process holds one
HIP runtime, one set of streams and one device context.

Nothing here falls back to another implementation.  When the library is
missing, `lib()` raises and every device entry point of the engine fails loudly.
"""

import ctypes
from functools import lru_cache
from pathlib import Path

import torch

LIB_NAME = "libmie_paged.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
ABI_VERSION = 16

# enum mie_dtype
DTYPE_CODES = {
    torch.float32: 0,
    torch.bfloat16: 1,
    torch.float16: 2,
    torch.float64: 3,
}
DECODE_DTYPES = (torch.float32, torch.bfloat16)

# enum mie_status codes the host acts on
ERR_WORKSPACE = 3

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

_SIGNATURES = {
    "mie_abi_version": (_i32, []),
    "mie_last_error": (ctypes.c_char_p, []),
    "mie_empty_launch": (_i32, [_i32, _c_void_p]),
    "mie_kv_append": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i32,  # pools, strides, num_blocks
         _c_void_p, _c_void_p, _i64, _i64, _i64,  # new K/V, strides b/h/s
         _c_void_p, _i64,  # block tables, stride
         _c_void_p, _i32,  # positions, position
         _i32, _i32, _i32, _i32, _i32,  # batch, seq_len, heads, head_dim, block_size
         _i32, _c_void_p],  # dtype, stream
    ),
    "mie_kv_gather": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i32,  # pools, strides, num_blocks
         _c_void_p, _i32,  # block table, length
         _c_void_p, _c_void_p, _i64, _i64,  # outputs, strides h/t
         _i32, _i32, _i32, _i32, _c_void_p],  # heads, head_dim, block_size, dtype, stream
    ),
    "mie_block_table_append": (_i32, [_c_void_p, _i32, _i32, ctypes.POINTER(_i32), _i32, _c_void_p]),
    "mie_paged_decode": (
        _i32,
        [_c_void_p, _i64, _i64,  # q, strides b/h
         _c_void_p, _c_void_p, _i64, _i64, _i32,  # pools, strides, num_blocks
         _c_void_p, _i64,  # block tables, stride
         _c_void_p, _c_void_p, _i32, _i32,  # ctx_lens (device), ctx_lens (host), ctx_len, max_ctx_len
         _i32, _i32, _i32, _i32,  # batch, heads, head_dim, block_size
         _f32,  # scale
         _c_void_p, _i64, _i64, _i32,  # out, strides b/h, out dtype
         _c_void_p, _i64, _i32,  # workspace, bytes, partition_tokens
         _i32, _c_void_p],  # dtype, stream
    ),
    "mie_paged_decode_append": (
        _i32,
        [_c_void_p, _i64, _i64,  # q, strides b/h
         _c_void_p, _c_void_p, _i64, _i64, _i32,  # pools, strides, num_blocks
         _c_void_p, _i64,  # block tables, stride
         _c_void_p, _c_void_p, _i32, _i32,  # ctx_lens (device), ctx_lens (host), ctx_len, max_ctx_len
         _i32, _i32, _i32, _i32,  # batch, heads, head_dim, block_size
         _f32,  # scale
         _c_void_p, _i64, _i64, _i32,  # out, strides b/h, out dtype
         _c_void_p, _i64, _i32,  # workspace, bytes, partition_tokens
         _c_void_p, _c_void_p, _i64, _i64,  # new K/V rows, strides b/h
         _i32, _c_void_p],  # dtype, stream
    ),
    "mie_paged_decode_noalloc": (
        _i32,
        [_c_void_p, _i64, _i64,  # q, strides b/h
         _c_void_p, _c_void_p, _i64, _i64, _i32,  # pools, strides, num_blocks
         _c_void_p, _i64,  # block tables, stride
         _c_void_p, _c_void_p, _i32, _i32,  # ctx_lens (device), ctx_lens (host), ctx_len, max_ctx_len
         _i32, _i32, _i32, _i32,  # batch, heads, head_dim, block_size
         _f32,  # scale
         _c_void_p, _i64, _i64, _i32,  # out, strides b/h, out dtype
         _i32,  # partition_tokens
         _i32, _c_void_p],  # dtype, stream
    ),
    "mie_paged_decode_plan": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i64)],
    ),
    "mie_paged_decode_supported": (_i32, [_i32, _i32]),
    "mie_qkv_append": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _f32,  # x, norm weight, norm bias, eps
         _c_void_p, _c_void_p, _i32,  # w_in, b_in, dim
         _c_void_p, _c_void_p, _i64, _i64, _i32,  # pools, strides, num_blocks
         _c_void_p, _i32, _c_void_p, _i32,  # block table, its length, position (device), position
         _c_void_p, _i32, _i32, _i32, _i32, _c_void_p],  # q_out, heads, head_dim, block_size, dtype, stream
    ),
    "mie_qkv_append_supported": (_i32, [_i32, _i32]),
    "mie_linear_residual": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # x, weight, bias, residual, out
         _i32, _i32, _i32, _c_void_p],  # rows, cols, dtype, stream
    ),
    "mie_moe_route": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i32, _i32,  # x, router weight, experts, top_k, dim
         _c_void_p, _c_void_p, _c_void_p, _i32, _c_void_p],  # logits, ids, weights, dtype, stream
    ),
    "mie_moe_decode": (
        _i32,
        [_c_void_p, _c_void_p,  # x, router weight
         _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # canonical w1, b1, w2, b2 storages
         _i32, _i32, _i32, _i32,  # experts, top_k, dim, hidden
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # logits, ids, weights, hidden, out
         _i32, _c_void_p],  # dtype, stream
    ),
    "mie_argmax": (_i32, [_c_void_p, _i64, _c_void_p, _i32, _c_void_p]),  # x, n, out (int64), dtype, stream
    "mie_embed": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i32,  # token ids (int64), positions (int32, device), position, n
         _c_void_p, _i32, _c_void_p, _i32, _i32,  # token table, vocab, position table, max positions, dim
         _c_void_p, _i32, _c_void_p],  # out, dtype, stream
    ),
    "mie_lm_head_workspace": (_i64, [_i32]),
    "mie_argmax_pairs": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p]),  # workspace, bytes, vocab, out, stream
    "mie_block_plan_bytes": (_i64, []),
    "mie_block_plan_init": (
        _i32,
        [_c_void_p, _i64, _i32, _i32, _i32, _i32, _i32,  # plan, its bytes, dim, heads, head_dim, block_size, dtype
         _c_void_p, _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # attn norm, eps, in/out proj
         _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _i32, _f32,  # pools, strides, blocks, table, len, scale
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,  # q, attn, h rows, workspace, its bytes
         _c_void_p, _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # moe norm, router, experts
         _i32, _i32, _i32,  # experts, top_k, hidden
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # router logits, ids, weights, hidden, out
         _c_void_p],  # accumulator (int64 [dim + 1]) or NULL
    ),
    "mie_block_decode": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i32, _c_void_p]),  # plan, x, counters, pos, stream
    "mie_block_plan_launches": (_i32, [_c_void_p, _i32]),  # plan, position
    "mie_block_plan_set_embedding": (
        _i32, [_c_void_p, _c_void_p, _i32, _c_void_p, _i32, _c_void_p]),  # plan, tables, vocab, max positions, x_out
    "mie_blocks_decode": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _i32, _c_void_p]),  # plans, n, token id, counters, position, stream
    "mie_block_decode_embed": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i32, _c_void_p]),  # plan, token id, ...
    "mie_attn_out_acc": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32,  # q, pools, strides, num_blocks
         _c_void_p, _i32, _c_void_p, _i32, _i32,  # block table, length, ctx (device), ctx, max_ctx
         _i32, _i32, _i32, _f32,  # heads, head_dim, block_size, scale
         _c_void_p, _c_void_p, _i32, _c_void_p],  # W_out, accumulator, dtype, stream
    ),
    "mie_moe_decode_block_acc": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p,  # x, accumulator, out_proj bias, h_out
         _c_void_p, _c_void_p, _f32,  # norm weight, norm bias, eps
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # router, canonical w1, b1, w2, b2
         _i32, _i32, _i32, _i32,  # experts, top_k, dim, hidden
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # logits, ids, weights, hidden, out
         _i32, _c_void_p],  # dtype, stream
    ),
    "mie_lm_head": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _f32, _c_void_p, _c_void_p,  # x, norm weight, norm bias, eps, W, bias
         _i32, _i32, _c_void_p, _c_void_p, _c_void_p, _i64,  # vocab, dim, logits, token, workspace, its bytes
         _c_void_p, _i32, _i32, _c_void_p],  # counters to advance (int32), their count, dtype, stream
    ),
    "mie_moe_decode_block": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _f32,  # x, norm weight, norm bias, eps
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # router, canonical w1, b1, w2, b2
         _i32, _i32, _i32, _i32,  # experts, top_k, dim, hidden
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # logits, ids, weights, hidden, out
         _i32, _c_void_p],  # dtype, stream
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def _open():
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.mie_abi_version()
    if version != ABI_VERSION:
        raise OSError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}")
    return lib


try:
    _LIB = _open()
    _LOAD_ERROR = None
except OSError as exc:  # reported by lib(); there is no substitute implementation
    _LIB = None
    _LOAD_ERROR = exc

HAS_HIP = _LIB is not None


def lib():
    """The loaded library; raises when it is missing or unloadable."""
    if _LIB is None:
        raise RuntimeError(
            f"the HIP paged-KV library {LIB_PATH} is not loaded ({_LOAD_ERROR}); "
            "build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "from the repository root"
        )
    return _LIB


def check(status: int, what: str) -> None:
    if status != 0:
        message = lib().mie_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed with status {status}: {message}")


def is_rocm_device(t: torch.Tensor) -> bool:
    """True for tensors on a ROCm GPU (torch names the device type 'cuda')."""
    return t.is_cuda and torch.version.hip is not None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of the current torch stream on `t`'s device."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"dtype {dtype} has no HIP paged-KV kernel") from None


@lru_cache(maxsize=256)
def decode_supported(head_dim: int, dtype: torch.dtype) -> bool:
    if _LIB is None or dtype not in DECODE_DTYPES:
        return False
    return bool(_LIB.mie_paged_decode_supported(head_dim, DTYPE_CODES[dtype]))


@lru_cache(maxsize=1024)
def decode_plan(batch, num_heads, head_dim, block_size, max_ctx_len, dtype, partition_tokens):
    """(partition_tokens, workspace_bytes) the decode launch will use."""
    part = _i32(0)
    ws = _i64(0)
    check(
        lib().mie_paged_decode_plan(
            batch, num_heads, head_dim, block_size, max_ctx_len, dtype_code(dtype), partition_tokens,
            ctypes.byref(part), ctypes.byref(ws),
        ),
        "mie_paged_decode_plan",
    )
    return part.value, ws.value
