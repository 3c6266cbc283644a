"""Token plus positional embedding through the HIP library (mie_embed).

The reference's `token_embedding(token_ids) + positional_embedding(pos)`
(src/moe_engine/model.py:558) as one launch.  The positions are consecutive
from a host int (eager forward) or read from device memory (the captured
decode step keeps its position on the device).
"""

import torch

from moe_engine import _native


def supported(token_embedding, positional_embedding) -> bool:
    """Both tables contiguous, float32 or bfloat16, on one ROCm device."""
    tok, pos = token_embedding.weight, positional_embedding.weight
    return (_native.is_rocm_device(tok) and tok.dtype in _native.DECODE_DTYPES and pos.dtype == tok.dtype
            and pos.device == tok.device and tok.shape[1] == pos.shape[1] and tok.is_contiguous()
            and pos.is_contiguous())


def embed(token_ids, positions, token_embedding, positional_embedding, out=None):
    """token_embedding(token_ids) + positional_embedding(positions) for the
    [batch, seq] int64 `token_ids`; `positions` is an int32 device tensor of
    batch * seq values (one per token), or, for one sequence (batch 1), a
    host int p for the positions p, p + 1, ... of its tokens.  Returns [batch, seq, dim] in the
    tables' dtype, bit-identical to the PyTorch sum.  Ids or positions outside
    their tables give rows of NaN."""
    tok, pos = token_embedding.weight, positional_embedding.weight
    dtype, device = tok.dtype, tok.device
    if not _native.is_rocm_device(tok):
        raise RuntimeError("mie_embed needs tensors on a ROCm device")
    if pos.dtype != dtype or pos.device != device or tok.shape[1] != pos.shape[1]:
        raise ValueError("the two tables must share dtype, device and width")
    if not (tok.is_contiguous() and pos.is_contiguous()):
        raise ValueError("the tables must be contiguous")
    if token_ids.dtype != torch.int64 or not token_ids.is_contiguous() or token_ids.device != device:
        raise ValueError("token_ids must be a contiguous int64 tensor on the tables' device")
    n = token_ids.numel()
    if isinstance(positions, int):
        if positions < 0 or (token_ids.dim() > 1 and token_ids.shape[0] != 1):
            raise ValueError("a host start position serves one sequence from a position >= 0")
        pos_ptr, first = None, positions
    elif positions.dtype != torch.int32 or positions.numel() != n or not positions.is_contiguous() \
            or positions.device != device:
        raise ValueError(f"positions must hold {n} contiguous int32 values on the tables' device")
    else:
        pos_ptr, first = positions.data_ptr(), 0
    dim = tok.shape[1]
    if out is None:
        out = torch.empty(*token_ids.shape, dim, dtype=dtype, device=device)
    elif out.numel() != n * dim or not out.is_contiguous() or out.dtype != dtype:
        raise ValueError(f"out must hold {n} x {dim} contiguous values of the tables' dtype")
    _native.check(
        _native.lib().mie_embed(
            token_ids.data_ptr(), pos_ptr, first, n, tok.data_ptr(), tok.shape[0], pos.data_ptr(),
            pos.shape[0], dim, out.data_ptr(), _native.dtype_code(dtype), _native.stream_of(tok),
        ),
        "mie_embed",
    )
    return out
