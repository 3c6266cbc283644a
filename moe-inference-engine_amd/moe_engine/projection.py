"""One-token linear layers through the HIP library (mie_linear_residual).

The attention's output projection and the block's residual add
(reference src/moe_engine/model.py:268 and :447, `x + out_proj(attn)`) as one
launch: out = residual + round(weight @ x + bias), float32 or bfloat16.
"""

import torch

from moe_engine import _native


def supported(cols: int, dtype: torch.dtype) -> bool:
    """Whether mie_linear_residual is built for this input width and dtype."""
    if not _native.HAS_HIP or dtype not in (torch.float32, torch.bfloat16):
        return False
    return bool(_native.lib().mie_qkv_append_supported(int(cols), _native.dtype_code(dtype)))


def linear_residual(x, weight, bias=None, residual=None, out=None):
    """residual + (weight @ x + bias) for one token; x holds `cols` contiguous
    values, weight is [rows, cols].  Returns out with residual's shape (or
    [rows] without a residual)."""
    if weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [rows, cols] matrix")
    rows, cols = weight.shape
    dtype, device = weight.dtype, weight.device
    if not _native.is_rocm_device(weight):
        raise RuntimeError("mie_linear_residual needs tensors on a ROCm device")
    if x.numel() != cols or not x.is_contiguous():
        raise ValueError(f"x must hold {cols} contiguous values")
    for name, t in (("bias", bias), ("residual", residual)):
        if t is not None and (t.numel() != rows or not t.is_contiguous()):
            raise ValueError(f"{name} must hold {rows} contiguous values")
    if any(t is not None and (t.dtype != dtype or t.device != device) for t in (x, bias, residual, out)):
        raise ValueError("x, bias, residual and out must match the weight's dtype and device")
    if not supported(cols, dtype):
        raise RuntimeError(f"mie_linear_residual is not built for width {cols} in {dtype}")
    if out is None:
        out = torch.empty(residual.shape if residual is not None else (rows,), dtype=dtype, device=device)
    elif out.numel() != rows or not out.is_contiguous():
        raise ValueError(f"out must hold {rows} contiguous values")
    if out.data_ptr() == x.data_ptr():
        raise ValueError("out must not alias x")
    _native.check(
        _native.lib().mie_linear_residual(
            x.data_ptr(), weight.data_ptr(), _native.ptr(bias), _native.ptr(residual), out.data_ptr(),
            rows, cols, _native.dtype_code(dtype), _native.stream_of(weight),
        ),
        "mie_linear_residual",
    )
    return out
