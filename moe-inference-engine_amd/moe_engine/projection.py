"""One-token linear layers through the HIP library.

- linear_residual (mie_linear_residual): the attention's output projection and
  the block's residual add (reference src/moe_engine/model.py:269 and :495,
  `x + out_proj(attn)`) as one launch: out = residual + round(weight @ x + bias).
- lm_head (mie_lm_head): the decode step's head, final_norm + output_projection
  (model.py:564-565), optionally with generate's greedy torch.argmax (:603)
  written to a device token, in two launches.
- argmax (mie_argmax): generate's greedy torch.argmax (model.py:603) over one
  row of float32 logits, in one launch.  For the logits an lm_head call with
  keep_pick=True just wrote it merges the head's per-workgroup picks
  (mie_argmax_pairs) instead of reading the row again.

float32 or bfloat16.
"""

import threading

import torch

from moe_engine import _native

# Per host thread: the logits of its last lm_head(keep_pick=True) call, with
# the picks its workgroups left - last_pick = (logits, their version counter
# then, picks, the stream the head ran on) - and the picks' workspaces by
# (device, vocab, stream).  Holding the logits keeps their memory from being
# reused, so a tensor at their address is one of their views, and views share
# the version counter, which counts every in-place write.  Threads keep their
# own workspaces, and so does each stream, so a head queued on one thread or
# stream never overwrites picks that an argmax queued on another is about to
# merge; the picks are merged only on the stream that wrote them.
_pick_state = threading.local()


def _state():
    st = _pick_state
    if not hasattr(st, "workspaces"):
        st.last_pick = None
        st.workspaces = {}
    return st


def _kept_picks(x):
    """The workspace of picks that describe x, or None."""
    rec = _state().last_pick
    if rec is None or x.is_inference():
        return None
    logits, version, workspace, stream = rec
    if x.data_ptr() != logits.data_ptr() or x.numel() != logits.numel() or x.device != logits.device:
        return None
    if _native.stream_of(x) != stream:
        return None
    return workspace if x._version == version else None


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


def lm_head(x, norm, linear, out=None, token_out=None, workspace=None, advance=None, keep_pick=False):
    """linear(norm(x)) for one token (norm a LayerNorm or None), written to
    `out` ([vocab], allocated when None); with `token_out` (an int64 device
    tensor of one element) also the index of the largest logit, as
    torch.argmax picks it.  `workspace` (uint8, at least
    head_workspace_bytes(vocab)) holds the per-workgroup picks; it is
    allocated when None.  `advance` (a contiguous int32 device tensor, with
    token_out): every element is incremented by one after the pick, in the
    same launch.  keep_pick (without token_out): the launch leaves its picks
    in a workspace of this module's, and argmax(out) merges them while out is
    unmodified and no later keep_pick call replaced them.
    Returns out."""
    st = _state()
    weight, bias = linear.weight, linear.bias
    if weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [vocab, dim] matrix")
    vocab, dim = weight.shape
    dtype, device = weight.dtype, weight.device
    if not _native.is_rocm_device(weight):
        raise RuntimeError("mie_lm_head needs tensors on a ROCm device")
    if x.numel() != dim or not x.is_contiguous():
        raise ValueError(f"x must hold {dim} contiguous values")
    ln_w = ln_b = None
    eps = 0.0
    if norm is not None:
        ln_w, ln_b, eps = norm.weight, norm.bias, float(norm.eps)
    params = (x, bias, ln_w, ln_b, out)
    if any(t is not None and (t.dtype != dtype or t.device != device) for t in params):
        raise ValueError("x, the norm, the bias and out must match the weight's dtype and device")
    if any(t is not None and not t.is_contiguous() for t in (bias, ln_w, ln_b)):
        raise ValueError("the bias and norm parameters must be contiguous")
    if not supported(dim, dtype):
        raise RuntimeError(f"mie_lm_head is not built for width {dim} in {dtype}")
    if out is None:
        out = torch.empty(vocab, dtype=dtype, device=device)
    elif out.numel() != vocab or not out.is_contiguous():
        raise ValueError(f"out must hold {vocab} contiguous values")
    ws_ptr, ws_bytes = 0, 0
    keep_pick = keep_pick and token_out is None and not out.is_inference()
    stream = _native.stream_of(weight)
    if keep_pick:
        key = (device, vocab, stream)
        workspace = st.workspaces.get(key)
        if workspace is None:
            workspace = st.workspaces[key] = torch.empty(head_workspace_bytes(vocab), dtype=torch.uint8,
                                                         device=device)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel()
        st.last_pick = None  # the picks are overwritten from here on
    elif st.last_pick is not None and out.data_ptr() == st.last_pick[0].data_ptr():
        st.last_pick = None  # the kernel rewrites the recorded logits without counting a version
    if not keep_pick and token_out is not None:
        if token_out.dtype != torch.int64 or token_out.numel() != 1 or token_out.device != device:
            raise ValueError("token_out must be one int64 value on the weight's device")
        need = head_workspace_bytes(vocab)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=device)
        elif workspace.numel() * workspace.element_size() < need or workspace.device != device:
            raise ValueError(f"workspace must hold {need} bytes on the weight's device")
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    if advance is not None:
        if token_out is None:
            raise ValueError("advance needs token_out")
        if advance.dtype != torch.int32 or not advance.is_contiguous() or advance.device != device \
                or not 0 < advance.numel() <= 64:
            raise ValueError("advance must be 1 to 64 contiguous int32 values on the weight's device")
    _native.check(
        _native.lib().mie_lm_head(
            x.data_ptr(), _native.ptr(ln_w), _native.ptr(ln_b), eps, weight.data_ptr(), _native.ptr(bias),
            vocab, dim, out.data_ptr(), _native.ptr(token_out), ws_ptr, ws_bytes,
            _native.ptr(advance), 0 if advance is None else advance.numel(),
            _native.dtype_code(dtype), stream,
        ),
        "mie_lm_head",
    )
    if keep_pick:
        st.last_pick = (out, out._version, workspace, stream)
    return out


def can_argmax(x) -> bool:
    """Whether argmax(x) applies: a contiguous float32 vector on a ROCm
    device, or the unmodified output of the last lm_head(keep_pick=True) in
    either dtype."""
    if not (_native.is_rocm_device(x) and x.is_contiguous()) or x.numel() == 0:
        return False
    return x.dtype == torch.float32 or _kept_picks(x) is not None


def argmax(x, out=None):
    """torch.argmax of the contiguous device vector x (the first index of the
    maximum, NaN counting as the largest), written to `out` (an int64 device
    tensor of one element, allocated when None): a merge of the head's kept
    picks when x is the unmodified output of the last lm_head(keep_pick=True)
    (float32 or bfloat16), else one pass over x (float32).  Returns out."""
    if not can_argmax(x):
        raise ValueError("mie_argmax takes a non-empty contiguous float32 vector on a ROCm device, or the "
                         "unmodified logits of the last lm_head(keep_pick=True)")
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=x.device)
    elif out.dtype != torch.int64 or out.numel() != 1 or out.device != x.device:
        raise ValueError("out must be one int64 value on x's device")
    picks = _kept_picks(x)
    if picks is not None:
        _native.check(
            _native.lib().mie_argmax_pairs(picks.data_ptr(), picks.numel(), x.numel(), out.data_ptr(),
                                           _native.stream_of(x)),
            "mie_argmax_pairs",
        )
        return out
    _native.check(
        _native.lib().mie_argmax(x.data_ptr(), x.numel(), out.data_ptr(), _native.dtype_code(x.dtype),
                                 _native.stream_of(x)),
        "mie_argmax",
    )
    return out


def head_workspace_bytes(vocab: int) -> int:
    """Bytes of the per-workgroup picks mie_lm_head needs for a greedy token."""
    return int(_native.lib().mie_lm_head_workspace(int(vocab)))
