"""Fused batch-one MoE decode on MI355X through hand-written HIP kernels.

Drop-in for the reference's src/moe_engine/fused_moe.py: the same functions
(`is_configuration_supported`, `is_supported`, `has_canonical_layout`, `route`,
`decode`) with the same arguments, workspaces and errors, plus an availability
flag.  Instead of three Triton programs it calls mie_moe_route / mie_moe_decode
(include/mie_paged_kv.h); the decode is two launches, the first routing in
every workgroup.

The reference fixes one shape (hidden 768, 8 experts, top-2, expert hidden
3072; fused_moe.py:27-53).  These kernels take the shape as arguments: up to
64 experts, top-k up to 8, hidden size up to 2048, hidden and expert-hidden
sizes multiples of 4 - which includes the reference's shape and the miniMoE
FFN-2048 variant.  `decode_block` is the block's x + MoE(moe_norm(x)) in the
same two launches.

Semantics (fused_moe.py:119-262, model.py:443-461):
  router_logits = router_weight @ x
  expert_ids    = top-k experts, largest logit first (lower id on ties)
  route_weights = softmax of the selected logits, same order
  hidden[s]     = GELU(W1[ids[s]] x + b1[ids[s]])   (exact erf GELU)
  out           = sum over slots in increasing expert id of
                  route_weights[s] * (W2[ids[s]] hidden[s] + b2[ids[s]])
The reference's Triton kernel sums the slots in route order; here they are
summed in expert-id order with each product rounded, as the PyTorch path's
index_add_ loop does, so the two paths differ only in their dot products.

The reference's kernels are float32 only.  These also take bfloat16 weights
and activations: the routing stays float32 (its logits and weights
workspaces are float32 for either dtype), every sum runs in float32, and each
bfloat16 value is rounded where the PyTorch path stores one (each Linear's
output, GELU's, the route weight, the weighted product, each partial sum).
"""

import torch

from moe_engine import _native

HAS_HIP = _native.HAS_HIP
MAX_EXPERTS = 64
MAX_TOP_K = 8
MAX_HIDDEN_DIM = 2048  # the W1 kernel holds x in 8 loads per lane
DTYPES = (torch.float32, torch.bfloat16)


def is_configuration_supported(
    *,
    device: torch.device,
    dtype: torch.dtype,
    batch_size: int,
    hidden_dim: int,
    num_experts: int,
    top_k: int,
    expert_hidden_dim: int,
) -> bool:
    """Whether model metadata can use the direct decode kernels
    (reference fused_moe.py:33-53)."""
    return (
        HAS_HIP
        and torch.device(device).type == "cuda"
        and torch.version.hip is not None
        and dtype in DTYPES
        and batch_size == 1
        and 0 < num_experts <= MAX_EXPERTS
        and 0 < top_k <= min(MAX_TOP_K, num_experts)
        and hidden_dim > 0
        and hidden_dim % 4 == 0
        and expert_hidden_dim > 0
        and expert_hidden_dim % 4 == 0
        and hidden_dim <= MAX_HIDDEN_DIM
    )


def is_supported(x: torch.Tensor, *, num_experts: int, top_k: int, expert_hidden_dim: int) -> bool:
    """Whether `x` [1, 1, hidden] and the model shape can use the direct
    kernels (reference fused_moe.py:56-74)."""
    if x.dim() != 3 or x.shape[:2] != (1, 1) or not x.is_contiguous():
        return False
    return is_configuration_supported(
        device=x.device,
        dtype=x.dtype,
        batch_size=x.shape[0],
        hidden_dim=x.shape[-1],
        num_experts=num_experts,
        top_k=top_k,
        expert_hidden_dim=expert_hidden_dim,
    )


def has_canonical_layout(router_weight, w1, b1, w2, b2, router_logits, expert_ids, route_weights, hidden, out) -> bool:
    """Shapes, contiguity, dtypes and device of the direct-kernel weights and
    workspaces (reference fused_moe.py:77-114), for the shape the router
    weight [E, dim] and w1 [E, expert_hidden, dim] describe: the weights and
    the hidden and output workspaces in the router weight's dtype (float32 or
    bfloat16), the routing workspaces in float32."""
    if router_weight.dim() != 2 or w1.dim() != 3:
        return False
    num_experts, dim = router_weight.shape
    expert_hidden = w1.shape[1]
    top_k = expert_ids.numel()
    dtype = router_weight.dtype
    parts = (
        (router_weight, (num_experts, dim), dtype),
        (w1, (num_experts, expert_hidden, dim), dtype),
        (b1, (num_experts, expert_hidden), dtype),
        (w2, (num_experts, dim, expert_hidden), dtype),
        (b2, (num_experts, dim), dtype),
        (router_logits, (num_experts,), torch.float32),
        (route_weights, (top_k,), torch.float32),
        (hidden, (top_k, expert_hidden), dtype),
        (out, (dim,), dtype),
    )
    device = router_weight.device
    return (
        dtype in DTYPES
        and all(
            t.shape == shape and t.is_contiguous() and t.device == device and t.dtype == want
            for t, shape, want in parts
        )
        and expert_ids.shape == (top_k,)
        and expert_ids.is_contiguous()
        and expert_ids.device == device
        and expert_ids.dtype == torch.int32
    )


def _require_rocm(tensors, routing=()) -> None:
    """Errors of the reference's _require_cuda_float32 (fused_moe.py:265-271):
    `tensors` (activations and parameters) in one dtype, float32 or bfloat16;
    `routing` (the logits and weights workspaces) in float32."""
    everything = (*tensors, *routing)
    if not HAS_HIP or any(not _native.is_rocm_device(t) for t in everything):
        raise RuntimeError("direct MoE needs a ROCm device and the HIP library")
    if tensors[0].dtype not in DTYPES or any(t.dtype != tensors[0].dtype for t in tensors[1:]):
        raise RuntimeError("direct MoE needs float32 or bfloat16 activations and parameters, all of one dtype")
    if any(t.dtype != torch.float32 for t in routing):
        raise RuntimeError("direct MoE keeps its routing logits and weights in float32")
    if any(t.device != everything[0].device for t in everything[1:]):
        raise ValueError("direct MoE tensors must be on the same ROCm device")


def route(x, router_weight, router_logits, expert_ids, route_weights) -> None:
    """Router logits, top-k expert ids and their softmax weights, written into
    the three workspaces (reference fused_moe.py:274-309)."""
    _require_rocm((x, router_weight), (router_logits, route_weights))
    if router_weight.dim() != 2 or not router_weight.is_contiguous():
        raise ValueError("direct MoE router weight must be a contiguous [experts, hidden] matrix")
    num_experts, dim = router_weight.shape
    if x.numel() != dim or not x.is_contiguous():
        raise ValueError(f"direct MoE router needs a contiguous x of {dim} values")
    if (
        not _native.is_rocm_device(expert_ids)
        or expert_ids.device != x.device
        or expert_ids.dtype != torch.int32
        or expert_ids.dim() != 1
        or not expert_ids.is_contiguous()
    ):
        raise ValueError("direct MoE expert id workspace must be a contiguous ROCm int32 vector")
    top_k = expert_ids.numel()
    if router_logits.shape != (num_experts,) or route_weights.shape != (top_k,):
        raise ValueError("direct MoE router workspaces have invalid shapes")
    _native.check(
        _native.lib().mie_moe_route(
            x.data_ptr(), router_weight.data_ptr(), num_experts, top_k, dim,
            router_logits.data_ptr(), expert_ids.data_ptr(), route_weights.data_ptr(),
            _native.dtype_code(x.dtype), _native.stream_of(x),
        ),
        "mie_moe_route",
    )


def decode(x, router_weight, w1_base, b1_base, w2_base, b2_base, *, router_logits, expert_ids, route_weights,
           hidden, out) -> torch.Tensor:
    """Router, the selected W1 + GELU rows and the weighted W2 sum for one
    token; returns `out` viewed as [1, 1, hidden] (reference fused_moe.py:312-380)."""
    _require_rocm((x, router_weight, w1_base, b1_base, w2_base, b2_base, hidden, out),
                  (router_logits, route_weights))
    if not has_canonical_layout(router_weight, w1_base, b1_base, w2_base, b2_base, router_logits, expert_ids,
                                route_weights, hidden, out):
        raise ValueError("direct MoE weights and workspaces must use canonical layouts")
    num_experts, dim = router_weight.shape
    if x.numel() != dim or not x.is_contiguous():
        raise ValueError(f"direct MoE needs a contiguous x of {dim} values")
    rc = _native.lib().mie_moe_decode(
        x.data_ptr(), router_weight.data_ptr(),
        w1_base.data_ptr(), b1_base.data_ptr(), w2_base.data_ptr(), b2_base.data_ptr(),
        num_experts, expert_ids.numel(), dim, w1_base.shape[1],
        router_logits.data_ptr(), expert_ids.data_ptr(), route_weights.data_ptr(), hidden.data_ptr(),
        out.data_ptr(), _native.dtype_code(x.dtype), _native.stream_of(x),
    )
    if rc:
        _native.check(rc, "mie_moe_decode")
    return out.view(1, 1, dim)


def decode_block(x, norm_weight, norm_bias, norm_eps, router_weight, w1_base, b1_base, w2_base, b2_base, *,
                 router_logits, expert_ids, route_weights, hidden, out) -> torch.Tensor:
    """The MoE half of a decoder block for one token, out = x + MoE(LayerNorm(x))
    (reference model.py:494-498), in two launches; the routing workspaces are
    filled as decode() fills them.  norm_weight None skips the norm.  Returns
    `out` viewed as [1, 1, hidden]."""
    params = [t for t in (norm_weight, norm_bias) if t is not None]
    _require_rocm((x, router_weight, w1_base, b1_base, w2_base, b2_base, hidden, out, *params),
                  (router_logits, route_weights))
    if not has_canonical_layout(router_weight, w1_base, b1_base, w2_base, b2_base, router_logits, expert_ids,
                                route_weights, hidden, out):
        raise ValueError("direct MoE weights and workspaces must use canonical layouts")
    num_experts, dim = router_weight.shape
    if x.numel() != dim or not x.is_contiguous():
        raise ValueError(f"direct MoE needs a contiguous x of {dim} values")
    if norm_bias is not None and norm_weight is None:
        raise ValueError("a norm bias needs a norm weight")
    if any(t.shape != (dim,) or not t.is_contiguous() for t in params):
        raise ValueError(f"norm parameters must be contiguous [{dim}] vectors")
    rc = _native.lib().mie_moe_decode_block(
        x.data_ptr(), _native.ptr(norm_weight), _native.ptr(norm_bias), float(norm_eps),
        router_weight.data_ptr(), w1_base.data_ptr(), b1_base.data_ptr(), w2_base.data_ptr(), b2_base.data_ptr(),
        num_experts, expert_ids.numel(), dim, w1_base.shape[1],
        router_logits.data_ptr(), expert_ids.data_ptr(), route_weights.data_ptr(), hidden.data_ptr(),
        out.data_ptr(), _native.dtype_code(x.dtype), _native.stream_of(x),
    )
    if rc:
        _native.check(rc, "mie_moe_decode_block")
    return out.view(1, 1, dim)
