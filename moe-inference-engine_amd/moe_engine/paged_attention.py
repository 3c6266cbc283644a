"""Direct paged decode attention on MI355X through hand-written HIP kernels.

Drop-in for the reference's src/moe_engine/paged_attention.py: the same
`is_supported(x)` / `decode(q, cache, layer_idx, context_len)` surface plus an
availability flag.  Instead of a Triton program per head it calls
mie_paged_decode (include/mie_paged_kv.h), which reads K/V in place from the
block pool through the block table:

    logical block  = p // block_size
    block offset   = p %  block_size
    physical block = block_table[logical block]

and, for long contexts, splits each sequence into partitions whose partial
softmax states are merged by a second launch.  `decode_batched` is the same
kernel for many sequences in one launch.

context_len is a host int, as in the reference (paged_attention.py:116-118):
the single-sequence path never reads a device value.
"""

import ctypes
import math

import torch

from moe_engine import _native

HAS_HIP = _native.HAS_HIP
SUPPORTED_DTYPES = _native.DECODE_DTYPES


def is_supported(x: torch.Tensor, head_dim: int = None) -> bool:
    """The kernel path needs a ROCm device, the HIP library and f32/bf16 inputs.

    `head_dim`, when given, must be one the library is built for; the
    reference's check (paged_attention.py:39-41) has no such argument because
    its Triton kernel pads any head_dim.
    """
    if not (HAS_HIP and _native.is_rocm_device(x) and x.dtype in SUPPORTED_DTYPES):
        return False
    return head_dim is None or _native.decode_supported(head_dim, x.dtype)


def _workspace(nbytes: int, device) -> torch.Tensor:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def decode_layer(
    q: torch.Tensor,
    k_layer: torch.Tensor,
    v_layer: torch.Tensor,
    block_tables: torch.Tensor,
    *,
    context_len: int = None,
    context_lens: torch.Tensor = None,
    max_context_len: int = None,
    scale: float = None,
    out: torch.Tensor = None,
    out_dtype: torch.dtype = None,
    partition_tokens: int = 0,
    context_lens_host=None,
    k_new: torch.Tensor = None,
    v_new: torch.Tensor = None,
) -> torch.Tensor:
    """Decode attention for q [B, H, D] over one layer's pools [NB, H, BS, D].

    Either `context_len` (one host int for every sequence) or `context_lens`
    (int32 device [B]) with `max_context_len` (a host upper bound that sizes the
    launch).  `context_lens_host`, a host sequence of the same lengths, lets
    the launch hold exactly the batch's work items (no idle workgroups on
    ragged batches).  block_tables is int32 [B, max_blocks], or 1-D when B == 1.
    Returns out [B, H, D] in `out_dtype` (q's dtype or float32).

    With k_new / v_new ([B, H, D], the pools' dtype) the step's append is
    fused in: each sequence's new token is its last context token, stored at
    position ctx_b - 1 through the table and attended to (mie_paged_decode_append;
    one launch when the plan takes the workgroup form).
    """
    lib = _native.lib()
    if q.dim() != 3:
        raise ValueError("q must be [batch, heads, head_dim]")
    batch, heads, head_dim = q.shape
    if k_layer.shape != v_layer.shape or k_layer.dim() != 4:
        raise ValueError("layer pools must both be [blocks, heads, block_size, head_dim]")
    nb, h2, block_size, d2 = k_layer.shape
    if (h2, d2) != (heads, head_dim):
        raise ValueError(f"q has heads/head_dim {heads}/{head_dim}, pool has {h2}/{d2}")
    if q.dtype != k_layer.dtype or v_layer.dtype != k_layer.dtype:
        raise ValueError("q and the pools must share a dtype")
    if not (_native.is_rocm_device(q) and q.device == k_layer.device == v_layer.device):
        raise RuntimeError("paged decode needs q and pools on the same ROCm device")
    if not (k_layer.stride(3) == 1 and k_layer.stride(2) == head_dim and k_layer.stride() == v_layer.stride()):
        raise ValueError("each (block, head) tile of the pools must be contiguous")
    if q.stride(2) != 1:
        q = q.contiguous()
    if block_tables.dtype != torch.int32 or block_tables.device != q.device:
        raise ValueError("block tables must be int32 on q's device")
    if block_tables.dim() == 1:
        if batch != 1:
            raise ValueError("a 1-D block table serves one sequence")
        if block_tables.numel() < nb or not block_tables.is_contiguous():
            raise ValueError("a 1-D block table must be contiguous with one entry per pool block")
        bt_stride = 0
    else:
        if block_tables.shape[0] != batch or block_tables.stride(1) != 1:
            raise ValueError("block tables must be [batch, max_blocks] with unit inner stride")
        bt_stride = block_tables.stride(0)
    host_lens = None
    if context_lens is None:
        if context_len is None:
            raise ValueError("pass context_len or context_lens")
        max_context_len = int(context_len)
        ctx_ptr = 0
    else:
        if max_context_len is None:
            raise ValueError("context_lens needs a host max_context_len")
        if context_lens.dtype != torch.int32 or context_lens.shape != (batch,) or context_lens.device != q.device:
            raise ValueError("context_lens must be an int32 device tensor [batch]")
        context_lens = context_lens.contiguous()
        ctx_ptr = context_lens.data_ptr()
        context_len = 0
        if context_lens_host is not None:
            if len(context_lens_host) != batch:
                raise ValueError("context_lens_host must hold one length per sequence")
            host_lens = (ctypes.c_int32 * batch)(*(int(c) for c in context_lens_host))
    if out_dtype is None:
        out_dtype = q.dtype if out is None else out.dtype
    if out is None:
        out = torch.empty((batch, heads, head_dim), dtype=out_dtype, device=q.device)
    elif out.shape != (batch, heads, head_dim) or out.dtype != out_dtype or out.stride(2) != 1:
        raise ValueError("out must be [batch, heads, head_dim] with unit inner stride")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    _, ws_bytes = _native.decode_plan(
        batch, heads, head_dim, block_size, int(max_context_len), q.dtype, int(partition_tokens)
    )
    ws = _workspace(ws_bytes, q.device)
    if k_new is not None or v_new is not None:
        if k_new is None or v_new is None:
            raise ValueError("pass both k_new and v_new")
        for t in (k_new, v_new):
            if t.shape != (batch, heads, head_dim) or t.dtype != k_layer.dtype or t.device != q.device:
                raise ValueError(f"new rows must be [{batch}, {heads}, {head_dim}] {k_layer.dtype} on q's device")
        if k_new.stride() != v_new.stride() or k_new.stride(2) != 1:
            k_new, v_new = k_new.contiguous(), v_new.contiguous()
        _native.check(
            lib.mie_paged_decode_append(
                q.data_ptr(), q.stride(0), q.stride(1),
                k_layer.data_ptr(), v_layer.data_ptr(), k_layer.stride(0), k_layer.stride(1), nb,
                block_tables.data_ptr(), bt_stride,
                ctx_ptr, host_lens, int(context_len), int(max_context_len),
                batch, heads, head_dim, block_size,
                float(scale),
                out.data_ptr(), out.stride(0), out.stride(1), _native.dtype_code(out.dtype),
                _native.ptr(ws), ws_bytes, int(partition_tokens),
                k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1),
                _native.dtype_code(q.dtype), _native.stream_of(q),
            ),
            "mie_paged_decode_append",
        )
        return out
    _native.check(
        lib.mie_paged_decode(
            q.data_ptr(), q.stride(0), q.stride(1),
            k_layer.data_ptr(), v_layer.data_ptr(), k_layer.stride(0), k_layer.stride(1), nb,
            block_tables.data_ptr(), bt_stride,
            ctx_ptr, host_lens, int(context_len), int(max_context_len),
            batch, heads, head_dim, block_size,
            float(scale),
            out.data_ptr(), out.stride(0), out.stride(1), _native.dtype_code(out.dtype),
            _native.ptr(ws), ws_bytes, int(partition_tokens),
            _native.dtype_code(q.dtype), _native.stream_of(q),
        ),
        "mie_paged_decode",
    )
    return out


def decode(q: torch.Tensor, cache, layer_idx: int, context_len: int) -> torch.Tensor:
    """Single-token paged attention over cached positions 0..context_len-1.

    q is [1, heads, 1, head_dim]; returns the same shape (reference
    paged_attention.py:113-154).  context_len is a host int, so this path never
    synchronizes the device to read a length.
    """
    allocator = cache.allocator
    num_heads, head_dim = q.shape[1], q.shape[3]
    graph_ctx = getattr(cache, "graph_ctx", None)
    if graph_ctx is not None:
        # HIP-graph decode: the length lives on the device and the launch is
        # sized for the pool's capacity, so one captured launch serves every step.
        out = decode_layer(
            q[:, :, 0],
            allocator.k_pool[layer_idx],
            allocator.v_pool[layer_idx],
            cache.block_table_device,
            context_lens=graph_ctx,
            max_context_len=allocator.num_blocks * allocator.block_size,
            partition_tokens=cache.graph_partition_tokens,
        )
        return out.view(1, num_heads, 1, head_dim)
    launch = getattr(allocator, "_launch", None)
    qs = q.stride()
    if (
        launch is not None
        and qs[3] == 1
        and q.dtype == allocator.k_pool.dtype
        and q.shape == (1, allocator.num_heads, 1, allocator.head_dim)
        and q.device == allocator.k_pool.device
        and 0 <= layer_idx < allocator.k_pool.shape[0]
        and 0 <= context_len <= allocator.num_blocks * allocator.block_size
    ):
        # Lean path for the engine's own calls: the launch constants are the
        # allocator's, the plan is cached, one C call.
        layer_bytes, sblk, shead, code = launch
        part, ws_bytes = _native.decode_plan(
            1, num_heads, head_dim, allocator.block_size, context_len, q.dtype, 0
        )
        out = torch.empty((1, num_heads, 1, head_dim), dtype=q.dtype, device=q.device)
        ws = _workspace(ws_bytes, q.device)
        off = layer_idx * layer_bytes
        rc = _native.lib().mie_paged_decode(
            q.data_ptr(), qs[0], qs[1],
            allocator.k_pool.data_ptr() + off, allocator.v_pool.data_ptr() + off, sblk, shead, allocator.num_blocks,
            cache.block_table_device.data_ptr(), 0,
            None, None, context_len, context_len,
            1, num_heads, head_dim, allocator.block_size,
            1.0 / math.sqrt(head_dim),
            out.data_ptr(), num_heads * head_dim, head_dim, code,
            _native.ptr(ws), ws_bytes, 0,
            code, _native.stream_of(q),
        )
        if rc:
            _native.check(rc, "mie_paged_decode")
        return out
    out = decode_layer(
        q[:, :, 0],
        allocator.k_pool[layer_idx],
        allocator.v_pool[layer_idx],
        cache.block_table_device,
        context_len=context_len,
    )
    return out.view(1, num_heads, 1, head_dim)


def decode_batched(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    layer_idx: int,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    max_context_len: int,
    **kwargs,
) -> torch.Tensor:
    """One launch of decode attention for B sequences sharing a block pool.

    q [B, H, D]; pools [L, NB, H, BS, D]; block_tables int32 [B, max_blocks];
    context_lens int32 [B] on the device; max_context_len a host bound.
    """
    return decode_layer(
        q,
        k_pool[layer_idx],
        v_pool[layer_idx],
        block_tables,
        context_lens=context_lens,
        max_context_len=max_context_len,
        **kwargs,
    )
