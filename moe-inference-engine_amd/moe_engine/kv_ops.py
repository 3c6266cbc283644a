"""Device-side KV append and gather through the HIP library.

These are the tensor operations under PagedKVCache.write / .read on a ROCm
device (reference: src/moe_engine/model.py:167-201).  Pools are the
allocator's [layers, blocks, heads, block_size, head_dim] tensors; the kernels
address one layer through `layer_idx`, the same view the reference takes with
k_pool[layer] (src/moe_engine/paged_attention.py:121-122).
"""

import torch

from moe_engine import _native


def _check_pools(k_pool: torch.Tensor, v_pool: torch.Tensor) -> None:
    if k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype:
        raise ValueError("K and V pools must share shape and dtype")
    if k_pool.dim() != 5:
        raise ValueError("pools are [layers, blocks, heads, block_size, head_dim]")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if not _native.is_rocm_device(k_pool):
        raise RuntimeError("the HIP KV kernels need pools on a ROCm device")


def _layer(pool: torch.Tensor, layer_idx: int) -> torch.Tensor:
    if not 0 <= layer_idx < pool.shape[0]:
        raise IndexError(f"layer {layer_idx} outside [0, {pool.shape[0]})")
    return pool[layer_idx]


def append(
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    layer_idx: int,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    block_tables: torch.Tensor,
    position: int = 0,
    positions: torch.Tensor = None,
) -> None:
    """Scatter new rows k_new/v_new [B, H, S, D] into one layer of the pools.

    Row (b, s) lands at logical position pos_b + s of sequence b, where pos_b is
    positions[b] (device int32 [B]) or `position`.  block_tables is an int32
    device tensor [B, max_blocks] (or the 1-D per-sequence mirror for B == 1).
    One launch writes K and V.
    """
    _check_pools(k_pool, v_pool)
    lib = _native.lib()
    kl, vl = _layer(k_pool, layer_idx), _layer(v_pool, layer_idx)
    nb, heads, block_size, head_dim = kl.shape
    if k_new.dim() != 4 or k_new.shape != v_new.shape:
        raise ValueError("k_new and v_new must both be [batch, heads, seq, head_dim]")
    batch, h2, seq_len, d2 = k_new.shape
    if (h2, d2) != (heads, head_dim):
        raise ValueError(f"new rows have heads/head_dim {h2}/{d2}, pool has {heads}/{head_dim}")
    if k_new.dtype != kl.dtype or v_new.dtype != kl.dtype:
        raise ValueError(f"new rows are {k_new.dtype}, pool is {kl.dtype}")
    if k_new.device != kl.device or v_new.device != kl.device:
        raise ValueError("new rows and pools must be on the same device")
    if k_new.stride() != v_new.stride() or k_new.stride(3) != 1:
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    if block_tables.dtype != torch.int32 or block_tables.device != kl.device:
        raise ValueError("block tables must be int32 on the pool's device")
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
    if positions is not None:
        if positions.dtype != torch.int32 or positions.shape != (batch,) or positions.device != kl.device:
            raise ValueError("positions must be an int32 device tensor [batch]")
        positions = positions.contiguous()
    _native.check(
        lib.mie_kv_append(
            kl.data_ptr(), vl.data_ptr(), kl.stride(0), kl.stride(1), nb,
            k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_new.stride(2),
            block_tables.data_ptr(), bt_stride,
            _native.ptr(positions), int(position),
            batch, seq_len, heads, head_dim, block_size,
            _native.dtype_code(kl.dtype), _native.stream_of(kl),
        ),
        "mie_kv_append",
    )


def gather(
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    layer_idx: int,
    block_table: torch.Tensor,
    length: int,
    out_k: torch.Tensor = None,
    out_v: torch.Tensor = None,
):
    """Copy tokens [0, length) of one sequence to contiguous K, V [1, H, length, D].

    Same result as the reference's pool[l, bt[:nb]].transpose(0, 1).reshape(...)
    (src/moe_engine/model.py:191-199), produced by one launch for K and V.
    """
    _check_pools(k_pool, v_pool)
    lib = _native.lib()
    kl, vl = _layer(k_pool, layer_idx), _layer(v_pool, layer_idx)
    nb, heads, block_size, head_dim = kl.shape
    if length < 0 or length > nb * block_size:
        raise ValueError(f"length {length} outside [0, {nb * block_size}]")
    if block_table.dtype != torch.int32 or block_table.dim() != 1 or block_table.device != kl.device:
        raise ValueError("block_table must be a 1-D int32 tensor on the pool's device")
    if not block_table.is_contiguous() or block_table.numel() < -(-length // block_size):
        raise ValueError("block_table must be contiguous and cover the gathered length")
    shape = (1, heads, length, head_dim)
    if out_k is None:
        out_k = torch.empty(shape, dtype=kl.dtype, device=kl.device)
    if out_v is None:
        out_v = torch.empty(shape, dtype=kl.dtype, device=kl.device)
    for out in (out_k, out_v):
        if out.shape != shape or out.dtype != kl.dtype or out.stride(3) != 1:
            raise ValueError(f"gather outputs must be {shape} {kl.dtype} with unit inner stride")
    if out_k.stride() != out_v.stride():
        raise ValueError("gather outputs must share strides")
    _native.check(
        lib.mie_kv_gather(
            kl.data_ptr(), vl.data_ptr(), kl.stride(0), kl.stride(1), nb,
            block_table.data_ptr(), length,
            out_k.data_ptr(), out_v.data_ptr(), out_k.stride(1), out_k.stride(2),
            heads, head_dim, block_size,
            _native.dtype_code(kl.dtype), _native.stream_of(kl),
        ),
        "mie_kv_gather",
    )
    return out_k, out_v


def qkv_append_supported(dim: int, dtype: torch.dtype) -> bool:
    """Whether mie_qkv_append is built for this model width and dtype."""
    if not _native.HAS_HIP or dtype not in (torch.float32, torch.bfloat16):
        return False
    return bool(_native.lib().mie_qkv_append_supported(int(dim), _native.dtype_code(dtype)))


def qkv_append(
    x: torch.Tensor,
    in_proj_weight: torch.Tensor,
    in_proj_bias: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    layer_idx: int,
    block_table: torch.Tensor,
    *,
    position: int = 0,
    position_dev: torch.Tensor = None,
    norm_weight: torch.Tensor = None,
    norm_bias: torch.Tensor = None,
    norm_eps: float = 1e-5,
    q_out: torch.Tensor = None,
) -> torch.Tensor:
    """QKV projection of one token with K and V stored into their pool slots.

    x holds one token's dim values (any shape of dim elements, contiguous);
    in_proj_weight [3*dim, dim] and in_proj_bias [3*dim] are the attention's
    packed projection (reference model.py:218-224); block_table is the
    sequence's 1-D int32 device table.  The token goes to logical position
    `position`, or to *position_dev (an int32 device [1]) when given.  With
    norm_weight the projection applies to LayerNorm(x) (the block's attn_norm).
    Returns q [1, heads, 1, head_dim] (written into q_out when given); the
    block for the position must already be reserved.
    """
    _check_pools(k_pool, v_pool)
    kl, vl = _layer(k_pool, layer_idx), _layer(v_pool, layer_idx)
    nb, heads, block_size, head_dim = kl.shape
    dim = heads * head_dim
    dtype = kl.dtype
    if x.numel() != dim or not x.is_contiguous():
        raise ValueError(f"x must hold {dim} contiguous values")
    if in_proj_weight.shape != (3 * dim, dim) or not in_proj_weight.is_contiguous():
        raise ValueError(f"in_proj_weight must be a contiguous [{3 * dim}, {dim}] matrix")
    if in_proj_bias is not None and (in_proj_bias.shape != (3 * dim,) or not in_proj_bias.is_contiguous()):
        raise ValueError(f"in_proj_bias must be a contiguous [{3 * dim}] vector")
    norm = [t for t in (norm_weight, norm_bias) if t is not None]
    if norm_bias is not None and norm_weight is None:
        raise ValueError("a norm bias needs a norm weight")
    for t in norm:
        if t.shape != (dim,) or not t.is_contiguous():
            raise ValueError(f"norm parameters must be contiguous [{dim}] vectors")
    params = [x, in_proj_weight, *([in_proj_bias] if in_proj_bias is not None else []), *norm]
    if any(t.dtype != dtype or t.device != kl.device for t in params):
        raise ValueError("x, the projection and norm parameters must match the pools' dtype and device")
    if not qkv_append_supported(dim, dtype):
        raise RuntimeError(f"mie_qkv_append is not built for dim {dim} in {dtype}")
    if block_table.dtype != torch.int32 or block_table.dim() != 1 or block_table.device != kl.device:
        raise ValueError("block_table must be a 1-D int32 tensor on the pool's device")
    if not block_table.is_contiguous():
        raise ValueError("block_table must be contiguous")
    if position_dev is not None:
        if position_dev.dtype != torch.int32 or position_dev.numel() != 1 or position_dev.device != kl.device:
            raise ValueError("position_dev must be an int32 device tensor of one element")
    elif not 0 <= position < block_table.numel() * block_size:
        raise ValueError(f"position {position} outside the block table's {block_table.numel() * block_size} slots")
    if q_out is None:
        q_out = torch.empty((1, heads, 1, head_dim), dtype=dtype, device=kl.device)
    elif q_out.numel() != dim or not q_out.is_contiguous() or q_out.dtype != dtype:
        raise ValueError(f"q_out must hold {dim} contiguous {dtype} values")
    _native.check(
        _native.lib().mie_qkv_append(
            x.data_ptr(), _native.ptr(norm_weight), _native.ptr(norm_bias), float(norm_eps),
            in_proj_weight.data_ptr(), _native.ptr(in_proj_bias), dim,
            kl.data_ptr(), vl.data_ptr(), kl.stride(0), kl.stride(1), nb,
            block_table.data_ptr(), block_table.numel(), _native.ptr(position_dev), int(position),
            q_out.data_ptr(), heads, head_dim, block_size,
            _native.dtype_code(dtype), _native.stream_of(kl),
        ),
        "mie_qkv_append",
    )
    return q_out.view(1, heads, 1, head_dim)
