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
