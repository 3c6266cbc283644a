"""mie_paged_decode_noalloc against mie_paged_decode, through the C ABI.

The allocation-free entry point keeps its split-context workspace in a device
array inside the library instead of a caller-passed buffer; its kernels are
mie_paged_decode's, so its outputs must be bit-identical.  Two calls in a row,
the second smaller (fewer partitions, another dtype), show that what the
first call left in the shared array is never read back.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from conftest import print_case
from moe_engine import _native
from oracle import paged_ref as ref
from paged_cases import bf16_close, make_workload, oracle_outputs

pytestmark = pytest.mark.gpu

MAX_SCRATCH = 16 << 20  # MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE


def _common_args(w, out):
    """The arguments both entry points share, in order, up to out_dtype."""
    kl, vl = w.k_pool[w.layer], w.v_pool[w.layer]
    batch, heads, dim = w.q.shape
    return [
        w.q.data_ptr(), w.q.stride(0), w.q.stride(1),
        kl.data_ptr(), vl.data_ptr(), kl.stride(0), kl.stride(1), kl.shape[0],
        w.block_tables.data_ptr(), w.block_tables.stride(0),
        w.context_lens.data_ptr(), (ctypes.c_int32 * batch)(*w.lens), 0, w.max_len,
        batch, heads, dim, w.block_size,
        1.0 / math.sqrt(dim),
        out.data_ptr(), out.stride(0), out.stride(1), _native.dtype_code(out.dtype),
    ]


def with_workspace(w, out_dtype):
    lib = _native.lib()
    out = torch.empty(w.q.shape, dtype=out_dtype, device="cuda")
    batch, heads, dim = w.q.shape
    _, ws_bytes = _native.decode_plan(batch, heads, dim, w.block_size, w.max_len, w.q.dtype, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    rc = lib.mie_paged_decode(*_common_args(w, out), ws.data_ptr(), ws_bytes, 0,
                              _native.dtype_code(w.q.dtype), _native.stream_of(w.q))
    _native.check(rc, "mie_paged_decode")
    return out, ws_bytes


def no_alloc(w, out_dtype):
    lib = _native.lib()
    out = torch.empty(w.q.shape, dtype=out_dtype, device="cuda")
    rc = lib.mie_paged_decode_noalloc(*_common_args(w, out), 0, _native.dtype_code(w.q.dtype),
                                      _native.stream_of(w.q))
    _native.check(rc, "mie_paged_decode_noalloc")
    return out


def test_noalloc_matches_workspace_entry_point_twice_second_smaller():
    cases = [
        # (lens, block size, dtype, output dtype): the first fills far more of
        # the scratch than the second reads.
        ([32768] * 8, 16, torch.bfloat16, torch.bfloat16),
        ([5000, 1, 0, 2600], 32, torch.float32, torch.float32),
    ]
    sizes = []
    for lens, bs, dtype, out_dtype in cases:
        print_case("noalloc", len(lens), max(lens), bs, dtype)
        w = make_workload(lens, block_size=bs, dtype=dtype, seed=31, heavy_fraction=0.01)
        want, ws_bytes = with_workspace(w, out_dtype)
        assert 0 < ws_bytes <= MAX_SCRATCH, "the case must use the split workspace"
        sizes.append(ws_bytes)
        got = no_alloc(w, out_dtype)
        torch.cuda.synchronize()
        assert np.array_equal(ref.raw_bits(got.cpu()), ref.raw_bits(want.cpu()))
        # And against the oracle, for the longest sequence.
        b = int(np.argmax(lens))
        want_b = oracle_outputs(w, [b])[0]
        if dtype == torch.float32:
            np.testing.assert_allclose(got[b].cpu().numpy(), want_b, rtol=0, atol=1e-5)
        else:
            assert bf16_close(got[b].float().cpu().numpy(), want_b)
    assert sizes[1] < sizes[0]


def test_noalloc_rejects_a_workspace_above_its_scratch():
    """64 x 131072 tokens needs ~26 MB of partials: refused before any launch."""
    _, ws = _native.decode_plan(64, 12, 64, 16, 131072, torch.bfloat16, 0)
    assert ws > MAX_SCRATCH
    lib = _native.lib()
    rc = lib.mie_paged_decode_noalloc(0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, None, 131072, 131072, 64, 12, 64, 16,
                                      0.125, 0, 0, 0, 1, 0, 1, 0)
    assert rc == 3 and b"scratch" in lib.mie_last_error()
