"""Oracle-side helpers for the GPU tests.

Workloads come from moe_engine.workloads (ATen-built pools, never the kernels
under test); expected attention comes from oracle.paged_ref on the CPU.
"""

import math

import numpy as np
import torch

from moe_engine.workloads import (  # noqa: F401  (re-exported for the tests)
    Workload,
    cfg4_lens,
    make_workload,
    scatter_tokens,
    sequence_kv,
    take_last_tokens,
)
from oracle import paged_ref as ref


def oracle_outputs(w: Workload, batches=None):
    """float64 attention per sequence from the oracle: [B, H, D] numpy."""
    out = []
    for b in range(len(w.lens)) if batches is None else batches:
        k, v = sequence_kv(w, b)
        out.append(ref.attention_fp64(ref.to_f64(w.q[b]), ref.to_f64(k), ref.to_f64(v)))
    return np.stack(out)


def oracle_scales(w: Workload, batches=None):
    """The scale of each output element, sum_t p_t |v_t| (the attention of
    |v| in float64): what float32 rounding of the weighted sum is relative to.
    It bounds |output| and does not shrink when the sum cancels."""
    out = []
    for b in range(len(w.lens)) if batches is None else batches:
        k, v = sequence_kv(w, b)
        out.append(ref.attention_fp64(ref.to_f64(w.q[b]), ref.to_f64(k), np.abs(ref.to_f64(v))))
    return np.stack(out)


def bf16_close(got, want, atol=2e-3):
    """bf16 outputs: |got - want| <= atol + 2^-8 |want| (one bf16 rounding of a
    value near |want| may add up to 2^-9 |want|; twice that is allowed)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return bool(np.all(np.abs(got - want) <= atol + math.ldexp(1.0, -8) * np.abs(want)))
