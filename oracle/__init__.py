"""CPU oracle for the paged-KV decode path.  TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (and torch CPU for the library routine), of what the
reference engine computes on this path (maokner/moe-inference-engine,
src/moe_engine/model.py and src/moe_engine/paged_attention.py).  Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg may import it, and
only as the checker: the engine never calls it.

Pinning (tests/test_oracle.py), per function:
  append_rows / gather_rows  round trip against contiguous storage, untouched
                             elements unchanged, the reference Triton kernel's
                             flat-offset formula, brute force on tiny pools,
                             planted-mistake variants rejected
  attention_fp64             known answers (one key, equal keys, zero query,
                             two keys by hand), torch SDPA in float64,
                             planted-mistake variants rejected
  split_attention_fp64       equals attention_fp64 for every partition size
  gather_sdpa                equals attention_fp64 on the same inputs
  LifoAllocator / reserve    the reference tests' allocation order,
                             exhaustion message and rollback
No function here is "parity unpinned".
"""
