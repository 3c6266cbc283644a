"""The C-ABI library loads and exports every entry point include/*.h declares.

No compute call is made here (no GPU is needed): only symbol lookup, the ABI
version, the host-only planning query and argument validation that fails
before any launch.
"""

import ctypes
import re
from pathlib import Path

import pytest

from moe_engine import _native

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(mie_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_headers_declare_the_entry_points():
    assert {"mie_kv_append", "mie_kv_gather", "mie_paged_decode"} <= set(declared_functions())


def test_library_loads():
    assert _native.HAS_HIP, f"{_native.LIB_PATH} failed to load: {_native._LOAD_ERROR}"
    assert _native.lib().mie_abi_version() == _native.ABI_VERSION


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports_declared_symbol(name):
    raw = ctypes.CDLL(str(_native.LIB_PATH))
    assert hasattr(raw, name), f"{name} declared in include/ but not exported"
    assert name in _native.EXPORTED_SYMBOLS, f"{name} has no ctypes signature in moe_engine._native"


def test_decode_plan_host_query():
    import torch

    # Short contexts run as one partition and need no workspace.
    part, ws = _native.decode_plan(1, 12, 64, 16, 96, torch.bfloat16, 0)
    assert part >= 96 and ws == 0
    # Long contexts split; the workspace holds (m, l, acc[D]) per partition.
    part, ws = _native.decode_plan(8, 12, 64, 16, 131072, torch.bfloat16, 0)
    parts = -(-131072 // part)
    assert parts > 1 and ws == 8 * 12 * parts * (64 + 2) * 4
    # An explicit partition size is honoured when it is a power of two multiple of the tile.
    assert _native.decode_plan(2, 12, 64, 16, 4096, torch.float32, 1024) == (1024, 2 * 12 * 4 * 66 * 4)


def test_decode_plan_rejects_bad_partition_and_unbuilt_shapes():
    import torch

    with pytest.raises(RuntimeError, match="partition_tokens"):
        _native.decode_plan(1, 12, 64, 16, 4096, torch.bfloat16, 100)
    with pytest.raises(RuntimeError, match="partition_tokens"):
        _native.decode_plan(1, 12, 64, 16, 4096, torch.bfloat16, -2)


def test_decode_plan_workgroup_form_needs_no_workspace():
    import torch

    # -1 forces one workgroup per (sequence, head): one partition, no workspace.
    part, ws = _native.decode_plan(8, 12, 64, 16, 131072, torch.bfloat16, -1)
    assert part >= 131072 and ws == 0
    # Automatic: short contexts take it too.
    assert _native.decode_plan(1, 12, 64, 16, 1024, torch.bfloat16, 0)[1] == 0
    assert not _native.decode_supported(72, torch.bfloat16)
    assert not _native.decode_supported(64, torch.float64)
    assert _native.decode_supported(96, torch.float32) and _native.decode_supported(4, torch.bfloat16)


def test_invalid_arguments_fail_before_launch():
    lib = _native.lib()
    # dtype 9 does not exist: rejected on the host, message recorded.
    rc = lib.mie_kv_append(0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 4, 4, 9, 0)
    assert rc == 2 and b"dtype" in lib.mie_last_error()
    rc = lib.mie_kv_gather(0, 0, 64, 64, 1, 0, 5, 0, 0, 0, 0, 1, 4, 16, 0, 0)
    assert rc == 1 and b"null pointer" in lib.mie_last_error()
    rc = lib.mie_paged_decode(
        0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, None, 10, 5, 1, 1, 64, 16, 1.0, 0, 0, 0, 0, 0, 0, 0, 1, 0
    )
    assert rc == 1 and b"ctx_len" in lib.mie_last_error()


def test_integration_binding_matches_the_library_signatures():
    """The ctypes binding the repository's integration notes give the
    reference declares, for every entry point it binds, the argument types
    moe_engine._native uses."""
    import types

    text = (Path(__file__).resolve().parents[1] / "INTEGRATION.md").read_text()
    block = re.search(r"## ctypes binding.*?```python\n(.*?)```", text, flags=re.S).group(1)
    fake = types.SimpleNamespace()

    class Entry:
        pass

    class FakeLib:
        def __getattr__(self, name):
            entry = Entry()
            setattr(self, name, entry)
            return entry

    lib = FakeLib()
    fake.CDLL = lambda path: lib
    ns = {}
    code = block.replace("import ctypes, math, torch", "import math, torch")
    ns["ctypes"] = types.SimpleNamespace(**{k: getattr(ctypes, k) for k in dir(ctypes) if not k.startswith("_")})
    ns["ctypes"].CDLL = fake.CDLL
    exec(code, ns)
    bound = {name: entry.argtypes for name, entry in vars(lib).items() if hasattr(entry, "argtypes")}
    assert len(bound) >= 10
    for name, argtypes in bound.items():
        want = _native._SIGNATURES[name][1]
        assert [t.__name__ for t in argtypes] == [t.__name__ for t in want], name


def test_block_plan_checks_fail_before_launch():
    """mie_block_plan_init refuses a short plan buffer and missing rows;
    mie_block_decode refuses a buffer that was never initialised - all on the
    host, before any launch."""
    lib = _native.lib()
    size = lib.mie_block_plan_bytes()
    assert 64 <= size <= 4096
    small = ctypes.create_string_buffer(size - 1)
    args = [0] * 42  # dim .. acc after (plan, plan_bytes); zeros are never dereferenced
    args[0:5] = [64, 2, 32, 16, 0]  # dim, heads, head_dim, block_size, dtype
    rc = lib.mie_block_plan_init(small, len(small), *args)
    assert rc == 1 and b"plan needs" in lib.mie_last_error()
    plan = ctypes.create_string_buffer(size)
    rc = lib.mie_block_plan_init(plan, len(plan), *args)
    assert rc == 1 and b"null scratch" in lib.mie_last_error()
    rc = lib.mie_block_decode(ctypes.create_string_buffer(size), 1 << 20, None, 5, None)
    assert rc == 1 and b"not initialised" in lib.mie_last_error()


def _valid_plan_args(**over):
    """mie_block_plan_init arguments after (plan, plan_bytes) that pass every
    host check: float32, d 64 = 2 heads x 32, block 16, 8 blocks, 4 experts,
    top-2, hidden 128.  Pointers are aligned stand-ins that the host checks
    never dereference."""
    names = ("dim heads head_dim block_size dtype attn_ln_w attn_ln_b attn_eps w_in b_in w_out b_out k_pool v_pool "
             "sblk shead num_blocks table table_len scale q attn h ws ws_bytes moe_ln_w moe_ln_b moe_eps router w1 "
             "b1 w2 b2 experts top_k hidden logits ids route_w hidden_act out acc").split()
    addr = iter(range(1 << 20, 1 << 30, 1 << 16))
    args = {name: next(addr) for name in names}
    args.update(dim=64, heads=2, head_dim=32, block_size=16, dtype=0, attn_eps=1e-5, moe_eps=1e-5,
                sblk=2 * 16 * 32, shead=16 * 32, num_blocks=8, table_len=8, scale=1.0, ws=0, ws_bytes=0,
                experts=4, top_k=2, hidden=128)
    args.update(over)
    assert len(args) == 42
    return [args[n] for n in names]


@pytest.mark.parametrize("change,code,message", [
    (dict(dtype=1), 0, b""),                        # bf16 passes every check
    (dict(hidden=130), 1, b"hidden=130"),           # an expert width only the MoE half sees
    (dict(dtype=3), 2, b""),                        # a dtype no launch is built for
    (dict(head_dim=48, heads=1, dim=48, sblk=16 * 48, shead=16 * 48), 2, b""),  # a head_dim the decode lacks
    (dict(table_len=0), 1, b"block table"),
    (dict(w1=(1 << 20) + 4), 1, b"aligned"),
    (dict(router=0), 1, b"null pointer"),
    (dict(experts=65), 1, b"experts"),
    (dict(sblk=16 * 32), 1, b"overlap"),
    (dict(acc=(1 << 20) + 8), 1, b"aligned"),   # the accumulator row of the four-launch form
])
def test_block_plan_init_makes_every_launch_check(change, code, message):
    """A plan that one of the five launches would refuse is refused when it is
    initialised, so mie_block_decode never stops between launches."""
    lib = _native.lib()
    plan = ctypes.create_string_buffer(lib.mie_block_plan_bytes())
    assert lib.mie_block_plan_init(plan, len(plan), *_valid_plan_args()) == 0
    rc = lib.mie_block_plan_init(plan, len(plan), *_valid_plan_args(**change))
    assert rc == code, lib.mie_last_error()
    assert message in lib.mie_last_error()


def test_block_decode_refuses_a_position_past_the_table_before_launching():
    """The new token's slot must lie inside the plan's block table (8 entries
    of 16 tokens here), and x must be aligned; both fail on the host."""
    lib = _native.lib()
    plan = ctypes.create_string_buffer(lib.mie_block_plan_bytes())
    assert lib.mie_block_plan_init(plan, len(plan), *_valid_plan_args()) == 0
    rc = lib.mie_block_decode(plan, 1 << 20, None, 8 * 16, None)
    assert rc == 1 and b"past the 8-entry block table" in lib.mie_last_error()
    rc = lib.mie_block_decode(plan, (1 << 20) + 4, None, 3, None)
    assert rc == 1 and b"aligned" in lib.mie_last_error()


def test_block_plan_ignores_the_accumulator_for_shapes_the_fused_attention_lacks():
    """head_dim 96 has the five-launch form only: a plan given an accumulator
    still initialises, and runs five launches at every position (six where
    the decode splits the context)."""
    lib = _native.lib()
    plan = ctypes.create_string_buffer(lib.mie_block_plan_bytes())
    args = _valid_plan_args(dim=192, heads=2, head_dim=96, sblk=2 * 16 * 96, shead=16 * 96)
    assert lib.mie_block_plan_init(plan, len(plan), *args) == 0, lib.mie_last_error()
    assert lib.mie_block_plan_launches(plan, 0) == 5
    assert lib.mie_block_plan_launches(plan, 100) == 5


def test_block_plan_launch_count_follows_the_form():
    """head_dim 32 with an accumulator: four launches up to 1024 cached
    tokens, then the five-launch form, six once the two-head decode splits
    its context (workspace needed); without the accumulator always the
    five-launch form.  Bad plans and positions are refused."""
    lib = _native.lib()
    plan = ctypes.create_string_buffer(lib.mie_block_plan_bytes())
    assert lib.mie_block_plan_init(plan, len(plan), *_valid_plan_args(table_len=200, num_blocks=200)) == 0
    assert lib.mie_block_plan_launches(plan, 0) == 4
    assert lib.mie_block_plan_launches(plan, 1023) == 4
    assert lib.mie_block_plan_launches(plan, 1024) in (5, 6)
    assert lib.mie_block_plan_launches(plan, 3000) == 6
    plain = ctypes.create_string_buffer(lib.mie_block_plan_bytes())
    assert lib.mie_block_plan_init(plain, len(plain), *_valid_plan_args(acc=0)) == 0
    assert lib.mie_block_plan_launches(plain, 0) == 5
    assert lib.mie_block_plan_launches(plan, -1) == -1
    assert lib.mie_block_plan_launches(ctypes.create_string_buffer(len(plan)), 0) == -1


@pytest.mark.parametrize("change,code,message", [
    (dict(dtype=3), 2, b"float32 or bfloat16 only"),
    (dict(head_dim=96), 2, b"head_dim 96"),
    (dict(max_ctx=1025 * 16), 2, b"contexts up to 1024 blocks"),
    (dict(acc=(1 << 20) + 4), 1, b"aligned"),
    (dict(ctx=17, max_ctx=16), 1, b"outside"),
])
def test_attn_out_checks_fail_before_launch(change, code, message):
    lib = _native.lib()
    args = dict(q=1 << 20, k=2 << 20, v=3 << 20, sblk=2 * 16 * 64, shead=16 * 64, num_blocks=8, table=4 << 20,
                table_len=8, ctx_dev=None, ctx=5, max_ctx=64, heads=2, head_dim=64, block_size=16, scale=0.125,
                w=5 << 20, acc=6 << 20, dtype=0)
    args.update(change)
    rc = lib.mie_attn_out_acc(*args.values(), None)
    assert rc == code and message in lib.mie_last_error(), lib.mie_last_error()
