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
    """The ctypes binding INTEGRATION.md offers the reference declares, for
    every entry point it binds, the argument types moe_engine._native uses."""
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
    args = [0] * 41  # dim .. out after (plan, plan_bytes); zeros are never dereferenced
    args[0:5] = [64, 2, 32, 16, 0]  # dim, heads, head_dim, block_size, dtype
    rc = lib.mie_block_plan_init(small, len(small), *args)
    assert rc == 1 and b"plan needs" in lib.mie_last_error()
    plan = ctypes.create_string_buffer(size)
    rc = lib.mie_block_plan_init(plan, len(plan), *args)
    assert rc == 1 and b"null scratch" in lib.mie_last_error()
    rc = lib.mie_block_decode(ctypes.create_string_buffer(size), 1 << 20, 5, None)
    assert rc == 1 and b"not initialised" in lib.mie_last_error()
