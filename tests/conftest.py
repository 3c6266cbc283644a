"""Test configuration: import paths, the `gpu` marker, device gating.

Tests marked `gpu` need a ROCm device (an MI355X).  When pytest is asked for
them explicitly (-m gpu) they run and fail loudly without a device; otherwise,
on a machine without a GPU, they are skipped so the CPU suite stays usable.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "moe-inference-engine_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    if (config.option.markexpr or "").strip() == "gpu":
        return  # asked for explicitly: let them fail on a machine without a GPU
    skip = pytest.mark.skip(reason="no ROCm GPU on this machine")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def print_case(*parts):
    """Name the case on stdout (flushed) before a GPU step, so a run that dies
    mid-test still says which case it was in."""
    print("[case]", *parts, flush=True)
