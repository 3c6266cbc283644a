"""Build libmie_paged.so (the HIP kernels and C ABI) for gfx950, in-tree.

    python moe-inference-engine_amd/build_native.py

compiles csrc/*.hip with hipcc into moe_engine/libmie_paged.so.  The library
is written to a temporary name first and renamed, so a process that already
mapped the old file keeps a consistent copy.
"""

import os
import shlex
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
OUTPUT = PKG_ROOT / "moe_engine" / "libmie_paged.so"
ARCH = os.environ.get("MIE_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def build(verbose: bool = True) -> Path:
    sources = sorted(str(p) for p in CSRC.glob("*.hip"))
    tmp = OUTPUT.with_name(OUTPUT.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *sources, "-o", str(tmp)]
    if verbose:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{stderr}")
    if stderr.strip() and verbose:
        print(stderr, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build())
