"""Build libmie_paged.so (the HIP kernels and C ABI) for gfx950, in-tree.

    python moe-inference-engine_amd/build_native.py

compiles each csrc/*.hip with hipcc (in parallel, one object per source) and
links the objects into moe_engine/libmie_paged.so.  The library is written to
a temporary name first and renamed, so a process that already mapped the old
file keeps a consistent copy.
"""

import os
import shlex
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
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
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    stderr = "\n".join(line for line in proc.stderr.splitlines() if NOISE not in line)
    return proc.returncode, stderr


def build(verbose: bool = True) -> Path:
    _link(sorted(CSRC.glob("*.hip")), OUTPUT, verbose)
    return OUTPUT


def _link(sources, output: Path, verbose: bool, extra=()) -> None:
    tmp = output.with_name(output.name + f".tmp{os.getpid()}")
    jobs = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with tempfile.TemporaryDirectory(prefix="mie_build_") as objdir:
        objs = [str(Path(objdir) / (src.stem + ".o")) for src in sources]
        compiles = [[hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", obj]
                    for src, obj in zip(sources, objs)]
        with ThreadPoolExecutor(jobs) as pool:
            results = list(pool.map(lambda c: _run(c, verbose), compiles))
        failed = [(c[-3], rc, err) for c, (rc, err) in zip(compiles, results) if rc != 0]
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n".join(f"{src} ({rc}):\n{err}" for src, rc, err in failed))
        for _, err in results:
            if err.strip() and verbose:
                print(err, file=sys.stderr)
        rc, err = _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)], verbose)
        if rc != 0:
            tmp.unlink(missing_ok=True)
            raise RuntimeError(f"hipcc link failed ({rc}):\n{err}")
    os.replace(tmp, output)


if __name__ == "__main__":
    print(build())
