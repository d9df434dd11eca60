"""Build the gfx950 HIP library in-tree: micro_vllm_amd/_lib/libmvllm_amd.so.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950``
into an object (in parallel), then linked into one shared library exposing
the C ABI declared in ``include/mvllm_amd.h``. No torch extension machinery
is involved: the library links only against the HIP runtime.

    python micro-vllm_amd/build.py [--jobs N] [--verbose]
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_ROOT.parent
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
OBJ_DIR = PACKAGE_ROOT / "_build"
LIB_DIR = PACKAGE_ROOT / "micro_vllm_amd" / "_lib"
LIB_NAME = "libmvllm_amd.so"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build the library")


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def _compile(source: Path, verbose: bool) -> Path:
    obj = OBJ_DIR / (source.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(INCLUDE), "-I", str(CSRC), "-c", str(source), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so; that is harmless.
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{stderr}")
    if stderr.strip() and verbose:
        print(stderr, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; return its path."""

    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    workers = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose), sources))
    target = library_path()
    tmp = target.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, target)
    return target


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("--verbose", action="store_true")
    args = parser.parse_args()
    path = build(jobs=args.jobs, verbose=args.verbose)
    print(path)


if __name__ == "__main__":
    main()
