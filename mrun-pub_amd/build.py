"""Build ``libqstore_hip.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python mrun-pub_amd/build.py`` or ``build()`` from Python.  Objects go to
``mrun-pub_amd/_build/``; the shared library lands next to this file so it travels
with the source tree.  Always recompiles every source (the build check must compile).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libqstore_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    # packed fp32 VALU forms are kept out of every kernel on this hardware
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # products and sums round separately unless a kernel asks for fmaf explicitly (the
    # reference's epilogues and reducers are unfused fp32 operations)
    "-ffp-contract=off",
    "-Wno-unused-command-line-argument",
    f"-I{PKG_DIR.parent / 'include'}",
]


def _sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.name + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd.insert(1, "-xhip")
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP/C++ source and link the shared library; returns its path."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: the QStore HIP library cannot be built")
    BUILD_DIR.mkdir(exist_ok=True)
    sources = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
