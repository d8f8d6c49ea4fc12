"""Build ``libqstore_hip.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python mrun-pub_amd/build.py`` or ``build()`` from Python.  Objects go to
``mrun-pub_amd/_build/``; the shared library lands next to this file so it travels
with the source tree.  Always recompiles every source (the build check must compile).
"""

from __future__ import annotations

import os
import re
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
    # kernels with scalar arguments get their first 16 argument dwords preloaded into SGPRs
    # by the hardware (gfx950), so their first loads do not wait for an argument fetch
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-command-line-argument",
    f"-I{PKG_DIR.parent / 'include'}",
]


def _sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _scratch_kernels(remarks: str) -> list[str]:
    """Kernels whose resource-usage remarks report scratch memory (stack or spills)."""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            bad.append(f"{name} ({m.group(1)} bytes/lane)")
    return bad


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.name + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        # every kernel must run without scratch memory: a run-time index into a local array
        # or a spill puts values in scratch, whose accesses share the vector-memory wait
        # counter with the weight stream (a 1.6x slower decode pass when it happened)
        cmd[1:1] = ["-xhip", "-Rpass-analysis=kernel-resource-usage"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    bad = _scratch_kernels(proc.stderr)
    if bad:
        raise RuntimeError(f"{src.name}: kernels use scratch memory: " + "; ".join(bad))
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
