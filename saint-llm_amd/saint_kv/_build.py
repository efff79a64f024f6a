"""Build ``libsaintkv.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Run as ``python -m saint_kv._build`` (with ``saint-llm_amd`` on ``sys.path``)
or through ``__graft_entry__.build()``.  Objects are compiled in parallel into
``saint_kv/_build/`` and linked into ``saint_kv/libsaintkv.so`` in-tree, so the
library travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PROJECT_DIR = PKG_DIR.parent
REPO_DIR = PROJECT_DIR.parent
CSRC_DIR = PROJECT_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libsaintkv.so"

ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _filter(stderr: str) -> str:
    # hipcc's host pass does not know the packed-fp32-ops feature; that warning is noise.
    keep = [ln for ln in stderr.splitlines() if "packed-fp32-ops" not in ln]
    return "\n".join(keep)


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{_filter(res.stderr)}")
    msg = _filter(res.stderr).strip()
    if msg:
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every ``csrc/*.hip`` and link ``libsaintkv.so``; returns its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if res.returncode != 0:
        raise RuntimeError(f"link of libsaintkv.so failed:\n{_filter(res.stderr)}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
