"""Build libgdn2_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m qwendopamine_amd.build`` (also called by ``__graft_entry__.build``).
The library is written next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB_NAME = "libgdn2_hip.so"
SOURCES = ["gdn2_api.hip", "gdn2_recurrent.hip", "gdn2_chunk_fwd.hip", "gdn2_chunk_bwd.hip", "gdn2_chunk_wide.hip", "gdn2_gate.hip",
           "gdn2_prologue.hip", "gdn2_prologue_bwd.hip", "gdn2_noalloc.hip", "gdn2_skinny.hip",
           "gdn2_attn.hip"]
ARCH = os.environ.get("GDN2_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed fp32 VALU ops are kept out of every kernel (never emitted).
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gdn2 HIP library cannot be built")


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    warn = "\n".join(
        ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()
    )
    if warn:
        print(warn, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link ``libgdn2_hip.so``; returns its path."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    objs = [objdir / (Path(s).stem + ".o") for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 4)) as ex:
        list(ex.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    out = PKG / LIB_NAME
    tmp = PKG / (LIB_NAME + ".tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
