"""Build recipe for the gfx950 HIP library behind the omniserver_amd C ABI.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only and linked
into ``omniserver_amd/_lib/libomniserver_amd.so`` (in-tree, so it travels with
the repository snapshot to the GPU box).  Run ``python -m omniserver_amd.build``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libomniserver_amd.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU ops are disabled for every device pass (this pool has seen
# silent wrong results from some of their forms); the host pass ignores it.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{CSRC}",
    f"-I{INCLUDE}",
]


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"  # the host pass warns it does not know the feature
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, flush=True)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources and link the shared library; returns its path."""
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], verbose), zip(srcs, objs)))
    out = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
