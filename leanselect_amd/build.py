"""Build ``libleanselect_hip.so`` for gfx950 with hipcc (in-tree).

Usage: ``python -m leanselect_amd.build`` (or ``__graft_entry__.build()``).
Each ``csrc/*.hip`` file is compiled to an object under ``_build/`` in parallel,
then linked into ``leanselect_amd/libleanselect_hip.so``.
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
BUILD = PKG / "_build"
LIB = PKG / "libleanselect_hip.so"
ARCH = os.environ.get("LEANSELECT_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Keep the compiler from forming packed float32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-file additions.  The attention kernel only handles finite and -inf
# scores, so it is built without IEEE NaN quieting: maxima then need no
# canonicalising moves and fuse into v_max3.
FILE_FLAGS = {
    "ls_attention": ["-mno-amdgpu-ieee", "-fno-honor-nans"],
    # MFMAs accumulate in ordinary VGPRs, so their results need no copies out
    # of the accumulation registers before the pooling reads them.  NaN is
    # honoured here: page maxima propagate NaN (v_maximum3_f32), as the
    # reference's max pooling does.
    "ls_select": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # The decoder kernels round every float32 product and sum separately, as
    # the reference's torch expressions do.
    "ls_model": ["-ffp-contract=off"],
}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the LeanSelect HIP library cannot be built")
    return exe


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.stem, []), "-I", str(PKG.parent / "include"),
           "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
