"""Build ``libworldattention_amd.so`` (all gfx950 HIP kernels + the C ABI) in-tree.

    python -m worldattention_amd.csrc.build          # or build() from Python

Each ``*.hip`` file compiles to an object under ``csrc/_build/`` in parallel, then one hipcc link
writes ``worldattention_amd/libworldattention_amd.so``. Always recompiles (the build check is meant
to exercise the compiler every time).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_NAME = "libworldattention_amd.so"
ARCH = os.environ.get("WA_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # Packed fp32 VALU ops are disabled for every HIP source (see the package docs).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _compile(src: str, obj: str) -> None:
    cmd = [HIPCC, *COMMON_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "is not a recognized feature" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build(verbose: bool = True) -> str:
    out_dir = os.path.join(HERE, "_build")
    os.makedirs(out_dir, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(HERE, "*.hip")))
    objs = [os.path.join(out_dir, os.path.basename(s).replace(".hip", ".o")) for s in sources]
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=max(jobs, 1)) as pool:
        list(pool.map(_compile, sources, objs))
    target = os.path.join(PKG, LIB_NAME)
    tmp = target + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{res.stderr}")
    os.replace(tmp, target)
    if verbose:
        print(f"built {target} from {len(sources)} sources")
    return target


if __name__ == "__main__":
    build()
