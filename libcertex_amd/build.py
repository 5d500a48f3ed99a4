"""Build libcertex_c.so (the C-ABI library with the gfx950 kernels) in this directory with hipcc.

    python -m libcertex_amd.build        # or: python libcertex_amd/build.py

Every source is compiled on every call (a few seconds each, in parallel); the library is written
next to this file so that it travels with the repository tree to the GPU box.
"""

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libcertex_c.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = [
    "kernels/screen.hip",
    "kernels/screen_wide.hip",
    "kernels/screen_tile.hip",
    "kernels/select.hip",
    "kernels/encode.hip",
    "kernels/partition.hip",
    "kernels/lists.hip",
    "certex.cpp",
    "c_api.cpp",
]

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    "-I",
    os.path.join(ROOT, "include"),
    # packed fp32 instructions are never emitted (they have given wrong results on these parts)
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src, obj_dir):
    path = os.path.join(CSRC, src)
    obj = os.path.join(obj_dir, src.replace("/", "_") + ".o")
    cmd = [HIPCC, "-x", "hip", *COMMON, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    workers = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
