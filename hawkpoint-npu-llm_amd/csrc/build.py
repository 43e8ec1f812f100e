"""Build libhk.so for gfx950 from the HIP sources in this directory.

Usage: python build.py [--jobs N]
Writes ../lib/libhk.so (next to the Python runtime that loads it).
"""

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
LIB_DIR = HERE.parent / "lib"
OBJ_DIR = HERE / "_build"
SOURCES = ["gemv.hip", "attention.hip", "ops.hip", "prefill.hip", "moe.hip", "experts.hip", "persistent.hip", "engine.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: a*b+c stays two roundings, as NumPy evaluates it.
# -packed-fp32-ops off: no v_pk_*_f32 generation.
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
    f"-I{HERE}",
]


def compile_one(src):
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(HERE / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    return src, obj, proc


def build(jobs=4, verbose=False):
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = []
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for src, obj, proc in pool.map(compile_one, SOURCES):
            out = (proc.stdout + proc.stderr).strip()
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{out}")
            if verbose and out:
                print(out, file=sys.stderr)
            objs.append(str(obj))
    lib = LIB_DIR / "libhk.so"
    tmp = LIB_DIR / "libhk.so.tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=4)
    parser.add_argument("-v", "--verbose", action="store_true")
    args = parser.parse_args()
    print(build(args.jobs, args.verbose))
