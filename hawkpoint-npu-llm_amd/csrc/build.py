"""Build libhk.so for gfx950 from the HIP sources in this directory.

Usage: python build.py [--jobs N] [--no-phases]
Writes ../lib/libhk.so (next to the Python runtime that loads it) and
../lib/libhk_phases.so: the same library with the decode step's phase stamps
compiled in (persistent.hip with -DHK_PHASE_STAMPS, read back by
hk_phase_stamps), which `bench.py --workload phases` loads.
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


PHASES = "persistent.hip+phases"  # persistent.hip with the phase stamps


def compile_one(src):
    stamps = src == PHASES
    name = "persistent.hip" if stamps else src
    obj = OBJ_DIR / (Path(name).stem + ("_phases" if stamps else "") + ".o")
    cmd = [HIPCC, *FLAGS, *(["-DHK_PHASE_STAMPS"] if stamps else []), "-c", str(HERE / name), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    return src, obj, proc


def link(objs, name):
    lib = LIB_DIR / name
    tmp = LIB_DIR / (name + ".tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, lib)
    return lib


def build(jobs=4, verbose=False, phases=True):
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = {}
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for src, obj, proc in pool.map(compile_one, SOURCES + ([PHASES] if phases else [])):
            out = (proc.stdout + proc.stderr).strip()
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{out}")
            if verbose and out:
                print(out, file=sys.stderr)
            objs[src] = str(obj)
    lib = link([objs[s] for s in SOURCES], "libhk.so")
    if phases:
        link([objs[PHASES] if s == "persistent.hip" else objs[s] for s in SOURCES], "libhk_phases.so")
    return lib


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=4)
    parser.add_argument("-v", "--verbose", action="store_true")
    parser.add_argument("--no-phases", action="store_true", help="skip libhk_phases.so")
    args = parser.parse_args()
    print(build(args.jobs, args.verbose, phases=not args.no_phases))
