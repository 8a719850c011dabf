"""Builds libbitexact_hip.so (every csrc/*.hip for gfx950) into bitexact/_lib/, in-tree, and its measurement
variant libbitexact_hip_phases.so (the same sources with -DBX_PHASES: kernels record phase timestamps that
bench.py --phases reads; loaded instead of the product library when BX_PHASES=1 is set).

Usage: python bitexact-llm_amd/build.py [jobs]   (also called by __graft_entry__.build()).
"""

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "bitexact", "_lib")
OBJ_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libbitexact_hip.so")
LIB_PHASES = os.path.join(OUT_DIR, "libbitexact_hip_phases.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-fwrapv",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",   # no packed fp32 ops
         "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]


def _compile(src, phases=False):
    obj = os.path.join(OBJ_DIR + ("_phases" if phases else ""), os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *(["-DBX_PHASES"] if phases else []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(jobs=8, phases=True):
    """Builds the product library, then (phases) the measurement variant."""
    lib = _build_one(jobs, False)
    if phases:
        _build_one(jobs, True)
    return lib


def _build_one(jobs, phases):
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR + ("_phases" if phases else ""), exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, phases), srcs))
    target = LIB_PHASES if phases else LIB
    tmp = target + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(int(sys.argv[1]) if len(sys.argv) > 1 else 8))
