"""Builds libea_exl3.so (the C ABI of include/ea_exl3.h) for gfx950 with hipcc, in-tree next to the ea_exl3
package. Every .hip (device) and .cpp (host) file under csrc/ compiles to its own object in parallel, then one link.

    python expertatlas-glm5.3_amd/build.py [--jobs N] [--stamps]

--stamps builds the timeline variant instead, libea_exl3_stamps.so (EA_STAMPS defined: the decode layer and the
small-row linear store per-block stage stamps into a region the host attaches; timeline.py reads them). The product
library is never built with it.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "ea_exl3", "libea_exl3.so")
STAMPS_OUT = os.path.join(HERE, "ea_exl3", "libea_exl3_stamps.so")
OBJ = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ROCM_INC = "/opt/rocm/include"

FLAGS = [
    "-O3", "--offload-arch=gfx950", "-fPIC", "-std=c++17",
    # keep every fp32 rounding point where the source puts it (no fused multiply-adds the source did not ask for)
    "-ffp-contract=off",
    # no packed fp32 (v_pk_*_f32) instructions: some of their forms have given wrong results on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


def _compile(src: str, obj_dir: str = OBJ, defs: tuple = ()) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(os.path.basename(src))[0] + ".o")
    # .hip: device code for gfx950; .cpp: host-only C++ (the bank reader) against the HIP runtime
    cmd = [HIPCC, *FLAGS, *defs, "-c", src, "-o", obj] if src.endswith(".hip") else \
        [CXX, "-O2", "-fPIC", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I" + ROCM_INC,
         "-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(jobs: int | None = None, stamps: bool = False) -> str:
    obj_dir = os.path.join(OBJ, "stamps") if stamps else OBJ
    out = STAMPS_OUT if stamps else OUT
    defs = ("-DEA_STAMPS",) if stamps else ()
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    jobs = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defs), srcs))
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--stamps", action="store_true", help="the timeline variant (libea_exl3_stamps.so)")
    a = ap.parse_args()
    print(build(a.jobs, a.stamps))
