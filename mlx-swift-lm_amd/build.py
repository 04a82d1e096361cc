"""Build recipe of liblsamp.so (gfx950) and of the oracle.

    python mlx-swift-lm_amd/build.py            # library + oracle
    python mlx-swift-lm_amd/build.py --lib-only

hipcc flags that matter for results, not only speed:
  -ffp-contract=off                         every fp32 op rounded as written
                                            (penalty arithmetic, the fixed-point
                                            draw weights)
  -fhip-fp32-correctly-rounded-divide-sqrt  x / T and x / p are IEEE divisions
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                            no packed fp32 instructions
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "liblsamp.so")
ORACLE_DIR = os.path.join(REPO, "oracle")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ARCH = os.environ.get("LSAMP_OFFLOAD_ARCH", "gfx950")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-ffp-contract=off",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
SOURCES_HIP = ["lsamp_kernels.hip", "lsamp_topk.hip", "lsamp_rank.hip", "lsamp_commit.hip",
               "lsamp_mask.hip", "lsamp_noalloc.hip", "lsamp_penalize.hip"]
SOURCES_CPP = ["lsamp_api.cpp"]
HEADERS = ["lsamp_internal.h", "lsamp_device.h"]


def run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib(verbose_asm: bool = False, jobs: int = 0) -> str:
    """Compile every source (in parallel, `jobs` at once; 0 = up to 8) and
    link liblsamp.so."""
    os.makedirs(LIB_DIR, exist_ok=True)
    cmds, objs = [], []
    for src in SOURCES_HIP:
        obj = os.path.join(LIB_DIR, src.replace(".hip", ".o"))
        cmds.append([HIPCC, "-x", "hip", *COMMON, *DEVICE, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in SOURCES_CPP:
        obj = os.path.join(LIB_DIR, src.replace(".cpp", ".o"))
        cmds.append([HIPCC, *COMMON, "-D__HIP_PLATFORM_AMD__", "-c", os.path.join(CSRC, src),
                     "-o", obj])
        objs.append(obj)
    jobs = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(run, c) for c in cmds]:
            f.result()
    tmp = LIB + ".tmp"
    run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    return LIB


def build_oracle() -> str:
    run(["make", "-s", "-C", ORACLE_DIR])
    return os.path.join(ORACLE_DIR, "liblsamp_oracle.so")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    args = ap.parse_args(argv)
    build_lib()
    if not args.lib_only:
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main())
