"""Build libfhecore.so (HIP, gfx950) in-tree.

    python fhe-mamba_amd/build.py [--jobs N]

Every source under csrc/ is compiled with hipcc for gfx950 and linked into
fhemamba_amd/libfhecore.so, next to the ctypes loader.  Compilation always
runs (no staleness check): the caller decides when to rebuild.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build", "obj")
LIB = os.path.join(HERE, "fhemamba_amd", "libfhecore.so")
ARCH = os.environ.get("FHEMAMBA_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # The CKKS encoder's rounding is defined on unfused IEEE operations.
    "-ffp-contract=off",
    # Packed-FP32 instructions are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-value", "-Wno-unused-function",
]
SOURCES = ["context.cpp", "ntt.hip", "poly_ops.hip", "keyswitch.hip", "encode.hip",
           "keygen.hip", "capi.cpp"]


def _compile(src: str) -> tuple[str, int, str]:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                      if "packed-fp32-ops" not in line and line.strip())
    return obj, res.returncode, noise


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, rc, msg in ex.map(_compile, SOURCES):
            if rc != 0:
                raise RuntimeError(f"hipcc failed for {obj}:\n{msg}")
            if verbose and msg:
                print(msg, file=sys.stderr)
            objs.append(obj)
    tmp = LIB + ".tmp"
    res = subprocess.run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
