"""Build libqwenny_hip.so in-tree for gfx950 with hipcc (no GPU needed: hipcc cross-compiles).

The host repacker is compiled without floating-point contraction so that its arithmetic matches the reference's
(Rust does not fuse multiply-adds); the device code is compiled with packed-FP32 instructions disabled.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libqwenny_hip.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("QWENNY_ARCH", "gfx950")

HOST_SRC = ["host.cpp"]
HIP_SRC = ["api.hip", "noalloc.hip", "dequant.hip", "consumers.hip", "diag.hip", "graph.hip"]
# kernels.hip is compiled once per (storage format, epilogue) pair and once for the dispatcher, in parallel; the
# formats are the F_* combinations that kernels.hip's launch() dispatches.
KERNEL_FORMATS = {"i4": 0, "i4s32": 4, "zp": 2, "zps32": 6, "i8": 5, "i8perch": 13, "bf16": 16}
KERNEL_EPIS = {"plain": 0, "silu": 1, "argmax": 2}

COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that warning is expected
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose=False, out=LIB, defines=()):
    """Compile and link the library into `out`; `defines`: extra -D macros (tuning experiments only)."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    build_dir = BUILD if out == LIB else out + ".build"
    os.makedirs(build_dir, exist_ok=True)
    extra = [f"-D{d}" for d in defines]
    jobs = []
    for src in HOST_SRC:
        obj = os.path.join(build_dir, src + ".o")
        jobs.append((obj, [hipcc, *COMMON, "-ffp-contract=off", "-pthread", "-c", os.path.join(CSRC, src), "-o", obj]))
    for src in HIP_SRC:
        obj = os.path.join(build_dir, src + ".o")
        jobs.append((obj, [hipcc, *COMMON, *DEVICE, *extra, "-c", "-x", "hip", os.path.join(CSRC, src), "-o", obj]))
    kern = os.path.join(CSRC, "kernels.hip")
    parts = [("dispatch", ["-DQH_PART_DISPATCH"])]
    parts += [(f"{f}_{e}", [f"-DQH_PART_F={fv}", f"-DQH_PART_EPI={ev}"])
              for f, fv in KERNEL_FORMATS.items() for e, ev in KERNEL_EPIS.items()]
    for name, defs in parts:
        obj = os.path.join(build_dir, f"kernels_{name}.o")
        jobs.append((obj, [hipcc, *COMMON, *DEVICE, *extra, *defs, "-c", "-x", "hip", kern, "-o", obj]))
    # the largest objects first; workers: this machine's cores, at most 16
    jobs.sort(key=lambda j: "plain" not in j[0] and "silu" not in j[0] and "argmax" not in j[0])
    workers = max(1, min(16, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(_run, [cmd for _, cmd in jobs]))
    objs = [obj for obj, _ in jobs]
    tmp = out + ".tmp"
    _run([hipcc, *DEVICE, "-shared", "-pthread", "-o", tmp, *objs])
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    build(verbose=True)
