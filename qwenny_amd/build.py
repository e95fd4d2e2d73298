"""Build libqwenny_hip.so in-tree for gfx950 with hipcc (no GPU needed: hipcc cross-compiles).

The host repacker is compiled without floating-point contraction so that its arithmetic matches the reference's
(Rust does not fuse multiply-adds); the device code is compiled with packed-FP32 instructions disabled.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libqwenny_hip.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("QWENNY_ARCH", "gfx950")

HOST_SRC = ["host.cpp"]
HIP_SRC = ["kernels.hip", "api.hip"]

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
    objs = []
    for src in HOST_SRC:
        obj = os.path.join(build_dir, src + ".o")
        _run([hipcc, *COMMON, "-ffp-contract=off", "-pthread", "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HIP_SRC:
        obj = os.path.join(build_dir, src + ".o")
        _run([hipcc, *COMMON, *DEVICE, *extra, "-c", "-x", "hip", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    tmp = out + ".tmp"
    _run([hipcc, *DEVICE, "-shared", "-pthread", "-o", tmp, *objs])
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    build(verbose=True)
