"""Builds libhip_matmul.so (the C-ABI HIP library) in-tree with hipcc for gfx950."""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libhip_matmul.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["hip_matmul.hip", "moe.hip", "attention.hip", "unsupported_ops.hip", "probes.hip"]

# Bit-exactness of the quantization, dequantization and SwiGLU paths relies on
# single IEEE operations: no contraction, correctly rounded division, IEEE
# denormals. Packed FP32 instructions are disabled for the device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

# Per-source additions. attention.hip: matrix-core results in VGPRs, so the
# attention kernel's output accumulators (rescaled on the VALU between
# products) are not copied to and from accumulation registers every tile.
EXTRA_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def build(verbose: bool = False, jobs: int = 3) -> str:
    """Compile every HIP source to an object, then link the shared library."""
    build_dir = os.path.join(PKG_DIR, "_build")
    os.makedirs(build_dir, exist_ok=True)
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    for p in procs:
        _wait(p)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _wait(item):
    cmd, proc = item
    out, _ = proc.communicate()
    text = out.decode(errors="replace")
    # hipcc's host pass does not know the device-only target feature.
    text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if proc.returncode != 0:
        sys.stderr.write(text + "\n")
        raise subprocess.CalledProcessError(proc.returncode, cmd)


if __name__ == "__main__":
    print(build(verbose=True))
