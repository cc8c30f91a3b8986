"""Builds libhip_matmul.so (the C-ABI HIP library) in-tree with hipcc for gfx950."""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libhip_matmul.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The product library's sources: every .hip file of csrc/ but probes.hip
# (measurement kernels for bench.py --probes), which is built into a library
# of its own. The largest first, so the parallel compile ends soonest.
PROBE_SOURCES = ["probes.hip"]
SOURCES = sorted((f for f in os.listdir(CSRC) if f.endswith(".hip") and f not in PROBE_SOURCES),
                 key=lambda f: (not f.startswith("launch_"), f))
PROBE_LIB_PATH = os.path.join(PKG_DIR, "libhip_probes.so")
FLAGS_FILE = os.path.join(CSRC, "hipcc_flags.txt")


def read_flags(path: str = FLAGS_FILE):
    """(common flags, {source: extra flags}) from hipcc_flags.txt, the file
    CMakeLists.txt reads too."""
    common, extra = [], {}
    with open(path) as f:
        for line in f:
            line = line.strip()
            if not line or line.startswith("#"):
                continue
            head, _, rest = line.partition(" ")
            if head.endswith(".hip"):
                extra.setdefault(head, []).extend(rest.split())
            else:
                common.append(line)
    return common, extra


HIPCC_FLAGS, EXTRA_FLAGS = read_flags()


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def _compile(sources, build_dir, jobs, verbose):
    objs, procs = [], []
    for src in sources:
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
    return objs


def _link(objs, path, verbose):
    tmp = path + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, path)


def build(verbose: bool = False, jobs: int = 8) -> str:
    """Compile every HIP source to an object, then link the shared library
    (libhip_matmul.so) and the measurement-probe library (libhip_probes.so)."""
    build_dir = os.path.join(PKG_DIR, "_build")
    os.makedirs(build_dir, exist_ok=True)
    objs = _compile(SOURCES + PROBE_SOURCES, build_dir, jobs, verbose)
    _link(objs[:len(SOURCES)], LIB_PATH, verbose)
    _link(objs[len(SOURCES):], PROBE_LIB_PATH, verbose)
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
