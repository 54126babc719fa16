"""Build the gfx950 HIP library `lib/libcausal_tuner_hip.so` in-tree.

Every kernel source under csrc/ is compiled by hipcc for gfx950 only and linked into one
shared library that exports the C ABI of include/causal_tuner_hip.h. The library is loaded
with ctypes after torch, so it binds to the HIP runtime torch already mapped (same soname).

    python causal-tuner_amd/build.py [--jobs N] [--incremental]
"""

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB_NAME = "libcausal_tuner_hip.so"
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # NF4 decoding must multiply and add separately (no FMA contraction).
    "-ffp-contract=off",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-I", os.path.join(ROOT, "include"),
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def library_path():
    return os.path.join(LIB_DIR, LIB_NAME)


def _compile(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def _stale(src):
    """True when src's object is missing or older than src or any header it may include."""
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    if not os.path.exists(obj):
        return True
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hpp", ".h"))]
    headers.append(os.path.join(ROOT, "include", "causal_tuner_hip.h"))
    return os.path.getmtime(obj) < max(os.path.getmtime(p) for p in [src, *headers])


def build(jobs=None, verbose=True, incremental=False):
    """Compile every source (or, with `incremental`, only those whose object is stale) and
    link the library."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    todo = [src for src in srcs if _stale(src)] if incremental else srcs
    jobs = jobs or min(max(len(todo), 1), max(1, (os.cpu_count() or 2) // 2))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(_compile, todo))
    objs = [os.path.join(OBJ_DIR, os.path.basename(src) + ".o") for src in srcs]
    out = library_path()
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("--incremental", action="store_true", help="recompile only stale objects")
    args = parser.parse_args()
    build(args.jobs, incremental=args.incremental)
    sys.exit(0)
