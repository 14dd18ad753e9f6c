"""Build libnaylis_mom.so (gfx950) in-tree with hipcc, then the torch
extension of the fused layer node over it.

    python -m naylis_amd.build [--jobs N]

Each .hip source is compiled to an object in parallel, then linked into
``naylis_amd/_lib/libnaylis_mom.so``.  Flags: -O3, gfx950 only, packed fp32
instructions disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``),
correctly rounded fp32 division (the router's prefix mean divides in fp32
exactly as the reference does).  ``csrc/torch_layer.cpp`` becomes
``naylis_amd/_lib/ext/naylis_torch.so`` (torch.utils.cpp_extension, host
code only); it calls the library's C ABI, whose symbols it takes from the
library loaded first with global visibility.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
OBJ_DIR = os.path.join(OUT_DIR, "obj")
LIB = os.path.join(OUT_DIR, "libnaylis_mom.so")
EXT_DIR = os.path.join(OUT_DIR, "ext")
EXT_NAME = "naylis_torch"
EXT = os.path.join(EXT_DIR, EXT_NAME + ".so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall", "-Wno-unused-result",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build naylis_amd)")
    return path


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build_torch_ext(verbose=False):
    """Compile csrc/torch_layer.cpp into the torch extension (every time: the
    previous outputs are removed first)."""
    import ctypes

    import torch.utils.cpp_extension as ce
    os.makedirs(EXT_DIR, exist_ok=True)
    for f in os.listdir(EXT_DIR):
        if f.endswith((".o", ".so")):
            os.remove(os.path.join(EXT_DIR, f))
    # cpp_extension imports the module it built: its C-ABI symbols come from
    # the library, loaded here with global visibility as naylis_amd._lib does
    ctypes.CDLL(LIB, mode=ctypes.RTLD_GLOBAL)
    ce.load(name=EXT_NAME, sources=[os.path.join(CSRC, "torch_layer.cpp")], build_directory=EXT_DIR,
            extra_include_paths=[INCLUDE], extra_cflags=["-O2"], verbose=verbose)
    if not os.path.exists(EXT):
        raise RuntimeError(f"torch extension build produced no {EXT}")
    return EXT


def _compile(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc()] + HIPCC_FLAGS + ["-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, err


def build(jobs=None, verbose=False):
    """Compile every csrc/*.hip and link the shared library. Returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    if verbose:
        for _, err in results:
            if err.strip():
                print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_torch_ext(verbose)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
