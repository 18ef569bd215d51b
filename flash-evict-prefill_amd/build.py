"""Build libflash_evict_hip.so (gfx950) into the flash_evict package directory.

Usage: python build.py [--jobs N] [--verbose]

HIP sources are compiled with hipcc for gfx950 only; the host-only API file is compiled
with g++. Objects go to ../_build (git-ignored); the shared library lands next to the
Python package so that it travels with the source tree.
"""
import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "flash_evict")
LIB_NAME = "libflash_evict_hip.so"
BUILD_DIR = os.path.join(os.path.dirname(HERE), "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["fe_attn.hip", "fe_attn_fast.hip", "fe_select.hip", "fe_gather.hip", "fe_snap.hip", "fe_static.hip"]
CXX_SOURCES = ["fe_api.cpp"]

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code (the host pass warns that it
# does not know the feature; that is expected). -munsafe-fp-atomics: hardware
# global_atomic_add_f32 for the importance accumulation.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-I" + os.path.join(ROCM, "include"),
             "-D__HIP_PLATFORM_AMD__"]


def _hipcc():
    path = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build flash_evict)")
    return path


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s" % (proc.returncode, " ".join(cmd), err))
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(jobs=None, verbose=False, out=None, defines=()):
    """Compile every source and link the shared library. Returns the library path.

    `out` overrides the library path and `defines` adds -D options (tuning variants).
    """
    build_dir = BUILD_DIR if not defines else os.path.join(BUILD_DIR, "_".join(defines).replace("=", ""))
    os.makedirs(build_dir, exist_ok=True)
    hipcc = _hipcc()
    dflags = ["-D" + d for d in defines]
    cmds, objs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(build_dir, src + ".o")
        cmds.append([hipcc] + HIPCC_FLAGS + dflags + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in CXX_SOURCES:
        obj = os.path.join(build_dir, src + ".o")
        cmds.append(["g++"] + CXX_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    t0 = time.time()
    jobs = jobs or min(len(cmds), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    out = out or os.path.join(OUT_DIR, LIB_NAME)
    tmp = out + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, out)
    if verbose:
        print("built %s in %.1fs" % (out, time.time() - t0), flush=True)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--out", default=None, help="library path (default: the package directory)")
    ap.add_argument("-D", dest="defines", action="append", default=[], help="extra preprocessor define")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.out, tuple(args.defines)))
