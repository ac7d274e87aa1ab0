"""Compile the HIP sources of the run-time SDM mixer into an in-tree shared library for gfx950.

    python -m sdmchat_amd.build

compiles every ``sdmchat_amd/csrc/*.hip`` translation unit with ``hipcc`` (in parallel) and links
``sdmchat_amd/lib/libsdm_rt.so``.  The library is loaded by ``sdmchat_amd._lib`` through ctypes; it exports the C ABI
declared in ``include/sdm_rt.h``.  ``build(incremental=True)`` recompiles only the units whose source, or a header
they may include, is newer than their object file.
"""
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(PKG, "lib")
OBJ_DIR = os.path.join(LIB_DIR, "obj")
LIB = os.path.join(LIB_DIR, "libsdm_rt.so")
ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from forming packed FP32 VALU instructions.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-Wno-pass-failed",
]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _compile(src, extra_flags, verbose):
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra_flags, "-I", INCLUDE, "-I", CSRC, "-c", src, "-o", obj + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        return src, res.stdout + res.stderr
    os.replace(obj + ".tmp", obj)
    return src, None


def build(verbose=False, extra_flags=(), incremental=False, jobs=None):
    """Compile the library and return its path (every unit, unless ``incremental``)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    headers = glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(INCLUDE, "*.h"))
    newest_header = max((os.path.getmtime(h) for h in headers), default=0.0)
    todo = []
    for src in srcs:
        obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
        if (not incremental or not os.path.exists(obj)
                or os.path.getmtime(obj) < max(os.path.getmtime(src), newest_header)):
            todo.append(src)
    jobs = jobs or min(len(todo) or 1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        failed = [(s, err) for s, err in ex.map(lambda s: _compile(s, extra_flags, verbose), todo) if err]
    for s, err in failed:
        sys.stderr.write(f"--- {os.path.basename(s)}\n{err}")
    if failed:
        raise RuntimeError(f"hipcc failed for {', '.join(os.path.basename(s) for s, _ in failed)}")
    objs = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"linking {LIB} failed ({res.returncode})")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv))
