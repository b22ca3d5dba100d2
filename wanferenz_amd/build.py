"""Build recipe for libwanferenz_amd.so (gfx950).

``python -m wanferenz_amd.build`` compiles every HIP source under
wanferenz_amd/csrc with hipcc, one object per source in parallel, and links
them into one shared library in wanferenz_amd/lib/.  No torch extension
machinery is involved: the library exposes a plain C ABI
(include/wanferenz_amd.h) and the Python side binds it with ctypes.

``build(incremental=True)`` (``python -m wanferenz_amd.build -i``) recompiles
only the objects older than their source or any header; the default rebuilds
everything.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(LIBDIR, "obj")
LIBNAME = "libwanferenz_amd.so"
ARCH = os.environ.get("WZ_OFFLOAD_ARCH", "gfx950")

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # packed fp32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]
LINK_FLAGS = [f"--offload-arch={ARCH}", "-shared", "-fPIC"]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def headers():
    inc = os.path.join(ROOT, "include")
    return [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")] + [
        os.path.join(inc, f) for f in os.listdir(inc) if f.endswith(".h")]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}): {cmd[-1]}")
    warn = [l for l in (r.stderr or "").splitlines() if "warning" in l and "packed-fp32-ops" not in l]
    if verbose and warn:
        sys.stderr.write("\n".join(warn) + "\n")


def _obj(src: str) -> str:
    return os.path.join(OBJDIR, os.path.basename(src)[:-4] + ".o")


def build(verbose: bool = False, incremental: bool = False, jobs: int = 0) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    out = os.path.join(LIBDIR, LIBNAME)
    srcs = sources()
    newest_header = max(os.path.getmtime(h) for h in headers())
    todo = []
    for s in srcs:
        o = _obj(s)
        if incremental and os.path.exists(o) and os.path.getmtime(o) >= max(os.path.getmtime(s), newest_header):
            continue
        todo.append(s)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    cmds = [[hipcc(), *COMPILE_FLAGS, *inc, "-c", "-o", _obj(s), s] for s in todo]
    jobs = jobs or min(len(cmds) or 1, max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = out + ".tmp"
    _run([hipcc(), *LINK_FLAGS, "-o", tmp, *[_obj(s) for s in srcs]], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, incremental="-i" in sys.argv[1:]))
