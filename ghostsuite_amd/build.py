"""Build recipe for libghost_hip.so: hipcc for gfx950, one object per source, in-tree.

The library is a plain C-ABI shared object (include/ghost_hip.h); it depends only on the HIP
runtime.  At run time it binds to the libamdhip64.so.7 that torch has already loaded (the
package imports torch before loading the library), so torch streams and the kernels share
one HIP runtime.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIBNAME = "libghost_hip.so"
INCLUDE = PKG.parent / "include"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists() and shutil.which(cand) is None:
        raise RuntimeError("hipcc not found; set HIPCC or install ROCm")
    return cand


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def library_path() -> Path:
    return LIBDIR / LIBNAME


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links libghost_hip.so (always rebuilds)."""
    cc = hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        errs = "\n".join(l for l in res.stderr.splitlines()
                         if "packed-fp32-ops" not in l)  # host pass does not know the feature
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{errs}")
        if verbose and errs.strip():
            print(errs, file=sys.stderr)
        return obj

    n = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=n) as ex:
        objs = list(ex.map(compile_one, srcs))
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
