"""Build libq36.so (every HIP source under csrc/) in-tree for gfx950.

The bundle's rebuild step (rebuild.json -> this file) and __graft_entry__.build() both call
build().  hipcc cross-compiles for gfx950 without a GPU.  Each translation unit is compiled to its
own object (in parallel), then the objects are linked with --no-undefined, so a unit that calls into
another one it is not linked with fails here rather than at load time.  link() is also how a loader
that builds one manifest op from its own cuda_sources list would link it.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libq36.so")
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # every fma in the kernels is written out; nothing else may be contracted
    "-ffp-contract=off",
    # packed fp32 instructions stay off (v_pk_*_f32 forms are not used on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
LINK_FLAGS = ["-shared", "-fPIC", f"--offload-arch={ARCH}", "-Wl,--no-undefined"]


def hipcc() -> str:
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))


def _quiet(stderr: str) -> str:
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is harmless
    return "\n".join(l for l in stderr.splitlines() if "packed-fp32-ops" not in l)


def compile_objects(srcs: list[str], out_dir: str, jobs: int | None = None, verbose: bool = False) -> list[str]:
    """Compile each source to out_dir/<stem>.o, in parallel; return the object paths in source order."""
    os.makedirs(out_dir, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc")]

    def one(src: str) -> str:
        obj = os.path.join(out_dir, os.path.splitext(os.path.basename(src))[0] + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, *inc, "-c", src, "-o", obj + ".tmp"]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({res.returncode}):\n{_quiet(res.stderr)}")
        if verbose and _quiet(res.stderr).strip():
            print(_quiet(res.stderr), file=sys.stderr)
        os.replace(obj + ".tmp", obj)
        return obj

    jobs = jobs or min(16, os.cpu_count() or 4, len(srcs))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        return list(pool.map(one, srcs))


def link(objs: list[str], out: str, verbose: bool = False) -> str:
    """Link objects into a shared library; an undefined symbol is an error."""
    tmp = out + ".tmp"
    cmd = [hipcc(), *LINK_FLAGS, *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(out)} failed ({res.returncode}):\n{_quiet(res.stderr)}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> str:
    return link(compile_objects(sources(), OBJ_DIR, verbose=verbose), LIB, verbose=verbose)


if __name__ == "__main__":
    print(build(verbose=True))
