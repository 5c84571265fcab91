"""Build libaxs6.so (the gfx950 C-ABI library) and the torch extension
axs._C in-tree.

    python axs-6_amd/build.py            # build into axs-6_amd/axs/
    python axs-6_amd/build.py --clean

Each csrc/*.hip file is compiled with hipcc to an object in axs-6_amd/_build/
(in parallel), then linked into axs-6_amd/axs/_lib/libaxs6.so, which exposes
the C ABI declared in include/axs6.h (bound with ctypes by axs/_lib.py).
csrc/torch_ext.cpp is compiled with the host C++ compiler against torch's
headers into axs-6_amd/axs/_C.so, a thin extension that calls that C ABI
(the linear's host logic and autograd node); it links libaxs6.so through an
$ORIGIN-relative run path.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
OUT_DIR = os.path.join(PKG, "axs", "_lib")
OUT = os.path.join(OUT_DIR, "libaxs6.so")
EXT_SRC = os.path.join(CSRC, "torch_ext.cpp")
EXT_OUT = os.path.join(PKG, "axs", "_C.so")
CXX = os.environ.get("CXX", "g++")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep hipcc from emitting packed-fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def ext_compile_command(obj: str) -> list[str]:
    """g++ command line compiling the torch extension (torch's include paths
    and C++ ABI flag; HIP headers for the current-stream query)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce

    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", "-Wno-deprecated-declarations",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"]
    for inc in (*ce.include_paths(), sysconfig.get_paths()["include"], "/opt/rocm/include",
                os.path.join(ROOT, "include")):
        cmd += ["-I", inc]
    return cmd + ["-c", EXT_SRC, "-o", obj]


def ext_link_command(obj: str, out: str) -> list[str]:
    """Links the extension against torch and libaxs6.so (found beside it at
    run time through $ORIGIN/_lib)."""
    from torch.utils import cpp_extension as ce

    torch_lib = ce.library_paths()[0]
    return [CXX, "-shared", "-fPIC", obj, "-o", out,
            "-L", torch_lib, "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
            "-L", OUT_DIR, "-laxs6", "-Wl,-rpath,$ORIGIN/_lib", f"-Wl,-rpath,{torch_lib}"]


def _run(cmd: list[str], what: str, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip() and verbose:
        print(r.stderr, file=sys.stderr)


def compile_ext(verbose: bool) -> str:
    obj = os.path.join(BUILD, "torch_ext.cpp.o")
    _run(ext_compile_command(obj), "torch extension compile", verbose)
    return obj


def link_ext(obj: str, verbose: bool) -> str:
    tmp = EXT_OUT + ".tmp"
    _run(ext_link_command(obj, tmp), "torch extension link", verbose)
    os.replace(tmp, EXT_OUT)
    return EXT_OUT


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def compile_one(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    # the host pass warns about the packed-fp32 target feature; drop that noise
    noise = ("packed-fp32-ops", "not a recognized feature")
    msg = "\n".join(l for l in r.stderr.splitlines() if l.strip() and not any(n in l for n in noise))
    if msg and verbose:
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs + 1) as ex:
        ext_obj = ex.submit(compile_ext, verbose)
        objs = list(ex.map(lambda s: compile_one(s, verbose), srcs))
        ext_obj = ext_obj.result()
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libaxs6.so", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    link_ext(ext_obj, verbose)
    return OUT


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--clean", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args()
    if a.clean:
        shutil.rmtree(BUILD, ignore_errors=True)
        for f in (OUT, EXT_OUT):
            if os.path.exists(f):
                os.remove(f)
        return
    print(build(a.verbose, a.jobs))


if __name__ == "__main__":
    main()
