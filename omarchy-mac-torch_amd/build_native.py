"""Builds, in-tree, the two native pieces of the package:

  1. libomt_hip.so, the C-ABI HIP library (csrc/, hipcc for gfx950, no torch headers: include/omt_hip.h);
  2. _native, the torch extension that registers the "omarchy_mac_torch" PrivateUse1 device on top of it
     (torch_ext/, host C++ against the installed torch-ROCm, linked to libomt_hip.so).

    python omarchy-mac-torch_amd/build_native.py [--jobs N] [--verbose] [--lib-only]

Objects go to _build/; both shared objects land in omarchy_mac_torch/ next to the Python package that loads them.
"""

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
PKG = HERE / "omarchy_mac_torch"
LIB = PKG / "libomt_hip.so"
ARCH = os.environ.get("OMT_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


COMMON = [
    "-std=c++17", "-O3", "-fPIC", "-fvisibility=hidden", f"--offload-arch={ARCH}",
    # packed FP32 VALU ops stay off (the compiler must not form v_pk_*_f32 from scalar float code)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def compile_one(src, verbose):
    obj = BUILD / (src.name + ".o")
    cmd = [hipcc(), "-x", "hip", "-c", str(src), "-o", str(obj)] + COMMON
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{r.stdout}\n{r.stderr}")
    if verbose and r.stderr.strip():
        print(r.stderr, file=sys.stderr)
    return obj


def build(jobs=None, verbose=False):
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: compile_one(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-Wl,-soname,libomt_hip.so", "-o", str(tmp)] + \
        [str(o) for o in objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"linking libomt_hip.so failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


TORCH_EXT = HERE / "torch_ext"


def build_torch_ext(verbose=False):
    """Compiles torch_ext/*.cpp with torch's extension toolchain into omarchy_mac_torch/_native.so.

    The compile runs in a child process: torch's extension loader imports what it builds, and the extension registers
    the PrivateUse1 device once per process, so the caller must stay free to import the package afterwards."""
    cmd = [sys.executable, str(pathlib.Path(__file__).resolve()), "--torch-ext-child"] + (["--verbose"] if verbose else [])
    subprocess.run(cmd, check=True)
    return PKG / "_native.so"


def _build_torch_ext_here(verbose=False):
    import torch
    import torch.utils.cpp_extension as ce

    import ctypes

    ctypes.CDLL(str(LIB), mode=ctypes.RTLD_GLOBAL)  # the build's import check resolves libomt_hip.so by SONAME
    tlib = pathlib.Path(torch.__file__).resolve().parent / "lib"
    bdir = BUILD / "torch_ext"
    bdir.mkdir(parents=True, exist_ok=True)
    ce.load(
        name="_native",
        sources=sorted(str(p) for p in TORCH_EXT.glob("*.cpp")),
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1", "-Wno-unused-function"],
        extra_include_paths=[str(ROOT / "include"), str(TORCH_EXT), "/opt/rocm/include"],
        extra_ldflags=[f"-L{tlib}", "-lc10_hip", "-ltorch_hip", "-lamdhip64", f"-L{PKG}", "-lomt_hip",
                       "-Wl,-rpath,\\$$ORIGIN"],
        build_directory=str(bdir),
        verbose=verbose,
        is_python_module=True,
    )
    out = PKG / "_native.so"
    tmp = out.with_suffix(".so.tmp")
    shutil.copyfile(bdir / "_native.so", tmp)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--lib-only", action="store_true", help="build libomt_hip.so only")
    ap.add_argument("--torch-ext-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.torch_ext_child:
        _build_torch_ext_here(args.verbose)
        sys.exit(0)
    print(build(args.jobs, args.verbose))
    if not args.lib_only:
        print(build_torch_ext(args.verbose))
