"""In-tree build of the MI355X RACE attention library.

Produces, next to this file:
  librace_mi355x.so      the C ABI (include/race_mi355x.h) and its gfx950 HIP
                         kernels, built by hipcc
  _race_torch<suffix>.so the PyTorch-ROCm binding, linked to librace_mi355x.so

Every HIP source is compiled for gfx950 only, with packed fp32 vector ops
disabled in device code (-Xclang -target-feature -Xclang -packed-fp32-ops).

Usage: python race-attention-kernel_amd/build.py [-v]
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys
import sysconfig

PKG = pathlib.Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = PKG / "_build"
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

LIB_NAME = "librace_mi355x.so"
EXT_NAME = "_race_torch"

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def hip_sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def ext_filename() -> str:
    return EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only target feature and says so.
    noise = ("packed-fp32-ops", "not a recognized feature", "warning generated")
    text = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines()
                     if l.strip() and not any(n in l for n in noise))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{text}")
    if verbose and text:
        print(text, flush=True)


def build_hip_library(verbose: bool = False, jobs: int = 8) -> pathlib.Path:
    """hipcc each .hip to an object, then link librace_mi355x.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = hip_sources()
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    headers = list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h"))

    def compile_one(src_obj):
        src, obj = src_obj
        _run([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)], verbose)

    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    out = PKG / LIB_NAME
    tmp = BUILD_DIR / (LIB_NAME + ".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          "-Wl,-soname," + LIB_NAME], verbose)
    os.replace(tmp, out)
    del headers
    return out


def build_torch_extension(verbose: bool = False) -> pathlib.Path:
    """g++ the pybind11/PyTorch binding against torch's headers and librace_mi355x.so."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = pathlib.Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths(device_type="cuda")]
    incs += [f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}"]
    out = PKG / ext_filename()
    tmp = BUILD_DIR / (ext_filename() + ".tmp")
    BUILD_DIR.mkdir(exist_ok=True)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *incs, str(CSRC / "torch_ext.cpp"), "-o", str(tmp),
        f"-L{PKG}", "-lrace_mi355x", f"-L{torch_lib}",
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    if not shutil.which(HIPCC) and not pathlib.Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_hip_library(verbose)
    build_torch_extension(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", PKG / LIB_NAME, "and", PKG / ext_filename())
