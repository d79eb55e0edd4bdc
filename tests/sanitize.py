"""Host-side sanitizer stage: AddressSanitizer + UndefinedBehaviorSanitizer
over the library's CPU code, no GPU needed.

Test infrastructure (pytest does not collect it).  Builds into
race-attention-kernel_amd/_build/asan/:
  librace_mi355x.so      every .hip source with its host code instrumented
                         (hipcc, -fsanitize=... after -Xarch_host: the gfx950
                         device code is compiled as usual) -- the C ABI's
                         argument and shape validation, workspace arithmetic,
                         tile planning and the allocation-free entry point's
                         size checks
  _race_torch<suffix>.so the PyTorch binding (torch_ext.cpp), clang++ with the
                         same sanitizers, linked to the instrumented library
  liboracle.so           the test oracle, oracle/race_oracle.c (gcc, its own
                         ASan runtime)

then runs, each in its own process with the matching runtime preloaded and
any report fatal:
  tests/test_abi_cpu.py   against the instrumented C ABI and binding
                          (RACE_MI355X_LIB_DIR points the package there)
  tests/test_oracle.py and tests/test_oracle_alg1.py against the
                          instrumented oracle (RACE_ORACLE_LIB)

The reference runs compute-sanitizer over small GPU cases
(infra/sanitize_cases.py:49-59); device-side sanitizers are not available on
the GPU pool this build runs on, so the stage covers the host side only.

Usage: python tests/sanitize.py [-v]   (exit status 0 = clean)
"""
from __future__ import annotations

import concurrent.futures
import glob
import os
import pathlib
import subprocess
import sys
import sysconfig

REPO = pathlib.Path(__file__).resolve().parents[1]
PKG = REPO / "race-attention-kernel_amd"
sys.path.insert(0, str(PKG))
import build as pkg_build  # noqa: E402  (race-attention-kernel_amd/build.py)

OUT = pkg_build.BUILD_DIR / "asan"
LLVM = pkg_build.ROCM / "llvm" / "bin"
SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all",
       "-fno-omit-frame-pointer", "-g"]


def clang_asan_runtime() -> str:
    hits = sorted(glob.glob(str(pkg_build.ROCM / "llvm" / "lib" / "clang" / "*" / "lib" / "linux" /
                                "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise RuntimeError("clang's shared ASan runtime was not found under ROCm's llvm")
    return hits[-1]


def gcc_asan_runtime() -> str:
    return subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                          check=True).stdout.strip()


def build_library(verbose: bool) -> None:
    objs = []
    host_san = []
    for flag in SAN:
        host_san += ["-Xarch_host", flag]

    def one(src: pathlib.Path) -> pathlib.Path:
        obj = OUT / (src.stem + ".o")
        pkg_build._run([pkg_build.HIPCC, *pkg_build.HIP_FLAGS, *host_san, "-c", str(src), "-o", str(obj)],
                       verbose)
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(one, pkg_build.hip_sources()))
    pkg_build._run([pkg_build.HIPCC, f"--offload-arch={pkg_build.ARCH}", "-shared", "-fPIC",
                    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                    "-shared-libsan", "-o", str(OUT / pkg_build.LIB_NAME), *map(str, objs),
                    "-Wl,-soname," + pkg_build.LIB_NAME], verbose)


def build_binding(verbose: bool) -> None:
    import torch
    from torch.utils import cpp_extension

    torch_lib = pathlib.Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths(device_type="cuda")]
    incs += [f"-I{sysconfig.get_paths()['include']}", f"-I{pkg_build.INCLUDE}"]
    pkg_build._run([
        str(LLVM / "clang++"), "-O1", "-std=c++17", "-fPIC", "-shared", *SAN, "-shared-libsan",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={pkg_build.EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *incs, str(pkg_build.CSRC / "torch_ext.cpp"),
        "-o", str(OUT / pkg_build.ext_filename()),
        f"-L{OUT}", "-lrace_mi355x", f"-L{torch_lib}",
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ], verbose)


def build_oracle(verbose: bool) -> None:
    pkg_build._run(["gcc", "-O1", "-fPIC", "-fopenmp", "-std=c11", "-Wall", "-Wextra", *SAN, "-shared",
                    "-o", str(OUT / "liboracle.so"), str(REPO / "oracle" / "race_oracle.c")], verbose)


def run_pytest(files: list[str], env_extra: dict, verbose: bool) -> int:
    env = dict(os.environ)
    env.update(env_extra)
    # Python and torch are not instrumented: leaks at exit are theirs, and the
    # runtime is preloaded because the interpreter was not linked with it.
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1:detect_odr_violation=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu", *files]
    print("$", " ".join(f"{k}={v}" for k, v in env_extra.items()), " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, cwd=REPO, env=env, capture_output=not verbose, text=True)
    if not verbose:
        tail = (proc.stdout + proc.stderr).strip().splitlines()[-15:]
        print("\n".join(tail), flush=True)
    return proc.returncode


def instrumented(lib: pathlib.Path) -> bool:
    """The library calls into the ASan runtime (its checks were compiled in)."""
    syms = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True, text=True,
                          check=True).stdout
    return "__asan_report_" in syms and "__ubsan_handle_" in syms


PREFLIGHT = """
import sys
sys.path.insert(0, {repo!r})
import __graft_entry__ as entry
race = entry.load_package()
race._lib.cdll(); race._lib.ext()
maps = open('/proc/self/maps').read()
for name in ('librace_mi355x.so', '_race_torch'):
    paths = {{l.split()[-1] for l in maps.splitlines() if name in l}}
    assert paths and all(p.startswith({out!r}) for p in paths), (name, paths)
print('preflight: the instrumented C ABI and binding are the ones loaded')
"""


def main() -> int:
    verbose = "-v" in sys.argv
    OUT.mkdir(parents=True, exist_ok=True)
    build_library(verbose)
    build_binding(verbose)
    build_oracle(verbose)
    for lib in (OUT / pkg_build.LIB_NAME, OUT / pkg_build.ext_filename(), OUT / "liboracle.so"):
        if not instrumented(lib):
            print(f"{lib.name} carries no sanitizer checks", flush=True)
            return 1
    print("built", OUT, flush=True)
    env = dict(os.environ, LD_PRELOAD=clang_asan_runtime(), RACE_MI355X_LIB_DIR=str(OUT),
               ASAN_OPTIONS="detect_leaks=0")
    pre = subprocess.run([sys.executable, "-c", PREFLIGHT.format(repo=str(REPO), out=str(OUT))], env=env,
                         capture_output=True, text=True)
    print((pre.stdout + pre.stderr).strip().splitlines()[-1], flush=True)
    if pre.returncode != 0:
        return 1
    rc = run_pytest(["tests/test_abi_cpu.py"],
                    {"LD_PRELOAD": clang_asan_runtime(), "RACE_MI355X_LIB_DIR": str(OUT)}, verbose)
    rc2 = run_pytest(["tests/test_oracle.py", "tests/test_oracle_alg1.py"],
                     {"LD_PRELOAD": gcc_asan_runtime(), "RACE_ORACLE_LIB": str(OUT / "liboracle.so")},
                     verbose)
    ok = rc == 0 and rc2 == 0
    print("sanitizer stage:", "clean" if ok else f"FAILED (C ABI rc={rc}, oracle rc={rc2})", flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
