"""Loads the in-tree native libraries; fails loudly when they are missing.

There is no CPU or PyTorch fallback: every op of this package runs the HIP
kernels of librace_mi355x.so or raises.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import pathlib
import sysconfig

PKG = pathlib.Path(__file__).resolve().parent
# RACE_MI355X_LIB_DIR names another directory holding both built libraries
# (the sanitizer stage's host-instrumented build, tests/sanitize.py); by default
# they are the in-tree ones next to this file.
LIB_DIR = pathlib.Path(os.environ.get("RACE_MI355X_LIB_DIR", PKG))
LIB_PATH = LIB_DIR / "librace_mi355x.so"
EXT_PATH = LIB_DIR / ("_race_torch" + sysconfig.get_config_var("EXT_SUFFIX"))

_ext = None
_cdll = None


class NativeLibraryMissing(RuntimeError):
    pass


def _require(path: pathlib.Path) -> None:
    if not path.exists():
        raise NativeLibraryMissing(
            f"{path.name} is not built; run `python race-attention-kernel_amd/build.py` "
            "(or __graft_entry__.build()) first")


def ext():
    """The PyTorch binding module (_race_torch)."""
    global _ext
    if _ext is None:
        # torch first: its HIP runtime (soname libamdhip64.so.7) is then the
        # one librace_mi355x.so binds to, so streams and pointers are shared.
        import torch  # noqa: F401

        _require(LIB_PATH)
        _require(EXT_PATH)
        spec = importlib.util.spec_from_file_location("_race_torch", EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ext = mod
    return _ext


def cdll() -> ctypes.CDLL:
    """librace_mi355x.so through ctypes (the raw C ABI)."""
    global _cdll
    if _cdll is None:
        import torch  # noqa: F401  (same runtime-sharing reason as ext())

        _require(LIB_PATH)
        _cdll = ctypes.CDLL(str(LIB_PATH))
    return _cdll
