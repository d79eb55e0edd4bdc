"""ctypes view of the C ABI in include/race_mi355x.h.

This is the binding a maintainer of the reference would add to call the
library without the PyTorch extension: plain pointers, sizes and a stream
handle.  The declarations mirror the header one to one.
"""
from __future__ import annotations

import ctypes

from . import _lib

RACE_SUCCESS = 0
RACE_ERROR_INVALID_VALUE = 1
RACE_ERROR_SCRATCH_TOO_SMALL = 2
RACE_ERROR_SINGLE_PASS_GAVE_UP = 4096
RACE_NOALLOC_SCRATCH_BYTES = 32 << 20
RACE_F32 = 0
RACE_BF16 = 1
RACE_KERNEL_AUTO = 0
RACE_KERNEL_VALU = 1
RACE_KERNEL_MFMA = 2
RACE_KERNEL_MFMA_WG = 3
RACE_KERNEL_DECODE = 4
RACE_KERNEL_SINGLE = 5
RACE_KERNEL_MFMA_PRECISE = 6
RACE_DECODE_TOKENS = 16
RACE_SUB_CHUNK_TOKENS = 64
RACE_ALG1_FP32 = 0
RACE_ALG1_BF16 = 1
RACE_ALG1_SUB_CHUNK_TOKENS = 64
RACE_ALG1_MAX_AUTO_TILE = 4096

EXPORTED_SYMBOLS = (
    "race_abi_version",
    "race_status_string",
    "race_shape_supported",
    "race_select_tile_tokens",
    "race_fwd_workspace_bytes",
    "race_fwd",
    "race_fwd_profiled",
    "race_fwd_noalloc",
    "race_fwd_single_status",
    "race_single_pass_test_give_up",
    "race_fwd_carry_workspace_bytes",
    "race_fwd_carry",
    "race_fwd_carry_profiled",
    "race_noncausal_bwd_workspace_bytes",
    "race_noncausal_bwd",
    "race_causal_bwd_workspace_bytes",
    "race_causal_bwd_from_records_workspace_bytes",
    "race_causal_bwd",
    "race_causal_bwd_from_records",
    "race_noncausal_bwd_profiled",
    "race_causal_bwd_profiled",
    "race_hash_probs",
    "race_hash_probs_bwd",
    "race_hashed_fwd_workspace_bytes",
    "race_hashed_fwd",
    "race_hashed_fwd_profiled",
    "race_alg1_shape_supported",
    "race_alg1_output_lds_bytes",
    "race_alg1_select_tile_tokens",
    "race_alg1_workspace_bytes",
    "race_alg1_fwd",
    "race_alg1_fwd_carry",
    "race_alg1_fwd_profiled",
)


class RaceAlg1Shape(ctypes.Structure):
    _fields_ = [
        ("batch_heads", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("head_dim", ctypes.c_int32),
        ("num_planes", ctypes.c_int32),
        ("num_tables", ctypes.c_int32),
    ]


class RaceShape(ctypes.Structure):
    _fields_ = [
        ("num_streams", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("num_tables", ctypes.c_int32),
        ("num_buckets", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


class RaceOptions(ctypes.Structure):
    _fields_ = [("tile_tokens", ctypes.c_int32), ("kernel", ctypes.c_int32)]


_configured = False


def lib() -> ctypes.CDLL:
    global _configured
    L = _lib.cdll()
    if not _configured:
        vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
        shp, opp = ctypes.POINTER(RaceShape), ctypes.POINTER(RaceOptions)
        L.race_abi_version.argtypes = []
        L.race_abi_version.restype = i32
        L.race_status_string.argtypes = [i32]
        L.race_status_string.restype = ctypes.c_char_p
        L.race_shape_supported.argtypes = [shp, ctypes.POINTER(i32), ctypes.POINTER(i32)]
        L.race_select_tile_tokens.argtypes = [shp, i32, opp, ctypes.POINTER(i32)]
        L.race_fwd_workspace_bytes.argtypes = [shp, i32, opp, ctypes.POINTER(sz),
                                               ctypes.POINTER(i64), ctypes.POINTER(i64)]
        L.race_fwd.argtypes = [vp, vp, vp, vp, vp, shp, i32, opp, vp, sz, vp]
        L.race_fwd_profiled.argtypes = [vp, vp, vp, vp, vp, shp, i32, opp, vp, sz, vp,
                                        ctypes.POINTER(vp), i32, ctypes.POINTER(i32)]
        L.race_fwd_noalloc.argtypes = [vp, vp, vp, vp, vp, shp, i32, opp, vp]
        L.race_fwd_single_status.argtypes = [shp, opp, vp, sz, vp]
        L.race_single_pass_test_give_up.argtypes = [i32]
        L.race_fwd_carry_workspace_bytes.argtypes = [shp, opp, ctypes.POINTER(sz)]
        L.race_fwd_carry.argtypes = [vp, vp, vp, vp, vp, vp, shp, opp, vp, sz, vp]
        L.race_fwd_carry_profiled.argtypes = [vp, vp, vp, vp, vp, vp, shp, opp, vp, sz, vp, vp, i32,
                                              ctypes.POINTER(i32)]
        L.race_noncausal_bwd_workspace_bytes.argtypes = [shp, opp, ctypes.POINTER(sz)]
        L.race_noncausal_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, shp, opp, vp, sz, vp]
        L.race_causal_bwd_workspace_bytes.argtypes = [shp, opp, ctypes.POINTER(sz)]
        L.race_causal_bwd_from_records_workspace_bytes.argtypes = [shp, opp, ctypes.POINTER(sz)]
        L.race_causal_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, shp, opp, vp, sz, vp]
        L.race_causal_bwd_from_records.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, shp, opp, vp,
                                                   sz, vp]
        L.race_noncausal_bwd_profiled.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, shp, opp, vp, sz,
                                                  vp, ctypes.POINTER(vp), i32, ctypes.POINTER(i32)]
        L.race_causal_bwd_profiled.argtypes = [vp, vp, vp, vp, vp, vp, vp, shp, opp, vp, sz, vp,
                                               ctypes.POINTER(vp), i32, ctypes.POINTER(i32)]
        L.race_hash_probs.argtypes = [vp, vp, vp, i64, i32, i32, i32, i32, vp]
        L.race_hash_probs_bwd.argtypes = [vp, vp, vp, vp, i64, i32, i32, i32, i32, vp]
        L.race_hashed_fwd_workspace_bytes.argtypes = [shp, i32, opp, ctypes.POINTER(sz),
                                                      ctypes.POINTER(i64), ctypes.POINTER(i64)]
        L.race_hashed_fwd.argtypes = [vp, vp, vp, vp, vp, vp, shp, i32, opp, vp, sz, vp]
        L.race_hashed_fwd_profiled.argtypes = [vp, vp, vp, vp, vp, vp, shp, i32, opp, vp, sz, vp,
                                               ctypes.POINTER(vp), i32, ctypes.POINTER(i32)]
        a1 = ctypes.POINTER(RaceAlg1Shape)
        L.race_alg1_shape_supported.argtypes = [a1, ctypes.POINTER(i32)]
        L.race_alg1_output_lds_bytes.argtypes = [a1, i32, ctypes.POINTER(sz)]
        L.race_alg1_select_tile_tokens.argtypes = [a1, i32, ctypes.POINTER(i32)]
        L.race_alg1_workspace_bytes.argtypes = [a1, i32, i32, ctypes.POINTER(sz), ctypes.POINTER(i64),
                                                ctypes.POINTER(i64)]
        L.race_alg1_fwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, a1, i32, i32, vp, sz, vp]
        L.race_alg1_fwd_carry.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, a1, i32, i32, vp, sz, vp]
        L.race_alg1_fwd_profiled.argtypes = [vp, vp, vp, vp, vp, vp, vp, a1, i32, i32, vp, sz, vp,
                                             ctypes.POINTER(vp), i32, ctypes.POINTER(i32)]
        for name in EXPORTED_SYMBOLS[2:]:
            getattr(L, name).restype = i32
        _configured = True
    return L


def shape(N: int, T: int, L: int, R: int, d: int, dtype: int = RACE_F32) -> RaceShape:
    return RaceShape(N, T, L, R, d, dtype)


def options(tile_tokens: int = 0, kernel: int = RACE_KERNEL_AUTO) -> RaceOptions:
    return RaceOptions(tile_tokens, kernel)


def status_string(status: int) -> str:
    return lib().race_status_string(status).decode()


def shape_supported(sh: RaceShape) -> tuple[bool, bool]:
    ok, mf = ctypes.c_int32(0), ctypes.c_int32(0)
    st = lib().race_shape_supported(ctypes.byref(sh), ctypes.byref(ok), ctypes.byref(mf))
    if st != RACE_SUCCESS:
        raise RuntimeError(status_string(st))
    return bool(ok.value), bool(mf.value)


def fwd_workspace_bytes(sh: RaceShape, causal: bool, opts: RaceOptions | None = None):
    """(status, bytes, tiles, record_floats)."""
    b, t, r = ctypes.c_size_t(0), ctypes.c_int64(0), ctypes.c_int64(0)
    st = lib().race_fwd_workspace_bytes(ctypes.byref(sh), int(causal),
                                        ctypes.byref(opts) if opts is not None else None,
                                        ctypes.byref(b), ctypes.byref(t), ctypes.byref(r))
    return st, b.value, t.value, r.value


def fwd_noalloc(q: int, k: int, v: int, out: int, state: int | None, sh: RaceShape, causal: bool,
                opts: RaceOptions | None, stream: int) -> int:
    """race_fwd_noalloc on raw device addresses (workspace from the library's
    per-GPU scratch array); returns the status."""
    return lib().race_fwd_noalloc(q, k, v, out, state, ctypes.byref(sh), int(causal),
                                  ctypes.byref(opts) if opts is not None else None, stream)


def fwd_single_status(sh: RaceShape, opts: RaceOptions, workspace: int | None, workspace_bytes: int,
                      stream: int = 0) -> int:
    """race_fwd_single_status: waits for `stream`, then reports whether a
    bounded wait of the last one-read launch on this workspace gave up
    (workspace None: the current GPU's no-alloc scratch)."""
    return lib().race_fwd_single_status(ctypes.byref(sh), ctypes.byref(opts), workspace,
                                        workspace_bytes, stream)


def single_pass_test_give_up(on: bool) -> int:
    """race_single_pass_test_give_up: preset the one-read kernel's error word."""
    return lib().race_single_pass_test_give_up(int(bool(on)))


def hashed_fwd_workspace_bytes(sh: RaceShape, planes_per_table: int, opts: RaceOptions | None = None):
    """(status, bytes, tiles, record_floats) of race_hashed_fwd."""
    b, t, r = ctypes.c_size_t(0), ctypes.c_int64(0), ctypes.c_int64(0)
    st = lib().race_hashed_fwd_workspace_bytes(ctypes.byref(sh), planes_per_table,
                                               ctypes.byref(opts) if opts is not None else None,
                                               ctypes.byref(b), ctypes.byref(t), ctypes.byref(r))
    return st, b.value, t.value, r.value


def hashed_fwd(k: int, q: int, v: int, planes: int, out: int, state: int | None, sh: RaceShape,
               planes_per_table: int, opts: RaceOptions | None, workspace: int | None,
               workspace_bytes: int, stream: int) -> int:
    """race_hashed_fwd on raw device addresses; returns the status."""
    return lib().race_hashed_fwd(k, q, v, planes, out, state, ctypes.byref(sh), planes_per_table,
                                 ctypes.byref(opts) if opts is not None else None, workspace,
                                 workspace_bytes, stream)


def hashed_fwd_profiled(k: int, q: int, v: int, planes: int, out: int, state: int | None,
                        sh: RaceShape, planes_per_table: int, opts: RaceOptions | None,
                        workspace: int | None, workspace_bytes: int, stream: int,
                        events) -> tuple[int, int]:
    """race_hashed_fwd_profiled; ``events`` a ctypes array of hipEvent_t.  Returns (status, n_events)."""
    n = ctypes.c_int32(0)
    st = lib().race_hashed_fwd_profiled(k, q, v, planes, out, state, ctypes.byref(sh), planes_per_table,
                                        ctypes.byref(opts) if opts is not None else None, workspace,
                                        workspace_bytes, stream, events, len(events), ctypes.byref(n))
    return st, n.value


def noncausal_bwd_workspace_bytes(sh: RaceShape, opts: RaceOptions | None = None):
    b = ctypes.c_size_t(0)
    st = lib().race_noncausal_bwd_workspace_bytes(ctypes.byref(sh),
                                                  ctypes.byref(opts) if opts is not None else None,
                                                  ctypes.byref(b))
    return st, b.value


def fwd(q: int, k: int, v: int, out: int, state: int | None, sh: RaceShape, causal: bool,
        opts: RaceOptions | None, workspace: int | None, workspace_bytes: int, stream: int) -> int:
    """race_fwd on raw device addresses; returns the status."""
    return lib().race_fwd(q, k, v, out, state, ctypes.byref(sh), int(causal),
                          ctypes.byref(opts) if opts is not None else None,
                          workspace, workspace_bytes, stream)


def fwd_profiled(q: int, k: int, v: int, out: int, state: int | None, sh: RaceShape, causal: bool,
                 opts: RaceOptions | None, workspace: int | None, workspace_bytes: int, stream: int,
                 events) -> tuple[int, int]:
    """race_fwd_profiled; ``events`` is a ctypes array of hipEvent_t.  Returns (status, n_events)."""
    n = ctypes.c_int32(0)
    st = lib().race_fwd_profiled(q, k, v, out, state, ctypes.byref(sh), int(causal),
                                 ctypes.byref(opts) if opts is not None else None, workspace,
                                 workspace_bytes, stream, events, len(events), ctypes.byref(n))
    return st, n.value


def fwd_carry_workspace_bytes(sh: RaceShape, opts: RaceOptions | None = None):
    b = ctypes.c_size_t(0)
    st = lib().race_fwd_carry_workspace_bytes(ctypes.byref(sh),
                                              ctypes.byref(opts) if opts is not None else None,
                                              ctypes.byref(b))
    return st, b.value


def fwd_carry(q: int, k: int, v: int, out: int, init_state: int, state: int | None, sh: RaceShape,
              opts: RaceOptions | None, workspace: int | None, workspace_bytes: int, stream: int) -> int:
    """race_fwd_carry on raw device addresses; returns the status."""
    return lib().race_fwd_carry(q, k, v, out, init_state, state, ctypes.byref(sh),
                                ctypes.byref(opts) if opts is not None else None,
                                workspace, workspace_bytes, stream)


def fwd_carry_profiled(q: int, k: int, v: int, out: int, init_state: int, state: int | None,
                       sh: RaceShape, opts: RaceOptions | None, workspace: int | None,
                       workspace_bytes: int, stream: int, events) -> tuple[int, int]:
    """race_fwd_carry_profiled; returns (status, n_events)."""
    n = ctypes.c_int32(0)
    st = lib().race_fwd_carry_profiled(q, k, v, out, init_state, state, ctypes.byref(sh),
                                       ctypes.byref(opts) if opts is not None else None, workspace,
                                       workspace_bytes, stream, events, len(events), ctypes.byref(n))
    return st, n.value


def noncausal_bwd(q: int, k: int, v: int, g: int, state: int, dq: int | None, dk: int | None,
                  dv: int | None, sh: RaceShape, opts: RaceOptions | None, workspace: int | None,
                  workspace_bytes: int, stream: int) -> int:
    return lib().race_noncausal_bwd(q, k, v, g, state, dq, dk, dv, ctypes.byref(sh),
                                    ctypes.byref(opts) if opts is not None else None,
                                    workspace, workspace_bytes, stream)


def causal_bwd_workspace_bytes(sh: RaceShape, opts: RaceOptions | None = None):
    b = ctypes.c_size_t(0)
    st = lib().race_causal_bwd_workspace_bytes(ctypes.byref(sh),
                                               ctypes.byref(opts) if opts is not None else None,
                                               ctypes.byref(b))
    return st, b.value


def causal_bwd_from_records_workspace_bytes(sh: RaceShape, opts: RaceOptions | None = None):
    b = ctypes.c_size_t(0)
    st = lib().race_causal_bwd_from_records_workspace_bytes(
        ctypes.byref(sh), ctypes.byref(opts) if opts is not None else None, ctypes.byref(b))
    return st, b.value


def causal_bwd(q: int, k: int, v: int, g: int, dq: int | None, dk: int | None, dv: int | None,
               sh: RaceShape, opts: RaceOptions | None, workspace: int | None, workspace_bytes: int,
               stream: int) -> int:
    return lib().race_causal_bwd(q, k, v, g, dq, dk, dv, ctypes.byref(sh),
                                 ctypes.byref(opts) if opts is not None else None,
                                 workspace, workspace_bytes, stream)


def causal_bwd_from_records(q: int, k: int, v: int, g: int, fwd_records: int | None,
                            dq: int | None, dk: int | None, dv: int | None, sh: RaceShape,
                            opts: RaceOptions | None, workspace: int | None, workspace_bytes: int,
                            stream: int) -> int:
    return lib().race_causal_bwd_from_records(q, k, v, g, fwd_records, dq, dk, dv, ctypes.byref(sh),
                                              ctypes.byref(opts) if opts is not None else None,
                                              workspace, workspace_bytes, stream)


def noncausal_bwd_profiled(q, k, v, g, state, dq, dk, dv, sh: RaceShape, opts, workspace,
                           workspace_bytes: int, stream: int, events) -> tuple[int, int]:
    n = ctypes.c_int32(0)
    st = lib().race_noncausal_bwd_profiled(q, k, v, g, state, dq, dk, dv, ctypes.byref(sh),
                                           ctypes.byref(opts) if opts is not None else None,
                                           workspace, workspace_bytes, stream, events, len(events),
                                           ctypes.byref(n))
    return st, n.value


def causal_bwd_profiled(q, k, v, g, dq, dk, dv, sh: RaceShape, opts, workspace,
                        workspace_bytes: int, stream: int, events) -> tuple[int, int]:
    n = ctypes.c_int32(0)
    st = lib().race_causal_bwd_profiled(q, k, v, g, dq, dk, dv, ctypes.byref(sh),
                                        ctypes.byref(opts) if opts is not None else None,
                                        workspace, workspace_bytes, stream, events, len(events),
                                        ctypes.byref(n))
    return st, n.value


def hash_probs(x: int, planes_T: int, probs: int, rows: int, head_dim: int, num_tables: int,
               planes_per_table: int, dtype: int, stream: int) -> int:
    return lib().race_hash_probs(x, planes_T, probs, rows, head_dim, num_tables, planes_per_table,
                                 dtype, stream)


def alg1_shape(BH: int, T: int, D: int, P: int, L: int) -> RaceAlg1Shape:
    return RaceAlg1Shape(BH, T, D, P, L)


def alg1_shape_supported(sh: RaceAlg1Shape) -> bool:
    ok = ctypes.c_int32(0)
    st = lib().race_alg1_shape_supported(ctypes.byref(sh), ctypes.byref(ok))
    if st != RACE_SUCCESS:
        raise RuntimeError(status_string(st))
    return bool(ok.value)


def alg1_output_lds_bytes(sh: RaceAlg1Shape, variant: int = RACE_ALG1_FP32):
    """(status, bytes)."""
    b = ctypes.c_size_t(0)
    st = lib().race_alg1_output_lds_bytes(ctypes.byref(sh), variant, ctypes.byref(b))
    return st, b.value


def alg1_workspace_bytes(sh: RaceAlg1Shape, variant: int = RACE_ALG1_FP32, tile_tokens: int = 0):
    """(status, bytes, tiles, record_floats)."""
    b, t, r = ctypes.c_size_t(0), ctypes.c_int64(0), ctypes.c_int64(0)
    st = lib().race_alg1_workspace_bytes(ctypes.byref(sh), variant, tile_tokens, ctypes.byref(b),
                                         ctypes.byref(t), ctypes.byref(r))
    return st, b.value, t.value, r.value


def alg1_fwd(q: int, k: int, v: int, W: int, beta: int, out: int, final_state: int | None,
             sh: RaceAlg1Shape, tile_tokens: int, variant: int, workspace: int | None,
             workspace_bytes: int, stream: int) -> int:
    """race_alg1_fwd on raw device addresses; returns the status."""
    return lib().race_alg1_fwd(q, k, v, W, beta, out, final_state, ctypes.byref(sh), tile_tokens,
                               variant, workspace, workspace_bytes, stream)


def alg1_fwd_carry(q: int, k: int, v: int, W: int, beta: int, out: int, init_state: int,
                   final_state: int | None, sh: RaceAlg1Shape, tile_tokens: int, variant: int,
                   workspace: int | None, workspace_bytes: int, stream: int) -> int:
    """race_alg1_fwd_carry on raw device addresses; returns the status."""
    return lib().race_alg1_fwd_carry(q, k, v, W, beta, out, init_state, final_state, ctypes.byref(sh),
                                     tile_tokens, variant, workspace, workspace_bytes, stream)


def alg1_fwd_profiled(q, k, v, W, beta, out, final_state, sh: RaceAlg1Shape, tile_tokens: int,
                      variant: int, workspace, workspace_bytes: int, stream: int, events):
    """race_alg1_fwd_profiled; returns (status, n_events)."""
    n = ctypes.c_int32(0)
    st = lib().race_alg1_fwd_profiled(q, k, v, W, beta, out, final_state, ctypes.byref(sh), tile_tokens,
                                      variant, workspace, workspace_bytes, stream, events, len(events),
                                      ctypes.byref(n))
    return st, n.value
