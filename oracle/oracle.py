"""CPU oracle for per-bucket RACE attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.  The product path (the HIP library and its Python op)
never calls it and has no CPU fallback.

What is here, and which reference lines each piece restates
(paths relative to the reference repository):

* ``causal_recurrence`` / ``causal_chunked`` / ``causal_tiled`` /
  ``noncausal_fwd`` / ``noncausal_bwd`` -- ctypes wrappers over
  ``race_oracle.c`` (fp64 accumulation).  The recurrence follows
  src/race_fused_fwd.cu:131-146 and src/test_kernel_math.py:32-39; the
  chunked form src/race_chunked.py:41-63; the tiled form the three-launch
  decomposition of src/causal_v2/kernels/race_causal_fwd.h:23-27 with the
  per-bucket function of src/causal_v2/reference.py:144-159.
* ``causal_tail`` -- the last outputs of long streams: the state before them
  summed in fp64 blocks, then ``causal_recurrence`` from it (the chunk
  identity); for checks at lengths the per-token scan of a whole stream
  would take minutes over.
* ``cumsum_bmm`` -- numpy transcription of the unchunked composition of
  src/race_baseline.py:45-51 (cumsum, broadcast product, cumsum, divide,
  bmm), in a chosen dtype.  Memory O(N*T*S*d): small T only.
* ``dense_causal`` -- the same function as a T x T masked matrix,
  out = M v with M[i, j] = [j <= i] * sum_s q[i,s] k[j,s] / (A[i,s] + eps).
  A different evaluation order from every other form; small T only.
* ``torch_reference_path`` -- the reference's CPU path as torch ops in fp32
  (src/race_baseline.py:45-51 verbatim in semantics).  It is the timed CPU
  baseline of bench.py and the fp32 comparison point of the tests.
* ``torch_noncausal_autograd`` -- torch.autograd on the non-causal formula
  (analysis/hot-path.md:157-162), the oracle the non-causal benchmark names for the
  gradients.
* ``hash_probs`` -- numpy restatement (fp64) of the hashing that produces the
  probabilities, src/race_baseline.py:41-44; ``hash_probs_product_form`` is
  the same function through the product identity softmax_r(sum_k u_k s_rk) =
  prod_k sigmoid(2 u_k s_rk), an independent evaluation that pins it.
* ``alg1_causal`` -- the causal forward with the hashing inside and one
  global normalization per query (paper Algorithm 1 made causal), fp64
  (race_oracle.c), following src/causal_v2/reference.py:100-128 with the
  softmax feature map of src/noncausal/reference.py:89-100; ``perbucket=True``
  is the per-bucket bridge of src/causal_v2/reference.py:144-159.  Pinned by
  ``alg1_dense`` (the masked T x T form of src/causal_v2/reference.py:131-141),
  ``alg1_features(form="bernoulli")`` (the product form of
  src/noncausal/reference.py:103-125), the closed forms T = 1 and constant V,
  and the bridge to ``hash_probs`` + ``causal_recurrence`` at beta = 1/sqrt(d).
* ``causal_bwd`` -- the closed-form VJP of the causal function (race_oracle.c,
  fp64).  The reference has no causal backward kernel; its outline is
  docs/causal_v2_design.md:689-742.  ``torch_causal_autograd`` is
  torch.autograd through the cumsum composition of src/race_baseline.py:45-51
  in fp64, the independent check of it.

Layouts: probsQ/probsK [N, T, S] (S = L*R, table-major), V/out [N, T, d].
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

EPS = 1e-6  # src/race_baseline.py:47

_HERE = pathlib.Path(__file__).resolve().parent
# RACE_ORACLE_LIB names another build of race_oracle.c to load instead (the
# sanitizer stage, tests/sanitize.py, sets it).
_LIB_OVERRIDE = os.environ.get("RACE_ORACLE_LIB")
_LIB_PATH = pathlib.Path(_LIB_OVERRIDE) if _LIB_OVERRIDE else _HERE / "liboracle.so"
_lib = None


def build(force: bool = False) -> pathlib.Path:
    """Compile liboracle.so with the Makefile beside this file."""
    if _LIB_OVERRIDE:
        return _LIB_PATH
    if force or not _LIB_PATH.exists() or (
        _LIB_PATH.stat().st_mtime < (_HERE / "race_oracle.c").stat().st_mtime
    ):
        subprocess.run(["make", "-s", "-C", str(_HERE), "-B" if force else "all"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        f64p = ctypes.POINTER(ctypes.c_double)
        i64 = ctypes.c_int64
        d = ctypes.c_double
        i = ctypes.c_int
        lib.race_oracle_causal_recurrence.argtypes = [f32p, f32p, f32p, f64p, f64p, f64p, i64, i64, i64, i64, d, i]
        lib.race_oracle_causal_chunked.argtypes = [f32p, f32p, f32p, f64p, f64p, i64, i64, i64, i64, d, i64, i]
        lib.race_oracle_causal_tiled.argtypes = [f32p, f32p, f32p, f64p, f64p, f64p, i64, i64, i64, i64, d, i64, i64, i]
        lib.race_oracle_noncausal_fwd.argtypes = [f32p, f32p, f32p, f64p, f64p, i64, i64, i64, i64, d, i]
        lib.race_oracle_noncausal_bwd.argtypes = [f32p, f32p, f32p, f32p, f64p, f64p, f64p, i64, i64, i64, i64, d, i]
        lib.race_oracle_causal_bwd.argtypes = [f32p, f32p, f32p, f32p, f64p, f64p, f64p, i64, i64, i64, i64, d, i]
        lib.race_oracle_alg1_causal.argtypes = [f32p, f32p, f32p, f32p, d, f64p, f64p, f64p, i64, i64, i64, i64,
                                                i64, i, d, i64, i]
        for name in ("race_oracle_causal_recurrence", "race_oracle_causal_chunked", "race_oracle_causal_tiled",
                     "race_oracle_noncausal_fwd", "race_oracle_noncausal_bwd", "race_oracle_causal_bwd",
                     "race_oracle_alg1_causal"):
            getattr(lib, name).restype = None
        _lib = lib
    return _lib


def _f32(x) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    return a


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _shape(q, v):
    N, T, S = q.shape
    d = v.shape[2]
    assert v.shape[:2] == (N, T)
    return N, T, S, d


def causal_recurrence(q, k, v, eps: float = EPS, nthreads: int = 0, want_state: bool = False,
                      init_state=None):
    """Per-token scan, fp64.  Returns out [N,T,d] (and the final state [N, S*d+S]).
    init_state [N, S*d+S] (B then A): the state carried in from earlier tokens
    (src/race_chunked.py:54-63); zero when None."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    N, T, S, d = _shape(q, v)
    out = np.empty((N, T, d), np.float64)
    st = np.empty((N, S * d + S), np.float64) if want_state else None
    init = None
    if init_state is not None:
        init = np.ascontiguousarray(np.asarray(init_state, dtype=np.float64))
        assert init.shape == (N, S * d + S), init.shape
    _load().race_oracle_causal_recurrence(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(out, ctypes.c_double),
        _ptr(st, ctypes.c_double) if st is not None else None,
        _ptr(init, ctypes.c_double) if init is not None else None, N, T, S, d, eps, nthreads)
    return (out, st) if want_state else out


def causal_tail(q, k, v, tail: int, eps: float = EPS, nthreads: int = 0, block: int = 1 << 20):
    """Outputs of the last ``tail`` tokens of every stream, fp64, [N, tail, d].

    The state before them, B = sum_t k_t v_t^T and A = sum_t k_t over the
    first T - tail tokens, is summed in fp64 blocks of ``block`` tokens
    (matrix products, so a stream of 2^24 tokens takes seconds); the tail
    then runs the per-token recurrence from that state, as ``init_state``
    of ``causal_recurrence`` (the chunk identity, src/race_chunked.py:54-63).
    """
    N, T, S = q.shape
    d = v.shape[2]
    t0 = T - tail
    assert 0 <= t0 <= T
    init = np.zeros((N, S * d + S), np.float64)
    for n in range(N):
        B = np.zeros((S, d), np.float64)
        A = np.zeros(S, np.float64)
        for b in range(0, t0, block):
            e = min(t0, b + block)
            kb = np.asarray(k[n, b:e], np.float64)
            B += kb.T @ np.asarray(v[n, b:e], np.float64)
            A += kb.sum(0)
        init[n, :S * d] = B.ravel()
        init[n, S * d:] = A
    return causal_recurrence(q[:, t0:], k[:, t0:], v[:, t0:], eps, nthreads, init_state=init)


def causal_chunked(q, k, v, chunk: int, eps: float = EPS, nthreads: int = 0):
    """Carried-state chunked form (chunk identity), fp64."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    N, T, S, d = _shape(q, v)
    out = np.empty((N, T, d), np.float64)
    _load().race_oracle_causal_chunked(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(out, ctypes.c_double),
        None, N, T, S, d, eps, chunk, nthreads)
    return out


def causal_tiled(q, k, v, tile: int, chunk: int, eps: float = EPS, nthreads: int = 0):
    """The GPU decomposition in fp64.  Returns (out, prefix_states [N,tiles,S*d+S], final [N,S*d+S])."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    N, T, S, d = _shape(q, v)
    tiles = -(-T // tile)
    out = np.empty((N, T, d), np.float64)
    pref = np.empty((N, tiles, S * d + S), np.float64)
    fin = np.empty((N, S * d + S), np.float64)
    _load().race_oracle_causal_tiled(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(out, ctypes.c_double),
        _ptr(pref, ctypes.c_double), _ptr(fin, ctypes.c_double), N, T, S, d, eps, tile, chunk, nthreads)
    return out, pref, fin


def noncausal_fwd(q, k, v, eps: float = EPS, nthreads: int = 0):
    """Non-causal forward, fp64.  Returns (out [N,T,d], state [N, S*d+S] = (B, A))."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    N, T, S, d = _shape(q, v)
    out = np.empty((N, T, d), np.float64)
    st = np.empty((N, S * d + S), np.float64)
    _load().race_oracle_noncausal_fwd(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(out, ctypes.c_double),
        _ptr(st, ctypes.c_double), N, T, S, d, eps, nthreads)
    return out, st


def noncausal_bwd(q, k, v, g, eps: float = EPS, nthreads: int = 0):
    """Closed-form VJP of the non-causal forward, fp64.  Returns (dq, dk, dv)."""
    q, k, v, g = _f32(q), _f32(k), _f32(v), _f32(g)
    N, T, S, d = _shape(q, v)
    dq = np.empty((N, T, S), np.float64)
    dk = np.empty((N, T, S), np.float64)
    dv = np.empty((N, T, d), np.float64)
    _load().race_oracle_noncausal_bwd(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(g, ctypes.c_float),
        _ptr(dq, ctypes.c_double), _ptr(dk, ctypes.c_double), _ptr(dv, ctypes.c_double), N, T, S, d, eps, nthreads)
    return dq, dk, dv


def causal_bwd(q, k, v, g, eps: float = EPS, nthreads: int = 0):
    """Closed-form VJP of the causal forward, fp64.  Returns (dq, dk, dv)."""
    q, k, v, g = _f32(q), _f32(k), _f32(v), _f32(g)
    N, T, S, d = _shape(q, v)
    dq = np.empty((N, T, S), np.float64)
    dk = np.empty((N, T, S), np.float64)
    dv = np.empty((N, T, d), np.float64)
    _load().race_oracle_causal_bwd(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(g, ctypes.c_float),
        _ptr(dq, ctypes.c_double), _ptr(dk, ctypes.c_double), _ptr(dv, ctypes.c_double), N, T, S, d, eps, nthreads)
    return dq, dk, dv


def cumsum_bmm(q, k, v, eps: float = EPS, dtype=np.float64):
    """src/race_baseline.py:45-51 transcribed to numpy, in ``dtype``.

    A_pref = cumsum(k); B_pref = cumsum(k[..., None] * v[:, :, None]);
    E_pref = B_pref / (A_pref[..., None] + eps); out = q . E_pref.
    """
    q, k, v = (np.asarray(x, dtype=dtype) for x in (q, k, v))
    a_pref = np.cumsum(k, axis=1)
    b_pref = np.cumsum(k[..., :, None] * v[..., None, :], axis=1)
    e_pref = b_pref / (a_pref[..., None] + dtype(eps))
    return np.einsum("nts,ntsc->ntc", q, e_pref)


def dense_causal(q, k, v, eps: float = EPS):
    """T x T masked-matrix form in fp64 (small T): out = M v."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    N, T, S = q.shape
    a_pref = np.cumsum(k, axis=1)                    # [N,T,S]
    w = q / (a_pref + eps)                           # [N,T,S]
    m = np.einsum("nis,njs->nij", w, k)              # [N,T,T]
    m = m * np.tril(np.ones((T, T)))[None]
    return m @ v


def torch_reference_path(q, k, v, eps: float = EPS):
    """The reference's CPU path (src/race_baseline.py:45-51) as fp32 torch ops.

    q, k: [N, T, S] float32 CPU tensors; v: [N, T, d].  Returns [N, T, d] fp32.
    """
    import torch

    N, T, S = q.shape
    d = v.shape[2]
    a_pref = k.cumsum(dim=1)
    b_pref = (k.unsqueeze(-1) * v.unsqueeze(2)).cumsum(dim=1)
    e_pref = b_pref.div(a_pref.unsqueeze(-1).add(eps))
    return torch.bmm(q.reshape(N * T, 1, S), e_pref.contiguous().view(N * T, S, d)).view(N, T, d)


def torch_noncausal_reference(q, k, v, eps: float = EPS):
    """analysis/hot-path.md:157-162 as torch ops (differentiable)."""
    import torch

    b_sum = k.transpose(1, 2).bmm(v)                 # [N,S,d]
    a = k.sum(1)                                     # [N,S]
    e = b_sum / (a.unsqueeze(-1) + eps)
    return q.bmm(e)


def torch_noncausal_autograd(q, k, v, g, eps: float = EPS):
    """Gradients of the non-causal formula by torch.autograd in fp64."""
    import torch

    qt, kt, vt = (torch.as_tensor(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v))
    gt = torch.as_tensor(np.asarray(g, np.float64))
    out = torch_noncausal_reference(qt, kt, vt, eps)
    dq, dk, dv = torch.autograd.grad(out, (qt, kt, vt), gt)
    return out.detach().numpy(), dq.numpy(), dk.numpy(), dv.numpy()


def torch_causal_reference(q, k, v, eps: float = EPS):
    """src/race_baseline.py:45-51 as differentiable torch ops (any dtype)."""
    import torch

    N, T, S = q.shape
    d = v.shape[2]
    a_pref = k.cumsum(dim=1)
    b_pref = (k.unsqueeze(-1) * v.unsqueeze(2)).cumsum(dim=1)
    e_pref = b_pref / (a_pref.unsqueeze(-1) + eps)
    return (q.unsqueeze(-1) * e_pref).sum(2)


def torch_causal_autograd(q, k, v, g, eps: float = EPS):
    """Gradients of the causal function by torch.autograd in fp64 (small T:
    the composition holds [N, T, S, d] tensors)."""
    import torch

    qt, kt, vt = (torch.as_tensor(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v))
    gt = torch.as_tensor(np.asarray(g, np.float64))
    out = torch_causal_reference(qt, kt, vt, eps)
    dq, dk, dv = torch.autograd.grad(out, (qt, kt, vt), gt)
    return out.detach().numpy(), dq.numpy(), dk.numpy(), dv.numpy()


def corners(K: int) -> np.ndarray:
    """[2^K, K] corners in itertools.product([-1, 1], repeat=K) order
    (src/race_baseline.py:28-30): s[r, k] = +1 iff bit K-1-k of r is set."""
    r = np.arange(1 << K)[:, None]
    return np.where((r >> (K - 1 - np.arange(K))[None, :]) & 1, 1.0, -1.0)


def hash_probs(x, planes_T, L: int, K: int):
    """src/race_baseline.py:41-44 in fp64: softmax over the corners of
    tanh(x planes_T) / sqrt(d_k) projected on the corners.  x [..., d_k] ->
    [..., L, 2^K]."""
    x = np.asarray(x, np.float64)
    dk = x.shape[-1]
    proj = (x @ np.asarray(planes_T, np.float64)).reshape(*x.shape[:-1], L, K)
    logits = (np.tanh(proj) / np.sqrt(dk)) @ corners(K).T
    logits = logits - logits.max(-1, keepdims=True)
    e = np.exp(logits)
    return e / e.sum(-1, keepdims=True)


def torch_hash_probs(x, planes_T, L: int, K: int):
    """src/race_baseline.py:41-44 as differentiable torch ops (any dtype):
    softmax over the 2^K corners of tanh(x planes_T) / sqrt(d_k) projected on
    the corners.  x [..., d_k] -> [..., L, 2^K]."""
    import torch

    dk = x.shape[-1]
    proj = (x @ planes_T).reshape(*x.shape[:-1], L, K)
    corner = torch.as_tensor(corners(K), dtype=x.dtype)     # [R, K]
    return torch.softmax((torch.tanh(proj) / np.sqrt(dk)) @ corner.T, dim=-1)


def torch_module_autograd(k_rows, q_rows, v, planes_T, L: int, K: int, g, eps: float = EPS):
    """BatchedACE's hashing and causal hot span (src/race_baseline.py:41-51) in
    fp64 torch, and its gradients w.r.t. the K, Q and V rows for upstream g
    (small T: the composition holds [N, T, S, d] tensors).  Returns (out, dK,
    dQ, dV) as numpy."""
    import torch

    kt, qt, vt = (torch.as_tensor(np.asarray(x, np.float64)).requires_grad_(True)
                  for x in (k_rows, q_rows, v))
    pt = torch.as_tensor(np.asarray(planes_T, np.float64))
    pk = torch_hash_probs(kt, pt, L, K).flatten(-2)
    pq = torch_hash_probs(qt, pt, L, K).flatten(-2)
    out = torch_causal_reference(pq, pk, vt, eps)
    dk, dq, dv = torch.autograd.grad(out, (kt, qt, vt), torch.as_tensor(np.asarray(g, np.float64)))
    return out.detach().numpy(), dk.numpy(), dq.numpy(), dv.numpy()


def hash_probs_product_form(x, planes_T, L: int, K: int):
    """The same probabilities as prod_k sigmoid(2 u_k s_{r,k})."""
    x = np.asarray(x, np.float64)
    dk = x.shape[-1]
    u = np.tanh((x @ np.asarray(planes_T, np.float64)).reshape(*x.shape[:-1], L, K)) / np.sqrt(dk)
    s = corners(K)                                          # [R, K]
    z = 2.0 * u[..., None, :] * s                           # [..., L, R, K]
    return (1.0 / (1.0 + np.exp(-z))).prod(-1)


def alg1_causal(q, k, v, W, beta: float, *, perbucket: bool = False, eps: float = EPS, tile: int = 0,
                want_state: bool = False, nthreads: int = 0):
    """Algorithm 1 with hashing, fp64 (race_oracle.c).  q, k, v [N, T, D]
    (bf16 values widened exactly), W [L, P, D].  Returns out [N, T, D], plus
    (prefix [N, tiles, S*D+S], final [N, S*D+S]) when tile > 0 or want_state
    (prefix is None without a tile)."""
    q, k, v, W = _f32(q), _f32(k), _f32(v), _f32(W)
    N, T, D = q.shape
    L, P = W.shape[0], W.shape[1]
    assert W.shape[2] == D and k.shape == q.shape and v.shape == q.shape
    S = L << P
    rec = S * D + S
    out = np.empty((N, T, D), np.float64)
    tiles = -(-T // tile) if tile > 0 else 0
    pref = np.empty((N, tiles, rec), np.float64) if tile > 0 else None
    fin = np.empty((N, rec), np.float64) if (want_state or tile > 0) else None
    _load().race_oracle_alg1_causal(
        _ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float), _ptr(W, ctypes.c_float),
        float(beta), _ptr(out, ctypes.c_double), _ptr(pref, ctypes.c_double) if pref is not None else None,
        _ptr(fin, ctypes.c_double) if fin is not None else None, N, T, D, L, P, int(perbucket), eps,
        int(tile), nthreads)
    if fin is None:
        return out
    return out, pref, fin


def alg1_features(x, W, beta: float, form: str = "softmax"):
    """Phi(x) [..., L*2^P] in fp64: the direct softmax over the corners
    (src/noncausal/reference.py:89-100) or the Bernoulli product
    prod_p sigmoid(+-2 beta u_p), built plane by plane with plane 0 as the
    most significant bit (src/noncausal/reference.py:103-125)."""
    x = np.asarray(x, np.float64)
    W = np.asarray(W, np.float64)
    L, P, _ = W.shape
    u = np.tanh(np.einsum("...d,lpd->...lp", x, W))
    if form == "softmax":
        logits = beta * (u @ corners(P).T)
        logits = logits - logits.max(-1, keepdims=True)
        e = np.exp(logits)
        phi = e / e.sum(-1, keepdims=True)
    else:
        plus = 1.0 / (1.0 + np.exp(-2.0 * beta * u))
        minus = 1.0 / (1.0 + np.exp(2.0 * beta * u))
        phi = np.ones(u.shape[:-1] + (1,))
        for p in range(P):
            phi = np.stack([phi * minus[..., p:p + 1], phi * plus[..., p:p + 1]], -1).reshape(
                *u.shape[:-1], -1)
    return phi.reshape(*x.shape[:-1], L * (1 << P))


def alg1_dense(q, k, v, W, beta: float):
    """Algorithm 1 as masked attention with kernel k_ij = <Phi(q_i), Phi(k_j)>,
    j <= i (src/causal_v2/reference.py:131-141), fp64; tiny T only."""
    fq, fk = alg1_features(q, W, beta), alg1_features(k, W, beta)
    T = fq.shape[-2]
    scores = fq @ np.swapaxes(fk, -1, -2) * np.tril(np.ones((T, T)))
    den = scores.sum(-1, keepdims=True)
    num = scores @ np.asarray(v, np.float64)
    return np.where(den == 0, 0.0, num / np.where(den == 0, 1.0, den))
