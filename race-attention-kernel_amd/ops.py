"""The drop-in op: race_fused_fwd(probsQ, probsK, V, causal).

Replaces the hot span of the reference's BatchedACE.forward
(src/race_baseline.py:45-51): given the bucket probabilities the hashing
produced (src/race_baseline.py:43-44), returns

    out[n, t] = sum_s probsQ[n, t, s] * B[n, t, s, :] / (A[n, t, s] + 1e-6)

with A, B the inclusive running sums of probsK and probsK (x) V over tokens
(causal) or their totals over the whole sequence (non-causal,
analysis/hot-path.md:157-162).  The 5-D prefix tensors of the reference never
exist: the HIP kernels carry the per-bucket state on chip.

The autograd wrapper follows the reference's non-causal op
(src/noncausal/ops.py:20-63): it saves the inputs (plus, non-causal, the
small per-bucket state), is once_differentiable, makes the incoming gradient
dense and returns only the gradients autograd asks for.  The causal backward
has no counterpart in the reference (its design outline is
docs/causal_v2_design.md:689-742); here the forward keeps its scanned tile
records (the prefix state at every tile start: (S*d + S)*4 bytes per tile,
i.e. that over the tile length per token -- 130 bytes per token at the cfg2
shape's automatic 1024-token tiles, 2 KB at S = 256, d = 128 with the
shortest 64-token tiles) and the backward starts from them instead of recomputing them.  The
reference's [N, T, S, d] prefix tensor is never formed.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _lib

KERNELS = {"auto": 0, "valu": 1, "mfma": 2, "mfma_wg": 3, "decode": 4, "single": 5, "mfma_precise": 6}


def _kernel_id(kernel: str | int) -> int:
    if isinstance(kernel, int):
        return kernel
    try:
        return KERNELS[kernel]
    except KeyError:
        raise ValueError(f"kernel must be one of {sorted(KERNELS)}, got {kernel!r}") from None


def _dense(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


class RaceFusedFunction(torch.autograd.Function):
    """out = race_fused_fwd(probsQ, probsK, V, causal) on the HIP kernels."""

    @staticmethod
    def forward(ctx, probsQ, probsK, V, causal, tile_tokens, kernel):
        needs = any(ctx.needs_input_grad[:3])
        ctx.causal = bool(causal)
        ctx.tile_tokens = int(tile_tokens)
        if needs and causal:
            # The scanned tile records (the prefix state at every tile start)
            # are kept, so the backward does not recompute them.
            out, records, tile = _lib.ext().forward_with_records(probsQ, probsK, V,
                                                                 int(tile_tokens), int(kernel))
            ctx.tile_tokens = int(tile)
            ctx.save_for_backward(probsQ, probsK, V, records)
            return out
        want_state = needs and not causal
        out, state = _lib.ext().forward(probsQ, probsK, V, bool(causal), int(tile_tokens),
                                        int(kernel), want_state)
        if needs:
            ctx.save_for_backward(probsQ, probsK, V, state)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        need_q, need_k, need_v = ctx.needs_input_grad[:3]
        if not (need_q or need_k or need_v):
            return None, None, None, None, None, None
        if ctx.causal:
            q, k, v, records = ctx.saved_tensors
            grad_out = _dense(grad_out.to(v.dtype))
            dq, dk, dv = _lib.ext().causal_backward(q, k, v, grad_out, need_q, need_k, need_v,
                                                   ctx.tile_tokens, 0, records)
            return dq, dk, dv, None, None, None
        q, k, v, state = ctx.saved_tensors
        grad_out = _dense(grad_out.to(v.dtype))
        dq, dk, dv = _lib.ext().noncausal_backward(q, k, v, grad_out, state, need_q, need_k,
                                                  need_v, ctx.tile_tokens)
        return dq, dk, dv, None, None, None


def race_fused_fwd(probsQ: torch.Tensor, probsK: torch.Tensor, V: torch.Tensor, causal: bool = True,
                   *, tile_tokens: int = 0, kernel: str | int = "auto") -> torch.Tensor:
    """Per-bucket RACE attention on MI355X.

    Args:
        probsQ, probsK: [N, T, L, R] (or [N, T, S]) bucket probabilities,
            float32 or bfloat16, on a ROCm device, contiguous.
        V: [N, T, d] values of the same dtype and device.
        causal: inclusive running sums (True) or full-sequence sums (False).
        tile_tokens: 0 for automatic, else a positive multiple of 64 (the
            tokens each workgroup of the causal output pass owns).
        kernel: "auto", "valu" (fp32 vector kernels), "mfma" (matrix cores),
            "mfma_wg" (the workgroup matrix-core kernels) or "mfma_precise"
            (causal: the workgroup kernels with every product fp32-accurate
            for bf16 inputs too; the backward keeps its own choice).

    Returns:
        out: [N, T, d] in V's dtype.
    """
    return RaceFusedFunction.apply(probsQ, probsK, V, causal, tile_tokens, _kernel_id(kernel))


def race_fused_fwd_with_state(probsQ, probsK, V, causal: bool = True, *, tile_tokens: int = 0,
                              kernel: str | int = "auto"):
    """(out, state): state [N, S*d + S] fp32 holds B [S, d] then A [S], the
    per-bucket sums over all T tokens (for causal=True the decode hand-off of
    src/causal_v2/kernels/race_causal_fwd.h:20-21).  No autograd."""
    return _lib.ext().forward(probsQ, probsK, V, bool(causal), int(tile_tokens),
                              _kernel_id(kernel), True)


def race_fused_fwd_carry(probsQ, probsK, V, state, *, inplace: bool = False, tile_tokens: int = 0,
                         kernel: str | int = "auto"):
    """(out, new_state): the causal op continued from a carried state.

    state [N, S*d + S] fp32 (B [S, d] then A [S] per stream, as
    race_fused_fwd_with_state returns it) holds the sums over all earlier
    tokens; the call advances it over these T tokens, as the reference's
    chunked forward carries A_state, B_state into its next chunk
    (src/race_chunked.py:54-63).  Splitting a sequence anywhere and carrying
    the state gives the unsplit outputs up to fp32 rounding.  With
    inplace=True the state tensor itself is advanced (a decode step) and
    returned.  Calls of at most 16 tokens run one decode launch; kernel
    "decode" forces it for any T, the other kernels force the tile path.
    No autograd."""
    return _lib.ext().forward_carry(probsQ, probsK, V, state, int(tile_tokens), _kernel_id(kernel),
                                    bool(inplace))


def race_noncausal_backward(probsQ, probsK, V, dOut, state, *, need=(True, True, True),
                            tile_tokens: int = 0):
    """(dQ, dK, dV) of the non-causal forward for upstream gradient dOut."""
    return _lib.ext().noncausal_backward(probsQ, probsK, V, _dense(dOut), state, *need,
                                         tile_tokens)


def race_causal_backward(probsQ, probsK, V, dOut, *, need=(True, True, True),
                         tile_tokens: int = 0, kernel: str | int = "auto"):
    """(dQ, dK, dV) of the causal forward for upstream gradient dOut.  kernel:
    "auto" (matrix cores where a specialization exists), "valu" or "mfma"."""
    return _lib.ext().causal_backward(probsQ, probsK, V, _dense(dOut), *need, tile_tokens,
                                      _kernel_id(kernel))


def select_tile_tokens(N: int, T: int, L: int, R: int, d: int, *, bf16: bool = False,
                       causal: bool = True, tile_tokens: int = 0, kernel: str | int = "auto") -> int:
    return _lib.ext().select_tile_tokens(N, T, L, R, d, bf16, causal, tile_tokens,
                                         _kernel_id(kernel))


class HashProbsFunction(torch.autograd.Function):
    """probs = race_hash_probs(x, planes_T, L, K), differentiable w.r.t. x.

    The planes are a buffer in the reference module (src/race_baseline.py:27),
    so they get no gradient.  The backward is race_hash_probs_bwd."""

    @staticmethod
    def forward(ctx, x, planes_T, L, K):
        x = _dense(x)
        planes_T = planes_T.float().contiguous()
        ctx.L, ctx.K = int(L), int(K)
        if ctx.needs_input_grad[0]:
            ctx.save_for_backward(x, planes_T)
        return _lib.ext().hash_probs(x, planes_T, ctx.L, ctx.K)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_probs):
        x, planes_T = ctx.saved_tensors
        dx = _lib.ext().hash_probs_backward(x, planes_T, _dense(grad_probs.to(x.dtype)), ctx.L, ctx.K)
        return dx, None, None, None


def race_hash_probs(x: torch.Tensor, planes_T: torch.Tensor, L: int, K: int) -> torch.Tensor:
    """Bucket probabilities [..., L, 2^K] of token rows x [..., d_k]: the
    hashing of src/race_baseline.py:41-44 (tanh of the shared-plane
    projections over sqrt(d_k), softmax over the 2^K corners), on the GPU.
    Differentiable w.r.t. x."""
    return HashProbsFunction.apply(x, planes_T, int(L), int(K))


class HashedRaceFunction(torch.autograd.Function):
    """out = race_fused_fwd_hashed(K, Q, V, planes, L): the causal op with the
    hashing inside the kernels (no probabilities in memory).

    Backward: the probabilities are recomputed (race_hash_probs), the causal
    backward starts from the forward's tile records, and the hashing backward
    (race_hash_probs_bwd) takes dprobs to the rows."""

    @staticmethod
    def forward(ctx, K, Q, V, planes, L, tile_tokens):
        needs = any(ctx.needs_input_grad[:3])
        out, records, _, tile = _lib.ext().hashed_forward(K, Q, V, planes, int(L), int(tile_tokens),
                                                          needs, False)
        if needs:
            ctx.save_for_backward(K, Q, V, planes, records)
            ctx.L, ctx.tile = int(L), int(tile)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        need_k, need_q, need_v = ctx.needs_input_grad[:3]
        K, Q, V, planes, records = ctx.saved_tensors
        L = ctx.L
        Kp = planes.shape[0] // L
        ext = _lib.ext()
        planes_T = planes.t().contiguous()
        probsK = ext.hash_probs(K, planes_T, L, Kp)
        probsQ = ext.hash_probs(Q, planes_T, L, Kp)
        g = _dense(grad_out.to(V.dtype))
        dpq, dpk, dv = ext.causal_backward(probsQ, probsK, V, g, need_q, need_k, need_v, ctx.tile, 0,
                                           records)
        dk = ext.hash_probs_backward(K, planes_T, dpk, L, Kp) if need_k else None
        dq = ext.hash_probs_backward(Q, planes_T, dpq, L, Kp) if need_q else None
        return dk, dq, dv, None, None, None


def race_fused_fwd_hashed(K: torch.Tensor, Q: torch.Tensor, V: torch.Tensor, planes: torch.Tensor,
                          L: int, *, tile_tokens: int = 0) -> torch.Tensor:
    """The causal op with the hashing inside: BatchedACE.forward's lines 41-51
    (src/race_baseline.py) in one op, the reference's fused forward
    race_fused_fwd(K, Q, V, planes, L) (src/race_fused_fwd.cu:150-171).

    Args:
        K, Q, V: [N, T, d] token rows (float32 or bfloat16, one dtype), d = d_k.
        planes: [L * K_planes, d] float32 hash planes (the reference's
            `planes`; BatchedACE's planes_T transposed).
        L: hash tables; R = 2^K_planes buckets each.

    Returns [N, T, d]: race_fused_fwd(hash(Q), hash(K), V, causal=True) with
    the probabilities computed inside the kernels.  Differentiable w.r.t. K,
    Q and V."""
    return HashedRaceFunction.apply(_dense(K), _dense(Q), _dense(V), planes.float().contiguous(), int(L),
                                    int(tile_tokens))


def hashed_supported(L: int, K: int, d: int) -> bool:
    """Whether race_fused_fwd_hashed has kernels for L tables of 2^K buckets, width d."""
    return bool(_lib.ext().hashed_supported(int(L), int(K), int(d)))
