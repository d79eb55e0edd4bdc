"""GPU parity of the non-causal forward and backward against the CPU oracle.

cfg4 (N = 384, T = 1024, L = 4, R = 16, d = 64, fp32): outputs
against the fp64 oracle, gradients w.r.t. probsQ, probsK and V against the
oracle's closed-form VJP and against torch.autograd on the reference formula
(analysis/hot-path.md:157-162).  The property tests follow the reference's
non-causal suite (src/noncausal/tests/test_backward_cuda.py): determinism,
needs_input_grad filtering, permutation invariance over keys.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, per_stream_rel_err, say, to_np, tol_for

pytestmark = pytest.mark.gpu


def forward_backward(race, q, k, v, g, cuda):
    qg, kg, vg = (x.to(cuda).requires_grad_(True) for x in (q, k, v))
    out = race.race_fused_fwd(qg, kg, vg, causal=False)
    out.backward(g.to(cuda))
    torch.cuda.synchronize()
    return out.detach(), qg.grad, kg.grad, vg.grad


def test_cfg4_forward_and_backward_match_oracle(race, oracle, cuda):
    say("cfg4 full size")
    q, k, v, g = race.make_inputs(384, 1024, 4, 16, 64, seed=4, grad_out=True)
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    ref_out, _ = oracle.noncausal_fwd(to_np(q), to_np(k), to_np(v), nthreads=16)
    rq, rk, rv = oracle.noncausal_bwd(to_np(q), to_np(k), to_np(v), to_np(g), nthreads=16)
    errs = {name: per_stream_rel_err(to_np(got), want)
            for name, got, want in (("out", out, ref_out), ("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv))}
    say("cfg4", {k_: f"{e_:.2e}" for k_, e_ in errs.items()})
    for name, err in errs.items():
        assert err <= FP32_TOL, (name, err)


def test_cfg4_gradients_match_torch_autograd(race, oracle, cuda):
    # The cfg4 gradient check is torch autograd on the reference formula; run
    # it on 16 of the 384 streams (fp64, CPU).
    say("cfg4 autograd")
    q, k, v, g = race.make_inputs(384, 1024, 4, 16, 64, seed=4, grad_out=True)
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    pick = list(range(0, 384, 24))
    a_out, aq, ak, av = oracle.torch_noncausal_autograd(to_np(q[pick]), to_np(k[pick]), to_np(v[pick]),
                                                        to_np(g[pick]))
    for got, want in ((out, a_out), (dq, aq), (dk, ak), (dv, av)):
        assert per_stream_rel_err(to_np(got[pick]), want) <= FP32_TOL


def dk_term_scale(q, k, v, g, eps=1e-6):
    """Per-stream max over (t, s) of sum_c |v[t,c] dB[s,c]| + |dA[s]|: the size of
    the terms whose sum is dK.  When they cancel (S = 1 makes dK = q g v eps /
    (k + eps)^2, ~1e-6 of each term), fp32 can only be accurate relative to
    this, so dK's error is bounded by tol * this scale."""
    q, k, v, g = (np.asarray(x, np.float64) for x in (q, k, v, g))
    A = k.sum(1)                                            # [N,S]
    E = np.einsum("nts,ntc->nsc", k, v) / (A[..., None] + eps)
    dE = np.einsum("nts,ntc->nsc", q, g)
    dB = dE / (A[..., None] + eps)
    dA = -(dE * E).sum(-1) / (A + eps)
    terms = np.einsum("ntc,nsc->nts", np.abs(v), np.abs(dB)) + np.abs(dA)[:, None, :]
    return terms.reshape(terms.shape[0], -1).max(1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d", [(1, 1, 1), (2, 8, 32), (4, 16, 64), (3, 5, 7), (8, 32, 128)])
@pytest.mark.parametrize("T", [1, 63, 65, 1000])
def test_shapes(race, oracle, cuda, dtype, L, R, d, T):
    say("nc-shape", dtype, L, R, d, T)
    q, k, v, g = race.make_inputs(3, T, L, R, d, seed=T + d, dtype=dtype, grad_out=True)
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    assert out.dtype == dtype and dq.dtype == dtype
    ref_out, _ = oracle.noncausal_fwd(to_np(q), to_np(k), to_np(v))
    rq, rk, rv = oracle.noncausal_bwd(to_np(q), to_np(k), to_np(v), to_np(g))
    tol = tol_for(dtype)
    assert per_stream_rel_err(to_np(out), ref_out) <= tol
    assert per_stream_rel_err(to_np(dq), rq) <= tol
    scale = dk_term_scale(to_np(q), to_np(k), to_np(v), to_np(g))
    dk_err = np.abs(to_np(dk).astype(np.float64) - rk).reshape(3, -1).max(1)
    assert (dk_err <= tol * scale).all()
    assert per_stream_rel_err(to_np(dv), rv) <= tol


@pytest.mark.parametrize("need", [(True, False, False), (False, True, False), (False, False, True),
                                  (True, True, False), (True, False, True), (False, True, True)])
@pytest.mark.parametrize("T", [200, 500])
def test_only_requested_gradients(race, cuda, need, T):
    # At S = d = 64 the requests take different kernels (the query-side and
    # key-side passes, or the separate reduction, finalize and maps); every
    # gradient must come out bit for bit the same either way.  T = 200 gives
    # 4 tiles of 64 per stream (the key side sums the dE records itself),
    # T = 500 gives 8 (after the finalize).
    say("needs-grad", need, T)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, T, 4, 16, 64, seed=3, grad_out=True))
    leaves = [x.clone().requires_grad_(n) for x, n in zip((q, k, v), need)]
    race.race_fused_fwd(*leaves, causal=False).backward(g)
    _, fq, fk, fv = forward_backward(race, q, k, v, g, cuda)
    for leaf, n, full in zip(leaves, need, (fq, fk, fv)):
        if n:
            assert torch.equal(leaf.grad, full)
        else:
            assert leaf.grad is None


def test_bitwise_reproducible(race, cuda):
    say("nc-bitwise")
    q, k, v, g = race.make_inputs(5, 3000, 4, 16, 64, seed=8, grad_out=True)
    first = forward_backward(race, q, k, v, g, cuda)
    for _ in range(2):
        again = forward_backward(race, q, k, v, g, cuda)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


def test_permuting_keys_changes_nothing_beyond_rounding(race, cuda):
    say("nc-permutation")
    q, k, v = (x.to(cuda) for x in race.make_inputs(2, 2000, 4, 16, 64, seed=9))
    perm = torch.randperm(2000, device=cuda)
    a = race.race_fused_fwd(q, k, v, causal=False)
    b = race.race_fused_fwd(q, k[:, perm].contiguous(), v[:, perm].contiguous(), causal=False)
    torch.cuda.synchronize()
    assert per_stream_rel_err(to_np(b), to_np(a).astype(np.float64)) <= 1e-5


def test_noncausal_row_equals_last_causal_row(race, cuda):
    say("nc-last-row")
    q, k, v = (x.to(cuda) for x in race.make_inputs(3, 1500, 4, 16, 64, seed=10))
    nc = race.race_fused_fwd(q, k, v, causal=False)
    c = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert per_stream_rel_err(to_np(c[:, -1:]), to_np(nc[:, -1:]).astype(np.float64)) <= 1e-5


def test_golden_gradients(race, cuda):
    import pathlib

    say("nc-golden")
    gd = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "race_golden.npz")
    q, k, v, g = (torch.from_numpy(gd[f"grad_{x}"]) for x in ("q", "k", "v", "g"))
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    assert per_stream_rel_err(to_np(out), gd["grad_out"]) <= 1e-5
    assert per_stream_rel_err(to_np(dq), gd["grad_dq"]) <= 1e-5
    assert per_stream_rel_err(to_np(dk), gd["grad_dk"]) <= 1e-5
    assert per_stream_rel_err(to_np(dv), gd["grad_dv"]) <= 1e-5



@pytest.mark.parametrize("L, R, d", [(4, 16, 64), (2, 8, 32), (3, 5, 7)])
def test_tile_sums_inside_the_map_match_the_separate_reduce(race, cuda, L, R, d):
    # With at most 4 tiles per stream the forward's map adds the tile records
    # itself (and writes the saved state); with more, a separate reduce forms
    # E first.  Both must give the oracle's totals and the same output.
    say("nc-fold", L, R, d)
    T = 2000
    q, k, v = race.make_inputs(3, T, L, R, d, seed=12)
    qc, kc, vc = (x.to(cuda) for x in (q, k, v))
    runs = {tile: race.race_fused_fwd_with_state(qc, kc, vc, causal=False, tile_tokens=tile)
            for tile in (64, 512, 2048)}  # 32 tiles (reduce), 4 and 1 (in the map)
    torch.cuda.synchronize()
    k64, v64 = to_np(k).astype(np.float64), to_np(v).astype(np.float64)
    S = L * R
    B = np.einsum("nts,ntc->nsc", k64, v64).reshape(3, S * d)
    A = k64.sum(1)
    want_state = np.concatenate([B, A], axis=1)
    out64, _ = runs[64]
    # fp32 sums of up to 2000 terms: about 2e-6 of the largest total.
    for tile, (out, state) in runs.items():
        assert per_stream_rel_err(to_np(state), want_state) <= 1e-5, tile
        assert per_stream_rel_err(to_np(out), to_np(out64).astype(np.float64)) <= 1e-5, tile
