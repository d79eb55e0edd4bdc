"""CPU tests that pin the Algorithm-1 oracle (oracle.alg1_causal) before the
GPU path is compared with it.

The function is the reference's causal v2 forward: hashing inside, one global
normalization per query (src/causal_v2/kernels/race_causal_fwd.h:6-10, ground
truth src/causal_v2/reference.py:100-128).  The fp64 recurrence in
race_oracle.c is checked against
  - the masked T x T form (src/causal_v2/reference.py:131-141), a different
    evaluation order sharing no code with it,
  - the Bernoulli product form of the features (src/noncausal/reference.py:
    103-125), which the direct softmax must equal,
  - closed forms: T = 1 returns v_0, a constant V returns the constant, the
    corner order of itertools.product,
  - the bridge of src/causal_v2/reference.py:144-159: with per-bucket
    normalization and beta = 1/sqrt(d) it must equal the per-bucket oracle fed
    by the hashing of src/race_baseline.py:41-44 (oracle.hash_probs, itself
    pinned in test_oracle.py) with planes_T = W viewed as [L*P, d]^T,
  - the tile prefix states against an exclusive cumsum of per-tile sums,
and plants plausible mistakes to show that these checks catch them.
"""
from __future__ import annotations

import numpy as np
import pytest

FP64_TOL = 1e-12


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-300))


def inputs(seed, N, T, D, L, P):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((N, T, D)).astype(np.float32) for _ in range(3))
    W = rng.standard_normal((L, P, D)).astype(np.float32)
    return q, k, v, W


@pytest.mark.parametrize("D, L, P", [(16, 3, 3), (8, 1, 1), (32, 4, 5), (8, 2, 2)])
@pytest.mark.parametrize("beta", [0.125, 1.0, 2.0])
def test_recurrence_equals_dense_form(oracle, D, L, P, beta):
    q, k, v, W = inputs(D + L + P, 2, 45, D, L, P)
    assert rel_err(oracle.alg1_causal(q, k, v, W, beta), oracle.alg1_dense(q, k, v, W, beta)) <= FP64_TOL


@pytest.mark.parametrize("L, P", [(1, 1), (2, 3), (4, 5)])
def test_softmax_features_equal_bernoulli_product(oracle, L, P):
    rng = np.random.default_rng(P)
    x = rng.standard_normal((5, 24))
    W = rng.standard_normal((L, P, 24))
    for beta in (0.1, 1.0, 3.0):
        a = oracle.alg1_features(x, W, beta)
        assert a.shape == (5, L << P)
        assert rel_err(a, oracle.alg1_features(x, W, beta, form="bernoulli")) <= FP64_TOL
        np.testing.assert_allclose(a.reshape(5, L, -1).sum(-1), 1.0, atol=1e-14)


def test_feature_corner_order(oracle):
    # Plane 0 is the most significant bit: a large positive projection on
    # plane 0 alone favours corners r >= R/2 (c_{r,0} = +1).
    W = np.zeros((1, 3, 2))
    W[0, 0, 0] = 50.0
    phi = oracle.alg1_features(np.array([[1.0, 0.0]]), W, 4.0)[0]
    assert phi[4:].min() > phi[:4].max()
    # x = 0: every corner equal.
    np.testing.assert_allclose(oracle.alg1_features(np.zeros((1, 2)), W, 1.0), 1.0 / 8)


def test_single_token_returns_its_value(oracle):
    q, k, v, W = inputs(3, 3, 1, 16, 2, 4)
    np.testing.assert_allclose(oracle.alg1_causal(q, k, v, W, 1.0), v, rtol=1e-15, atol=0)


@pytest.mark.parametrize("beta", [0.125, 2.0])
def test_constant_values_come_back(oracle, beta):
    q, k, _, W = inputs(4, 2, 300, 16, 4, 4)
    v = np.full_like(q, 0.7)
    assert rel_err(oracle.alg1_causal(q, k, v, W, beta), v) <= FP64_TOL


def test_per_bucket_bridge_to_hashing_and_recurrence(oracle):
    # src/causal_v2/reference.py:144-159: per-bucket normalization at
    # beta = 1/sqrt(d) is BatchedACE.forward with planes_T = W as [L*P, d]^T.
    D, L, P = 32, 4, 3
    q, k, v, W = inputs(5, 2, 200, D, L, P)
    planes_T = W.reshape(L * P, D).T.copy()
    pq = oracle.hash_probs(q, planes_T, L, P).reshape(2, 200, -1)
    pk = oracle.hash_probs(k, planes_T, L, P).reshape(2, 200, -1)
    want = oracle.causal_recurrence(pq.astype(np.float32), pk.astype(np.float32), v)
    got = oracle.alg1_causal(q, k, v, W, 1.0 / np.sqrt(D), perbucket=True)
    # The per-bucket oracle reads fp32 probabilities: compare at fp32 accuracy.
    assert rel_err(got, want) <= 1e-6
    # And in fp64 throughout, through the dense features.
    fq = oracle.alg1_features(q, W, 1.0 / np.sqrt(D))
    fk = oracle.alg1_features(k, W, 1.0 / np.sqrt(D))
    assert rel_err(fq, pq) <= FP64_TOL and rel_err(fk, pk) <= FP64_TOL


@pytest.mark.parametrize("T, tile", [(300, 64), (64, 64), (65, 64), (1, 128), (1000, 256)])
def test_tile_prefix_states(oracle, T, tile):
    D, L, P = 8, 2, 3
    q, k, v, W = inputs(6, 2, T, D, L, P)
    out, pref, fin = oracle.alg1_causal(q, k, v, W, 0.7, tile=tile)
    S = L << P
    fk = oracle.alg1_features(k, W, 0.7)                                   # [N, T, S]
    tiles = -(-T // tile)
    pad = tiles * tile - T
    fk = np.pad(fk, ((0, 0), (0, pad), (0, 0))).reshape(2, tiles, tile, S)
    vv = np.pad(v.astype(np.float64), ((0, 0), (0, pad), (0, 0))).reshape(2, tiles, tile, D)
    tB = np.einsum("ntjs,ntjd->ntsd", fk, vv).reshape(2, tiles, S * D)
    tA = fk.sum(2)
    tot = np.concatenate([tB, tA], -1)
    excl = np.cumsum(tot, 1) - tot
    assert pref.shape == (2, tiles, S * D + S)
    assert np.abs(pref[:, 0]).max() == 0.0
    assert rel_err(pref, excl) <= FP64_TOL
    assert rel_err(fin, tot.sum(1)) <= FP64_TOL
    assert rel_err(out, oracle.alg1_causal(q, k, v, W, 0.7)) == 0.0


def test_future_tokens_do_not_change_the_past(oracle):
    q, k, v, W = inputs(7, 1, 200, 16, 2, 3)
    k2, v2 = k.copy(), v.copy()
    k2[:, 120:] *= 3.0
    v2[:, 120:] = -v2[:, 120:]
    a = oracle.alg1_causal(q, k, v, W, 1.0)
    b = oracle.alg1_causal(q, k2, v2, W, 1.0)
    assert np.array_equal(a[:, :120], b[:, :120]) and not np.array_equal(a[:, 120:], b[:, 120:])


# --- planted mistakes: each must fail a check above ----------------------------------------

def _mutant_features(x, W, beta, *, lsb_first=False, beta_inside=False):
    x = np.asarray(x, np.float64)
    W = np.asarray(W, np.float64)
    L, P, _ = W.shape
    proj = np.einsum("...d,lpd->...lp", x, W)
    u = np.tanh(beta * proj) if beta_inside else np.tanh(proj)
    R = 1 << P
    c = np.array([[1.0 if (r >> (p if lsb_first else P - 1 - p)) & 1 else -1.0 for p in range(P)]
                  for r in range(R)])
    lg = (u @ c.T) * (1.0 if beta_inside else beta)
    e = np.exp(lg - lg.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).reshape(*x.shape[:-1], L * R)


def _mutant_dense(q, k, v, W, beta, *, strict=False, **kw):
    fq, fk = _mutant_features(q, W, beta, **kw), _mutant_features(k, W, beta, **kw)
    T = fq.shape[-2]
    scores = fq @ np.swapaxes(fk, -1, -2) * np.tril(np.ones((T, T)), -1 if strict else 0)
    den = scores.sum(-1, keepdims=True)
    return np.where(den == 0, 0.0, scores @ np.asarray(v, np.float64) / np.where(den == 0, 1.0, den))


def test_planted_mistakes_are_caught(oracle):
    q, k, v, W = inputs(8, 2, 60, 16, 2, 3)
    want = oracle.alg1_causal(q, k, v, W, 1.0)
    assert rel_err(_mutant_dense(q, k, v, W, 1.0), want) <= FP64_TOL
    # Diagonal excluded from the mask: the T = 1 closed form and the dense check fail.
    assert rel_err(_mutant_dense(q, k, v, W, 1.0, strict=True), want) > 1e-3
    # Beta applied inside the tanh instead of to the corner logits.
    assert rel_err(_mutant_dense(q, k, v, W, 2.0, beta_inside=True), oracle.alg1_causal(q, k, v, W, 2.0)) > 1e-3
    # Plane 0 as the least significant bit: the output is invariant (a
    # permutation of buckets shared by q and k), so the feature-order check
    # is what catches it.
    phi = _mutant_features(np.array([[1.0, 0.0]]), np.pad(np.eye(1, 2)[None] * 50.0, ((0, 0), (0, 2), (0, 0))),
                           4.0, lsb_first=True)[0]
    assert not phi[4:].min() > phi[:4].max()
