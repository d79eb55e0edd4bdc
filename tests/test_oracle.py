"""CPU tests that pin the oracle (oracle/) before anything is compared with it.

Each formulation of the oracle is checked against the exact-arithmetic golden
vectors (tests/golden/make_golden.py), against the others (they share no
code), against closed forms the mathematics fixes, and against invariants.
The last group plants plausible mistakes in numpy copies of the oracle and
shows that the checks above catch each of them.

The cases mirror the reference's own run-time pins: chunked == unchunked at
several (T, chunk) including uneven, 1-token and chunk >= T
(src/test_equivalence.py:49-59), the per-token recurrence == the cumsum
composition (src/test_kernel_math.py:43-61), and the blocked per-bucket
bridge in fp64 at 1e-12 (src/causal_v2/tests/test_reference.py:52-65).
"""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "race_golden.npz"
FP64_TOL = 1e-12


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-300))


def probs(rng, N, T, L, R):
    logits = rng.standard_normal((N, T, L, R)) * 4.0
    e = np.exp(logits - logits.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).reshape(N, T, L * R).astype(np.float32)


def inputs(seed, N, T, L, R, d):
    rng = np.random.default_rng(seed)
    return probs(rng, N, T, L, R), probs(rng, N, T, L, R), rng.standard_normal((N, T, d)).astype(np.float32)


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


# --- golden vectors (exact rational arithmetic) ------------------------------------------

@pytest.mark.parametrize("name", ["small", "one_token", "wide", "s1", "eps"])
def test_causal_forms_match_exact_golden(oracle, golden, name):
    q, k, v = golden[f"{name}_q"], golden[f"{name}_k"], golden[f"{name}_v"]
    want = golden[f"{name}_causal"]
    assert rel_err(oracle.causal_recurrence(q, k, v), want) <= FP64_TOL
    assert rel_err(oracle.causal_chunked(q, k, v, 4), want) <= FP64_TOL
    assert rel_err(oracle.causal_tiled(q, k, v, 4, 2)[0], want) <= FP64_TOL
    assert rel_err(oracle.cumsum_bmm(q, k, v), want) <= FP64_TOL
    assert rel_err(oracle.dense_causal(q, k, v), want) <= FP64_TOL


@pytest.mark.parametrize("name", ["small", "one_token", "wide", "s1", "eps"])
def test_noncausal_matches_exact_golden(oracle, golden, name):
    q, k, v = golden[f"{name}_q"], golden[f"{name}_k"], golden[f"{name}_v"]
    out, _ = oracle.noncausal_fwd(q, k, v)
    assert rel_err(out, golden[f"{name}_noncausal"]) <= FP64_TOL


def test_noncausal_backward_matches_exact_dual_number_gradients(oracle, golden):
    q, k, v, g = golden["grad_q"], golden["grad_k"], golden["grad_v"], golden["grad_g"]
    dq, dk, dv = oracle.noncausal_bwd(q, k, v, g)
    assert rel_err(dq, golden["grad_dq"]) <= 1e-11
    assert rel_err(dk, golden["grad_dk"]) <= 1e-11
    assert rel_err(dv, golden["grad_dv"]) <= 1e-11
    out, aq, ak, av = oracle.torch_noncausal_autograd(q, k, v, g)
    assert rel_err(out, golden["grad_out"]) <= FP64_TOL
    for got, want in ((aq, golden["grad_dq"]), (ak, golden["grad_dk"]), (av, golden["grad_dv"])):
        assert rel_err(got, want) <= 1e-11


# --- the formulations agree with each other ----------------------------------------------

@pytest.mark.parametrize("T, chunk", [(512, 512), (2048, 512), (2048, 300), (2048, 1), (1000, 4096)])
def test_chunked_equals_recurrence_fp64(oracle, T, chunk):
    # src/test_equivalence.py:166-176 cases, at N=2 to keep the CPU suite short.
    q, k, v = inputs(T + chunk, 2, T, 4, 16, 64)
    rec = oracle.causal_recurrence(q, k, v)
    assert rel_err(oracle.causal_chunked(q, k, v, chunk), rec) <= FP64_TOL


@pytest.mark.parametrize("T, tile, chunk", [(777, 64, 32), (777, 128, 64), (300, 2048, 64), (65, 64, 64),
                                            (1, 64, 32)])
def test_tiled_decomposition_equals_recurrence(oracle, T, tile, chunk):
    q, k, v = inputs(T * 7 + tile, 2, T, 4, 16, 32)
    rec, fin_rec = oracle.causal_recurrence(q, k, v, want_state=True)
    out, pref, fin = oracle.causal_tiled(q, k, v, tile, chunk)
    assert rel_err(out, rec) <= FP64_TOL
    assert rel_err(fin, fin_rec) <= FP64_TOL
    # The prefix of tile t is the recurrence's state after token t*tile - 1.
    S, d = 64, 32
    for t in range(pref.shape[1]):
        end = t * tile
        if end == 0:
            assert not pref[:, 0].any()
            continue
        _, st = oracle.causal_recurrence(q[:, :end], k[:, :end], v[:, :end], want_state=True)
        assert rel_err(pref[:, t], st) <= FP64_TOL
    assert pref.shape[2] == S * d + S


@pytest.mark.parametrize("split", [0, 1, 63, 200, 299, 300])
def test_recurrence_continued_from_carried_state(oracle, split):
    # Running tokens [0, split) and then [split, T) from the carried state is
    # the unsplit run (the carry of src/race_chunked.py:54-63): outputs of the
    # second part and the final state both match.
    q, k, v = inputs(split + 11, 3, 300, 2, 16, 24)
    full, fin = oracle.causal_recurrence(q, k, v, want_state=True)
    _, mid = oracle.causal_recurrence(q[:, :split], k[:, :split], v[:, :split], want_state=True)
    out2, fin2 = oracle.causal_recurrence(q[:, split:], k[:, split:], v[:, split:], want_state=True,
                                          init_state=mid)
    assert rel_err(fin2, fin) <= FP64_TOL
    if split < 300:
        assert rel_err(out2, full[:, split:]) <= FP64_TOL
    # A zero carried state is no carried state.
    assert np.array_equal(oracle.causal_recurrence(q, k, v, init_state=np.zeros_like(fin)), full)


@pytest.mark.parametrize("tail, block", [(1, 7), (50, 64), (299, 1000), (300, 3), (120, 1)])
def test_tail_from_block_sums_is_the_scan(oracle, tail, block):
    # causal_tail (state from blocked k^T v products, then the scan) gives the
    # last outputs of the full per-token scan, whatever the block length; a
    # transposed B in the carried state would fail (S != d here).
    q, k, v = inputs(tail + block, 3, 300, 2, 16, 24)
    full = oracle.causal_recurrence(q, k, v)
    got = oracle.causal_tail(q, k, v, tail, block=block)
    assert got.shape == (3, tail, 24)
    assert rel_err(got, full[:, 300 - tail:]) <= FP64_TOL


def test_cumsum_bmm_and_dense_forms_agree(oracle):
    q, k, v = inputs(5, 3, 200, 2, 8, 16)
    rec = oracle.causal_recurrence(q, k, v)
    assert rel_err(oracle.cumsum_bmm(q, k, v), rec) <= FP64_TOL
    assert rel_err(oracle.dense_causal(q, k, v), rec) <= FP64_TOL


def test_torch_fp32_reference_path_is_within_fp32_rounding(oracle):
    import torch

    q, k, v = inputs(6, 8, 512, 4, 16, 64)
    ref = oracle.causal_recurrence(q, k, v)
    got = oracle.torch_reference_path(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v))
    assert rel_err(got.numpy(), ref) <= 1e-5


def test_noncausal_forward_forms_agree(oracle):
    import torch

    q, k, v = inputs(7, 3, 300, 4, 16, 64)
    out, st = oracle.noncausal_fwd(q, k, v)
    tq, tk, tv = (torch.from_numpy(x).double() for x in (q, k, v))
    assert rel_err(oracle.torch_noncausal_reference(tq, tk, tv).numpy(), out) <= FP64_TOL
    # B and A are the totals: the causal final state.
    _, fin = oracle.causal_recurrence(q, k, v, want_state=True)
    assert rel_err(st, fin) <= FP64_TOL


def test_noncausal_backward_closed_form_equals_autograd(oracle):
    q, k, v = inputs(8, 2, 150, 2, 8, 16)
    g = np.random.default_rng(9).standard_normal((2, 150, 16)).astype(np.float32)
    dq, dk, dv = oracle.noncausal_bwd(q, k, v, g)
    _, aq, ak, av = oracle.torch_noncausal_autograd(q, k, v, g)
    assert rel_err(dq, aq) <= 1e-11 and rel_err(dk, ak) <= 1e-11 and rel_err(dv, av) <= 1e-11


def test_noncausal_backward_gradcheck():
    import torch

    torch.manual_seed(0)
    q = torch.rand(1, 5, 6, dtype=torch.float64, requires_grad=True)
    k = torch.rand(1, 5, 6, dtype=torch.float64, requires_grad=True)
    v = torch.randn(1, 5, 3, dtype=torch.float64, requires_grad=True)
    import __graft_entry__ as entry

    oracle = entry.load_oracle()
    assert torch.autograd.gradcheck(lambda a, b, c: oracle.torch_noncausal_reference(a, b, c, eps=1e-3),
                                    (q, k, v))


@pytest.mark.parametrize("name", ["cgrad", "cgrad_wide"])
def test_causal_backward_matches_exact_dual_number_gradients(oracle, golden, name):
    q, k, v, g = (golden[f"{name}_{x}"] for x in "qkvg")
    dq, dk, dv = oracle.causal_bwd(q, k, v, g)
    assert rel_err(dq, golden[f"{name}_dq"]) <= FP64_TOL
    assert rel_err(dk, golden[f"{name}_dk"]) <= FP64_TOL
    assert rel_err(dv, golden[f"{name}_dv"]) <= FP64_TOL


@pytest.mark.parametrize("N,T,L,R,d", [(2, 150, 2, 8, 16), (1, 1, 4, 16, 8), (3, 33, 1, 1, 2)])
def test_causal_backward_closed_form_equals_autograd(oracle, N, T, L, R, d):
    q, k, v = inputs(30 + T, N, T, L, R, d)
    g = np.random.default_rng(31).standard_normal((N, T, d)).astype(np.float32)
    dq, dk, dv = oracle.causal_bwd(q, k, v, g)
    out, aq, ak, av = oracle.torch_causal_autograd(q, k, v, g)
    assert rel_err(out, oracle.causal_recurrence(q, k, v)) <= FP64_TOL
    assert rel_err(dq, aq) <= 1e-11 and rel_err(dk, ak) <= 1e-11 and rel_err(dv, av) <= 1e-11


def test_causal_backward_gradcheck():
    import torch

    torch.manual_seed(1)
    q = torch.rand(1, 6, 4, dtype=torch.float64, requires_grad=True)
    k = torch.rand(1, 6, 4, dtype=torch.float64, requires_grad=True)
    v = torch.randn(1, 6, 3, dtype=torch.float64, requires_grad=True)
    import __graft_entry__ as entry

    oracle = entry.load_oracle()
    assert torch.autograd.gradcheck(lambda a, b, c: oracle.torch_causal_reference(a, b, c, eps=1e-3),
                                    (q, k, v))


def test_causal_backward_single_token_closed_form(oracle):
    # T = 1: out = v * sum_s q_s k_s / (k_s + eps), so
    #   dq_s = <v, g> k_s / (k_s + eps),  dk_s = <v, g> q_s eps / (k_s + eps)^2,
    #   dv   = g * sum_s q_s k_s / (k_s + eps).
    q, k, v = inputs(32, 2, 1, 4, 16, 8)
    g = np.random.default_rng(33).standard_normal((2, 1, 8)).astype(np.float32)
    q0, k0, v0, g0 = (x[:, 0].astype(np.float64) for x in (q, k, v, g))
    vg = (v0 * g0).sum(-1, keepdims=True)
    dq, dk, dv = oracle.causal_bwd(q, k, v, g)
    assert rel_err(dq[:, 0], vg * k0 / (k0 + 1e-6)) <= FP64_TOL
    assert rel_err(dk[:, 0], vg * q0 * 1e-6 / (k0 + 1e-6) ** 2) <= 1e-9
    assert rel_err(dv[:, 0], g0 * (q0 * k0 / (k0 + 1e-6)).sum(-1, keepdims=True)) <= FP64_TOL


def test_causal_backward_last_token_matches_noncausal(oracle):
    # The gradient w.r.t. the last query only sees the totals: dq_{T-1} of the
    # causal function equals dq_{T-1} of the non-causal one.
    q, k, v = inputs(34, 2, 40, 2, 8, 4)
    g = np.zeros((2, 40, 4), np.float32)
    g[:, -1] = np.random.default_rng(35).standard_normal((2, 4)).astype(np.float32)
    cq, ck, cv = oracle.causal_bwd(q, k, v, g)
    nq, nk, nv = oracle.noncausal_bwd(q, k, v, g)
    assert rel_err(cq, nq) <= FP64_TOL and rel_err(ck, nk) <= 1e-11 and rel_err(cv, nv) <= FP64_TOL


# --- closed forms ---------------------------------------------------------------------------

def test_single_token_closed_form(oracle):
    # T = 1: out_0 = v_0 * sum_s q_s k_s / (k_s + eps).
    q, k, v = inputs(10, 3, 1, 4, 16, 8)
    q0, k0, v0 = (x[:, 0].astype(np.float64) for x in (q, k, v))
    want = v0 * (q0 * k0 / (k0 + 1e-6)).sum(-1, keepdims=True)
    assert rel_err(oracle.causal_recurrence(q, k, v)[:, 0], want) <= FP64_TOL


def test_uniform_keys_closed_form(oracle):
    # probsK = 1/R everywhere: out_t = (sum_s q_ts) * (sum_{j<=t} v_j / R) / ((t+1)/R + eps).
    N, T, L, R, d = 2, 50, 2, 8, 4
    q, _, v = inputs(11, N, T, L, R, d)
    k = np.full((N, T, L * R), np.float32(1.0 / R), np.float32)
    kval = np.float64(np.float32(1.0 / R))
    t = np.arange(1, T + 1, dtype=np.float64)[None, :, None]
    want = q.astype(np.float64).sum(-1, keepdims=True) * (np.cumsum(v.astype(np.float64), 1) * kval) / (t * kval + 1e-6)
    assert rel_err(oracle.causal_recurrence(q, k, v), want) <= FP64_TOL


def test_one_hot_buckets_give_running_bucket_means(oracle):
    # One-hot probs: out_t = (count / (count + eps)) * mean of v_j over j <= t in q_t's bucket.
    rng = np.random.default_rng(12)
    N, T, S, d = 1, 64, 8, 3
    kb = rng.integers(0, S, T)
    qb = rng.integers(0, S, T)
    q = np.zeros((N, T, S), np.float32)
    k = np.zeros((N, T, S), np.float32)
    q[0, np.arange(T), qb] = 1
    k[0, np.arange(T), kb] = 1
    v = rng.integers(-5, 6, (N, T, d)).astype(np.float32)
    want = np.zeros((N, T, d))
    for t in range(T):
        members = [j for j in range(t + 1) if kb[j] == qb[t]]
        if members:
            want[0, t] = v[0, members].astype(np.float64).sum(0) / (len(members) + 1e-6)
    assert rel_err(oracle.causal_recurrence(q, k, v), want) <= FP64_TOL


# --- invariants ---------------------------------------------------------------------------

def test_last_causal_row_equals_noncausal_row(oracle):
    q, k, v = inputs(13, 3, 97, 4, 16, 16)
    causal = oracle.causal_recurrence(q, k, v)
    nc, _ = oracle.noncausal_fwd(q, k, v)
    assert rel_err(causal[:, -1], nc[:, -1]) <= FP64_TOL


def test_future_tokens_do_not_change_the_past(oracle):
    q, k, v = inputs(14, 2, 120, 4, 16, 8)
    base = oracle.causal_chunked(q, k, v, 32)
    k2, v2 = k.copy(), v.copy()
    k2[:, 70:] = k[:, 70:][:, ::-1]
    v2[:, 70:] = -3 * v[:, 70:]
    got = oracle.causal_chunked(q, k2, v2, 32)
    assert np.array_equal(got[:, :70], base[:, :70])
    assert not np.array_equal(got[:, 70:], base[:, 70:])


def test_streams_are_independent_and_bounded(oracle):
    q, k, v = inputs(15, 4, 80, 4, 16, 8)
    full = oracle.causal_recurrence(q, k, v)
    one = oracle.causal_recurrence(q[2:3], k[2:3], v[2:3])
    assert np.array_equal(full[2:3], one)
    # Weights q_s * k_js / (A_s + eps) are >= 0 and sum to < sum_s q_s = L.
    L = 4
    assert np.abs(full).max() <= L * np.abs(v).max()


# --- planted mistakes: the checks above must catch each -----------------------------------

def _mutant(q, k, v, *, exclusive=False, no_eps=False, swap_qk=False, drop_carry=False, chunk=16):
    """A numpy causal forward with one plausible mistake switched on."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    if swap_qk:
        q, k = k, q
    a = np.cumsum(k, 1)
    b = np.cumsum(k[..., :, None] * v[..., None, :], 1)
    if exclusive:
        a, b = a - k, b - k[..., :, None] * v[..., None, :]
    if drop_carry:  # forgets the carried state at every chunk boundary
        T = q.shape[1]
        for t0 in range(chunk, T, chunk):
            a[:, t0:] -= a[:, t0 - 1:t0]
            b[:, t0:] -= b[:, t0 - 1:t0]
    eps = 0.0 if no_eps else 1e-6
    with np.errstate(divide="ignore", invalid="ignore"):
        e = b / (a[..., None] + eps)
    e = np.nan_to_num(e)
    return np.einsum("nts,ntsc->ntc", q, e)


def test_planted_mistakes_are_caught(oracle, golden):
    # Sanity: the mutant with no mistake matches the golden vectors.
    q, k, v = golden["small_q"], golden["small_k"], golden["small_v"]
    assert rel_err(_mutant(q, k, v), golden["small_causal"]) <= FP64_TOL
    # Exclusive prefix (diagonal dropped): the golden and single-token checks fail.
    assert rel_err(_mutant(q, k, v, exclusive=True), golden["small_causal"]) > 1e-3
    # Probabilities of Q and K transposed in roles: golden fails.
    assert rel_err(_mutant(q, k, v, swap_qk=True), golden["small_causal"]) > 1e-3
    # eps dropped: the eps golden case (probsK == 1e-6 in a bucket) fails.
    qe, ke, ve = golden["eps_q"], golden["eps_k"], golden["eps_v"]
    assert rel_err(_mutant(qe, ke, ve, no_eps=True), golden["eps_causal"]) > 1e-3
    # Carry dropped at chunk boundaries: the recurrence/chunk agreement fails.
    q2, k2, v2 = inputs(16, 1, 64, 4, 16, 8)
    assert rel_err(_mutant(q2, k2, v2, drop_carry=True), oracle.causal_recurrence(q2, k2, v2)) > 1e-3


def _mutant_bwd(q, k, v, g, *, exclusive_suffix=False, drop_alpha=False):
    """A numpy causal backward with one plausible mistake switched on."""
    q, k, v, g = (np.asarray(x, np.float64) for x in (q, k, v, g))
    a = np.cumsum(k, 1)
    b = np.cumsum(k[..., :, None] * v[..., None, :], 1)
    r = 1.0 / (a + 1e-6)
    dq = r * np.einsum("ntsc,ntc->nts", b, g)
    w = q * r
    alpha = np.zeros_like(dq) if drop_alpha else -w * dq
    wg = w[..., :, None] * g[..., None, :]
    z = np.cumsum(wg[:, ::-1], 1)[:, ::-1]
    y = np.cumsum(alpha[:, ::-1], 1)[:, ::-1]
    if exclusive_suffix:
        z, y = z - wg, y - alpha
    dk = np.einsum("ntsc,ntc->nts", z, v) + y
    dv = np.einsum("nts,ntsc->ntc", k, z)
    return dq, dk, dv


def test_planted_backward_mistakes_are_caught(golden):
    q, k, v, g = (golden[f"cgrad_{x}"] for x in "qkvg")
    want = [golden[f"cgrad_{x}"] for x in ("dq", "dk", "dv")]
    got = _mutant_bwd(q, k, v, g)
    assert all(rel_err(a, b) <= FP64_TOL for a, b in zip(got, want))
    # Suffix sums that skip the diagonal token: dk and dv fail.
    got = _mutant_bwd(q, k, v, g, exclusive_suffix=True)
    assert rel_err(got[1], want[1]) > 1e-3 and rel_err(got[2], want[2]) > 1e-3
    # The denominator's gradient dropped: dk fails.
    got = _mutant_bwd(q, k, v, g, drop_alpha=True)
    assert rel_err(got[1], want[1]) > 1e-3


# --- the hashing front end (src/race_baseline.py:41-44) --------------------------------------

@pytest.mark.parametrize("dk, L, K", [(64, 4, 4), (8, 1, 1), (128, 8, 5), (16, 2, 8)])
def test_hash_probs_product_identity_and_invariants(oracle, dk, L, K):
    rng = np.random.default_rng(40 + K)
    x = rng.standard_normal((3, 17, dk)).astype(np.float32)
    planes_T = rng.standard_normal((dk, L * K)).astype(np.float32)
    p = oracle.hash_probs(x, planes_T, L, K)
    assert p.shape == (3, 17, L, 1 << K)
    assert rel_err(p, oracle.hash_probs_product_form(x, planes_T, L, K)) <= FP64_TOL
    np.testing.assert_allclose(p.sum(-1), 1.0, atol=1e-13)
    # x = 0 gives uniform probabilities; -x maps corner r to its complement.
    np.testing.assert_allclose(oracle.hash_probs(np.zeros((2, dk)), planes_T, L, K), 1.0 / (1 << K))
    assert rel_err(oracle.hash_probs(-x, planes_T, L, K), p[..., ::-1]) <= FP64_TOL


def test_hash_probs_corner_order(oracle):
    # itertools.product([-1, 1], repeat=3): r = 0 is (-1,-1,-1), r = 1 is (-1,-1,+1), r = 7 all +1.
    s = oracle.corners(3)
    assert s[0].tolist() == [-1, -1, -1] and s[1].tolist() == [-1, -1, 1] and s[7].tolist() == [1, 1, 1]
    # One positive projection on plane k=0 favours the corners with s_0 = +1 (r >= 4).
    planes_T = np.zeros((2, 3))
    planes_T[0, 0] = 50.0
    p = oracle.hash_probs(np.array([[1.0, 0.0]]), planes_T, 1, 3)[0, 0]
    assert p[4:].min() > p[:4].max()


def test_hash_probs_matches_torch_composition(oracle):
    import torch

    rng = np.random.default_rng(41)
    x = rng.standard_normal((2, 33, 64))
    planes_T = rng.standard_normal((64, 16))
    protos_T = torch.from_numpy(oracle.corners(4).T.copy())
    xt = torch.from_numpy(x)
    proj = (xt @ torch.from_numpy(planes_T)).view(2, 33, 4, 4)
    want = torch.softmax(proj.tanh().div(8.0) @ protos_T, dim=-1).numpy()
    assert rel_err(oracle.hash_probs(x, planes_T, 4, 4), want) <= FP64_TOL
