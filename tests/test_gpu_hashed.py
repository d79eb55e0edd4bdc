"""GPU parity of the causal op with the hashing inside (race_fused_fwd_hashed,
the reference's fused forward race_fused_fwd(K, Q, V, planes, L),
src/race_fused_fwd.cu:80-171) and of the hashing's backward.

The oracle is BatchedACE's lines 41-51 (src/race_baseline.py) restated in
fp64: oracle.hash_probs of the Q and K rows (pinned by the product form, the
corner order and the torch composition in tests/test_oracle.py), fed to
oracle.causal_recurrence (pinned by the exact golden vectors).  bf16 cases run
the oracle on the bf16-rounded rows.  Gradients through the drop-in module are
compared with torch.autograd through an fp64 torch restatement of the same
lines.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, assert_bf16_floor, per_stream_rel_err, say, to_np, tol_for

pytestmark = pytest.mark.gpu


def rows_and_planes(N, T, d, L, K, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    k, q, v = (torch.randn(N, T, d, generator=g) for _ in range(3))
    planes = torch.randn(L * K, d, generator=g)
    k, q, v = (x.to(dtype) for x in (k, q, v))
    return (k.to(device), q.to(device), v.to(device), planes.to(device))


def oracle_out(oracle, k, q, v, planes, L, K):
    planes_T = planes.cpu().double().numpy().T
    pk = oracle.hash_probs(k.cpu().double().numpy(), planes_T, L, K).reshape(k.shape[0], k.shape[1], -1)
    pq = oracle.hash_probs(q.cpu().double().numpy(), planes_T, L, K).reshape(q.shape[0], q.shape[1], -1)
    return oracle.causal_recurrence(pq, pk, v.cpu().double().numpy())


# (L, K, d): every (S, d) specialization the fused kernels take (S = L 2^K in
# {64, 128, 256}, d in {64, 128}), one, two, three and four 16-plane blocks
# (L K up to 16, 32, 48, 64), and plane counts K = 2 ... 8.
SHAPES = [(4, 4, 64), (2, 5, 64), (8, 3, 64), (16, 2, 64), (8, 4, 128), (4, 5, 128), (8, 5, 128),
          (1, 6, 64), (4, 6, 128),
          (2, 5, 128),   # S = 64, d = 128
          (8, 4, 64),    # S = 128, d = 64, L K = 32
          (16, 4, 64),   # S = 256, d = 64, L K = 64: four plane blocks
          (32, 2, 128),  # S = 128, d = 128, L K = 64
          (1, 7, 64),    # S = 128, K = 7
          (1, 8, 128)]   # S = 256, K = 8


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, K, d", SHAPES)
@pytest.mark.parametrize("T", [1, 63, 65, 300, 1000])
def test_hashed_forward_matches_the_oracle(race, oracle, cuda, dtype, L, K, d, T):
    say("hashed", L, K, d, T, dtype)
    k, q, v, planes = rows_and_planes(2, T, d, L, K, dtype, 100 + T + 7 * L + K, cuda)
    out = race.race_fused_fwd_hashed(k, q, v, planes, L)
    torch.cuda.synchronize()
    ref = oracle_out(oracle, k, q, v, planes, L, K)
    assert per_stream_rel_err(to_np(out), ref) <= tol_for(dtype)


@pytest.mark.parametrize("tile", [64, 128, 1024])
def test_hashed_forward_at_explicit_tiles(race, oracle, cuda, tile):
    # Several tiles per stream: the scan of hashed tile sums is exercised.
    say("hashed tiles", tile)
    k, q, v, planes = rows_and_planes(3, 3000, 64, 4, 4, torch.float32, 7, cuda)
    out = race.race_fused_fwd_hashed(k, q, v, planes, 4, tile_tokens=tile)
    torch.cuda.synchronize()
    assert per_stream_rel_err(to_np(out), oracle_out(oracle, k, q, v, planes, 4, 4)) <= FP32_TOL


def test_hashed_forward_cfg2_full_length(race, oracle, cuda):
    # The cfg2 shape (N = 8, L = 4, R = 16, d = 64, T = 65536, fp32): every
    # stream against the oracle.
    say("hashed cfg2 full length")
    k, q, v, planes = rows_and_planes(8, 65536, 64, 4, 4, torch.float32, 2024, cuda)
    out = race.race_fused_fwd_hashed(k, q, v, planes, 4)
    torch.cuda.synchronize()
    err = per_stream_rel_err(to_np(out), oracle_out(oracle, k, q, v, planes, 4, 4))
    say("hashed cfg2 max rel err", f"{err:.3e}")
    assert err <= FP32_TOL


def test_hashed_forward_bf16_long(race, oracle, cuda):
    # bf16 rows at T = 2^18, N = 8, L = 4, K = 4, d = 64 (rows generated on
    # the GPU): every stream within the north-star bound and the rounding
    # floor bound (max <= 2.5 F, rms <= 2.0 F_rms).
    T = 1 << 18
    say("hashed bf16 long", T)
    gen = torch.Generator(device=cuda).manual_seed(9)
    k, q, v = (torch.randn(8, T, 64, generator=gen, device=cuda).to(torch.bfloat16) for _ in range(3))
    planes = torch.randn(16, 64, generator=gen, device=cuda)
    out = race.race_fused_fwd_hashed(k, q, v, planes, 4)
    torch.cuda.synchronize()
    ref = oracle_out(oracle, k, q, v, planes, 4, 4)
    o = to_np(out)
    err = per_stream_rel_err(o, ref)
    say("hashed bf16 long max rel err", f"{err:.3e}")
    assert err <= tol_for(torch.bfloat16)
    assert_bf16_floor(o, ref, float(v.float().abs().max()), "hashed bf16 long")


def test_hashed_equals_hashing_then_the_op(race, cuda):
    # The fused path and the two-launch path (race_hash_probs, then
    # race_fused_fwd) compute the same function; both are fp32-accurate.
    k, q, v, planes = rows_and_planes(3, 2000, 64, 4, 4, torch.float32, 11, cuda)
    fused = race.race_fused_fwd_hashed(k, q, v, planes, 4)
    pt = planes.t().contiguous()
    two = race.race_fused_fwd(race.race_hash_probs(q, pt, 4, 4), race.race_hash_probs(k, pt, 4, 4), v)
    torch.cuda.synchronize()
    assert per_stream_rel_err(to_np(fused), to_np(two).astype(np.float64)) <= 2e-5


def test_hashed_state_and_records_match_the_probability_path(race, ext, cuda):
    # The state and the tile records are the per-bucket sums of the hashed
    # keys: the same as the probability path's up to fp32 rounding.
    k, q, v, planes = rows_and_planes(2, 1500, 64, 4, 4, torch.float32, 12, cuda)
    out, records, state, tile = ext.hashed_forward(k, q, v, planes, 4, 256, True, True)
    pt = planes.t().contiguous()
    pk, pq = ext.hash_probs(k, pt, 4, 4), ext.hash_probs(q, pt, 4, 4)
    out2, rec2, state2, tile2 = ext.forward_debug(pq, pk, v, True, 256, 3)
    torch.cuda.synchronize()
    assert tile == tile2 == 256 and records.shape == rec2.shape
    scale = state2.abs().max()
    assert (state - state2).abs().max() <= 1e-5 * scale
    assert (records - rec2).abs().max() <= 1e-5 * scale


def test_hashed_is_bitwise_reproducible_and_causal(race, cuda):
    k, q, v, planes = rows_and_planes(2, 900, 64, 4, 4, torch.float32, 13, cuda)
    a = race.race_fused_fwd_hashed(k, q, v, planes, 4)
    b = race.race_fused_fwd_hashed(k, q, v, planes, 4)
    k2, q2, v2 = k.clone(), q.clone(), v.clone()
    for x in (k2, q2, v2):
        x[:, 500:] = torch.randn_like(x[:, 500:])
    c = race.race_fused_fwd_hashed(k2, q2, v2, planes, 4)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(a[:, :500], c[:, :500])


def test_hashed_empty_and_rejected(race, ext, cuda):
    k, q, v, planes = rows_and_planes(2, 0, 64, 4, 4, torch.float32, 1, cuda)
    assert race.race_fused_fwd_hashed(k, q, v, planes, 4).shape == (2, 0, 64)
    k, q, v, planes = rows_and_planes(2, 10, 32, 4, 4, torch.float32, 1, cuda)
    with pytest.raises(RuntimeError, match="race_fused_fwd_hashed: no kernel"):
        race.race_fused_fwd_hashed(k, q, v, planes, 4)
    k, q, v, planes = rows_and_planes(2, 10, 64, 4, 4, torch.float32, 1, cuda)
    with pytest.raises(RuntimeError, match="planes has shape"):
        race.race_fused_fwd_hashed(k, q, v, planes[:15], 4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, K, d", [(4, 4, 64), (2, 3, 16), (3, 1, 8), (8, 5, 128)])
def test_hashing_backward_matches_autograd(race, oracle, cuda, dtype, L, K, d):
    # dx of race_hash_probs against torch.autograd through the fp64
    # composition of src/race_baseline.py:41-44.
    say("hash bwd", L, K, d, dtype)
    g = torch.Generator().manual_seed(5 + L + K + d)
    x = torch.randn(3, 50, d, generator=g).to(dtype)
    planes_T = torch.randn(d, L * K, generator=g)
    dp = torch.randn(3, 50, L, 1 << K, generator=g).to(dtype)
    xd = x.to(cuda).requires_grad_(True)
    probs = race.race_hash_probs(xd, planes_T.to(cuda), L, K)
    probs.backward(dp.to(cuda))
    torch.cuda.synchronize()
    x64 = x.double().requires_grad_(True)
    ref = oracle.torch_hash_probs(x64, planes_T.double(), L, K)
    (dx_ref,) = torch.autograd.grad(ref, (x64,), dp.double())
    err = (xd.grad.double().cpu() - dx_ref).abs().max() / dx_ref.abs().max()
    assert err <= (2e-2 if dtype == torch.bfloat16 else 1e-5), err


@pytest.mark.parametrize("causal", [True, False])
def test_module_gradients_reach_the_rows(race, oracle, cuda, causal):
    # The drop-in BatchedACE trains: gradients w.r.t. Khf, Qhf and Vhf match
    # torch.autograd through the reference's composition (fp64), on the
    # hashed path (causal) and the hash-then-op path (non-causal).
    say("module grads", causal)
    torch.manual_seed(3)
    M, B, T, H, dk, K, L = 1, 2, 96, 2, 64, 4, 4
    ace = race.BatchedACE(dk, K, L, M, device=cuda, causal=causal)
    g = torch.Generator().manual_seed(4)
    Khf, Vhf, Qhf = (torch.randn(M, B, T, H, dk, generator=g) for _ in range(3))
    up = torch.randn(M, B, T, H, dk, generator=g)
    ins = [x.to(cuda).requires_grad_(True) for x in (Khf, Vhf, Qhf)]
    out = ace(*ins)
    out.backward(up.to(cuda))
    torch.cuda.synchronize()
    N = M * B * H

    def flat(x):
        return x.permute(0, 1, 3, 2, 4).reshape(N, T, dk).numpy()

    planes_T = ace.planes_T.cpu().double().numpy()
    if causal:
        ref, dK, dQ, dV = oracle.torch_module_autograd(flat(Khf), flat(Qhf), flat(Vhf), planes_T, L, K,
                                                       flat(up))
    else:
        kt, qt, vt = (torch.as_tensor(flat(x), dtype=torch.float64).requires_grad_(True)
                      for x in (Khf, Qhf, Vhf))
        pt = torch.as_tensor(planes_T)
        o = oracle.torch_noncausal_reference(oracle.torch_hash_probs(qt, pt, L, K).flatten(-2),
                                             oracle.torch_hash_probs(kt, pt, L, K).flatten(-2), vt)
        dK, dQ, dV = (t.numpy() for t in torch.autograd.grad(o, (kt, qt, vt),
                                                              torch.as_tensor(flat(up), dtype=torch.float64)))
        ref = o.detach().numpy()
    got_out = out.detach().cpu().permute(0, 1, 3, 2, 4).reshape(N, T, dk).numpy()
    assert per_stream_rel_err(got_out, ref) <= FP32_TOL
    errs = {}
    for name, got, want in (("dK", ins[0].grad, dK), ("dQ", ins[2].grad, dQ), ("dV", ins[1].grad, dV)):
        errs[name] = per_stream_rel_err(got.cpu().permute(0, 1, 3, 2, 4).reshape(N, T, dk).numpy(), want)
    say("module grad errors", {k: f"{v:.2e}" for k, v in errs.items()})
    # dK of the probabilities is a sum of cancelling terms (the running-mass
    # gradient against the value term), so its error is bounded by the size
    # of those terms, not of the result; through the hashing that gives a
    # looser bound relative to max |dK| than dQ and dV get.
    assert errs["dQ"] <= 1e-4 and errs["dV"] <= 1e-4 and errs["dK"] <= 1e-3
