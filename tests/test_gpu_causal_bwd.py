"""GPU parity of the causal backward against the CPU oracle.

The reference has no causal backward (its design outline is
docs/causal_v2_design.md:689-742); the oracle is the closed-form VJP of
oracle/race_oracle.c, itself pinned to exact dual-number gradients and to
torch.autograd through the reference's cumsum composition
(tests/test_oracle.py).  Gradients are checked here through autograd on
race_fused_fwd(causal=True), against:
  - the oracle on a grid of shapes, ragged T and both dtypes,
  - the exact golden gradients (tests/golden/race_golden.npz),
  - torch.autograd on the reference formula in fp64,
with the properties of the non-causal suite: bitwise reproducibility,
needs_input_grad filtering, independence from the tile length.
"""
from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, assert_bf16_floor, per_stream_rel_err, say, to_np, tol_for

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "race_golden.npz"
# cfg5 dQ and dV (bf16) against k F + atol, k_rms F_rms + rms_atol, F the
# rounding floor of each stream's fp64 gradient: the pair the forward's bf16
# outputs meet.  dK is a difference of terms much larger than itself (T = 1
# gives dK = <v, g> q eps / (k + eps)^2), so its error is not bounded by its
# own rounding floor; it keeps the relative bound.
CFG5_BWD_FLOOR_FACTORS = (2.5, 2.0)


def forward_backward(race, q, k, v, g, cuda):
    qg, kg, vg = (x.to(cuda).requires_grad_(True) for x in (q, k, v))
    out = race.race_fused_fwd(qg, kg, vg, causal=True)
    out.backward(g.to(cuda))
    torch.cuda.synchronize()
    return out.detach(), qg.grad, kg.grad, vg.grad


def dk_term_scale(q, k, v, g, eps=1e-6):
    """Per-stream max over (t, s) of the magnitude of the terms whose sum is
    dK: sum_c |Z_t[s][c]| |v_t[c]| + |Y|_t[s] with |Z|, |Y| the suffix sums of
    |W| (x) |g| and |alpha|.  Where they cancel (T = 1 gives dK = <v, g> q
    eps / (k + eps)^2, ~1e-6 of each term) fp32 is only accurate relative to
    this, so dK's error is bounded by tol * this scale."""
    q, k, v, g = (np.asarray(x, np.float64) for x in (q, k, v, g))
    a = np.cumsum(k, 1)
    b = np.cumsum(k[..., :, None] * v[..., None, :], 1)
    r = 1.0 / (a + eps)
    w = q * r
    alpha = w * r * np.abs(np.einsum("ntsc,ntc->nts", b, g))
    zabs = np.cumsum((np.abs(w)[..., :, None] * np.abs(g)[..., None, :])[:, ::-1], 1)[:, ::-1]
    yabs = np.cumsum(alpha[:, ::-1], 1)[:, ::-1]
    terms = np.einsum("ntsc,ntc->nts", zabs, np.abs(v)) + yabs
    return terms.reshape(terms.shape[0], -1).max(1)


def check_grads(oracle, q, k, v, g, out, dq, dk, dv, tol, dk_scale=True):
    qn, kn, vn, gn = (to_np(x) for x in (q, k, v, g))
    rq, rk, rv = oracle.causal_bwd(qn, kn, vn, gn, nthreads=16)
    assert per_stream_rel_err(to_np(out), oracle.causal_recurrence(qn, kn, vn, nthreads=16)) <= tol
    eq = per_stream_rel_err(to_np(dq), rq)
    ev = per_stream_rel_err(to_np(dv), rv)
    if dk_scale:
        scale = dk_term_scale(qn, kn, vn, gn)
        n = qn.shape[0]
        ek = float((np.abs(to_np(dk).astype(np.float64) - rk).reshape(n, -1).max(1) / scale).max())
    else:
        ek = per_stream_rel_err(to_np(dk), rk)
    say("errors", f"dQ {eq:.2e} dK {ek:.2e} dV {ev:.2e}")
    assert eq <= tol, ("dQ", eq)
    assert ek <= tol, ("dK", ek)
    assert ev <= tol, ("dV", ev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d", [(1, 1, 1), (2, 8, 32), (4, 16, 64), (3, 5, 7), (8, 32, 64),
                                     (4, 32, 128), (8, 32, 128), (4, 64, 128), (2, 128, 120)])
@pytest.mark.parametrize("T", [1, 63, 65, 700])
def test_shapes(race, oracle, cuda, dtype, L, R, d, T):
    # Through autograd, so the backward starts from the forward's saved
    # records: for (4, 32, 128) those come from the MFMA tile sums of S = d =
    # 128, for S = d = 64 from the register-direct ones, else the VALU sums.
    # S = 256 with d = 128 (cfg5) or d = 120: the state of all d columns does
    # not fit one workgroup's LDS, the walks take two column groups (of 64 or
    # 60 columns).
    say("c-bwd-shape", dtype, L, R, d, T)
    q, k, v, g = race.make_inputs(3, T, L, R, d, seed=T + d + 1, dtype=dtype, grad_out=True)
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    assert dq.dtype == dtype and dk.dtype == dtype and dv.dtype == dtype
    check_grads(oracle, q, k, v, g, out, dq, dk, dv, tol_for(dtype))


def test_cfg2_shape_full_length(race, oracle, cuda):
    # The whole cfg2 shape (N = 8, S = 64, d = 64, fp32, T = 65536): 64 tiles
    # per stream, every stream, the north-star fp32 bound on dQ, dK and dV.
    say("c-bwd cfg2 T=65536")
    q, k, v = race.make_inputs(8, 65536, 4, 16, 64, seed=23, device=cuda, gen_device="cuda")
    g = torch.randn(v.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(24))
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    check_grads(oracle, q, k, v, g, out, dq, dk, dv, FP32_TOL, dk_scale=False)


def test_cfg2_shape_long_sequence(race, oracle, cuda):
    # The cfg2 shape (N = 8, S = 64, d = 64, fp32) at T = 16384: 32 tiles per
    # stream, so the suffix scan crosses many tile boundaries.
    say("c-bwd cfg2 T=16384")
    q, k, v, g = race.make_inputs(8, 16384, 4, 16, 64, seed=21, grad_out=True)
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    check_grads(oracle, q, k, v, g, out, dq, dk, dv, FP32_TOL, dk_scale=False)


@pytest.mark.parametrize("tile", [64, 128, 1024])
def test_tile_lengths(race, oracle, cuda, tile):
    say("c-bwd tile", tile)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, 1500, 4, 16, 64, seed=22, grad_out=True))
    dq, dk, dv = race.race_causal_backward(q, k, v, g, tile_tokens=tile)
    out = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    check_grads(oracle, q, k, v, g, out, dq, dk, dv, FP32_TOL)


@pytest.mark.parametrize("L, R", [(4, 32), (8, 32)])
@pytest.mark.parametrize("tile", [64, 256, 1024])
def test_block_walks_at_explicit_tiles(race, oracle, cuda, L, R, tile):
    # bf16, d = 128, S = 128 and 256: the walks over 128 x 128 blocks with
    # many tiles per stream (the reverse scan of the block's four record
    # arrays crosses them) and a ragged last tile and sub-chunk.
    say("c-bwd block tile", L, R, tile)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, 1500, L, R, 128, seed=26, dtype=torch.bfloat16,
                                                         grad_out=True))
    dq, dk, dv = race.race_causal_backward(q, k, v, g, tile_tokens=tile)
    out = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    check_grads(oracle, q, k, v, g, out, dq, dk, dv, tol_for(torch.bfloat16))


def test_block_walks_many_streams(race, oracle, cuda):
    # S = 256: the reverse scan takes the suffix records of both 128-bucket
    # blocks as 8 N record streams, past the 65535 streams of one scan launch
    # for N > 8191; it runs in launches of at most 65535.  Record stream
    # (4 b + a) N + n (block b, array a) of the streams checked here falls on
    # both sides of the launch boundaries (65535 and 131070 at N = 16400).
    N, T = 16400, 40
    say("c-bwd block many streams", N, T)
    q, k, v = race.make_inputs(N, T, 8, 32, 128, seed=28, dtype=torch.bfloat16, device=cuda, gen_device="cuda")
    g = torch.randn(v.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(29)).to(v.dtype)
    dq, dk, dv = race.race_causal_backward(q, k, v, g)
    torch.cuda.synchronize()
    pick = [0, 8000, 16269, 16270, 16334, 16335, 16399]
    qn, kn, vn, gn = (to_np(x[pick]) for x in (q, k, v, g))
    rq, rk, rv = oracle.causal_bwd(qn, kn, vn, gn, nthreads=16)
    errs = [per_stream_rel_err(to_np(x[pick]), r) for x, r in ((dq, rq), (dk, rk), (dv, rv))]
    say("c-bwd many streams errors", *(f"{e:.2e}" for e in errs))
    assert max(errs) <= tol_for(torch.bfloat16)


@pytest.mark.parametrize("R", [16, 32])
def test_block_walks_whole_streams_and_tiled(race, oracle, cuda, R):
    # With the streams times the 128-bucket blocks covering the device's CUs,
    # each forward walk goes through its whole stream from a zero prefix (the
    # forward's tile sums and scan, or the saved records, are not used), from
    # the inputs and through autograd; one stream fewer walks tile by tile.
    # Four 256-token tiles, the last one ragged; all against the oracle VJP
    # on a sample of streams.
    S = 8 * R
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    N, T, tile = -(-cus // (S // 128)), 1000, 256
    say("c-bwd whole streams", N, T, S, tile)
    q, k, v = race.make_inputs(N, T, 8, R, 128, seed=31 + R, dtype=torch.bfloat16, device=cuda, gen_device="cuda")
    g = torch.randn(v.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(32 + R)).to(v.dtype)
    whole = race.race_causal_backward(q, k, v, g, tile_tokens=tile)
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    race.race_fused_fwd(qg, kg, vg, causal=True, tile_tokens=tile).backward(g)
    # One stream fewer than the CUs need: the tiled walks after the tile sums and scan.
    tiled = race.race_causal_backward(*(x[: N - 1] for x in (q, k, v, g)), tile_tokens=tile)
    torch.cuda.synchronize()
    pick = [0, 1, N // 2, N - 2]
    qn, kn, vn, gn = (to_np(x[pick]) for x in (q, k, v, g))
    refs = oracle.causal_bwd(qn, kn, vn, gn, nthreads=16)
    for name, grads in (("whole", whole), ("autograd", (qg.grad, kg.grad, vg.grad)), ("tiled", tiled)):
        errs = [per_stream_rel_err(to_np(x[pick]), r) for x, r in zip(grads, refs)]
        say("c-bwd", name, *(f"{e:.2e}" for e in errs))
        assert max(errs) <= tol_for(torch.bfloat16)


def test_block_walks_bitwise_reproducible(race, cuda):
    say("c-bwd block bitwise")
    q, k, v, g = race.make_inputs(3, 2100, 8, 32, 128, seed=27, dtype=torch.bfloat16, grad_out=True)
    first = forward_backward(race, q, k, v, g, cuda)
    for _ in range(2):
        again = forward_backward(race, q, k, v, g, cuda)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("T", [1, 31, 33, 100, 2000])
def test_kernel_families(race, oracle, cuda, dtype, kernel, T):
    # Both kernel families at S = d = 64 (the matrix-core specialization),
    # ragged T around the 32-token sub-chunk.
    say("c-bwd family", kernel, dtype, T)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(3, T, 4, 16, 64, seed=28 + T, dtype=dtype,
                                                       grad_out=True))
    dq, dk, dv = race.race_causal_backward(q, k, v, g, kernel=kernel)
    out = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    check_grads(oracle, q, k, v, g, out, dq, dk, dv, tol_for(dtype))


@pytest.mark.parametrize("name", ["cgrad", "cgrad_wide"])
def test_golden_gradients(race, cuda, name):
    say("c-bwd golden", name)
    gd = np.load(GOLDEN)
    q, k, v, g = (torch.from_numpy(gd[f"{name}_{x}"]) for x in "qkvg")
    _, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    assert per_stream_rel_err(to_np(dq), gd[f"{name}_dq"]) <= 1e-5
    assert per_stream_rel_err(to_np(dk), gd[f"{name}_dk"]) <= 1e-5
    assert per_stream_rel_err(to_np(dv), gd[f"{name}_dv"]) <= 1e-5


def test_matches_torch_autograd(race, oracle, cuda):
    say("c-bwd autograd")
    q, k, v, g = race.make_inputs(4, 300, 4, 16, 64, seed=23, grad_out=True)
    out, dq, dk, dv = forward_backward(race, q, k, v, g, cuda)
    a_out, aq, ak, av = oracle.torch_causal_autograd(to_np(q), to_np(k), to_np(v), to_np(g))
    for got, want in ((out, a_out), (dq, aq), (dk, ak), (dv, av)):
        assert per_stream_rel_err(to_np(got), want) <= FP32_TOL


@pytest.mark.parametrize("need", [(True, False, False), (False, True, False), (False, False, True),
                                  (False, True, True)])
@pytest.mark.parametrize("L, R, d, dtype", [(4, 16, 64, torch.float32), (4, 32, 128, torch.bfloat16),
                                            (8, 32, 128, torch.bfloat16)])
def test_only_requested_gradients(race, cuda, need, L, R, d, dtype):
    # bf16 with d = 128: walks over 128-bucket x 128-column blocks, one block
    # at S = 128 (4, 32) and two at S = 256 (8, 32), whose dV goes through a
    # running sum over the blocks.
    say("c-bwd needs-grad", need, L, R, d, dtype)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, 500, L, R, d, seed=24, dtype=dtype, grad_out=True))
    leaves = [x.clone().requires_grad_(n) for x, n in zip((q, k, v), need)]
    race.race_fused_fwd(*leaves, causal=True).backward(g)
    _, fq, fk, fv = forward_backward(race, q, k, v, g, cuda)
    for leaf, n, full in zip(leaves, need, (fq, fk, fv)):
        if n:
            assert torch.equal(leaf.grad, full)
        else:
            assert leaf.grad is None


def test_bitwise_reproducible(race, cuda):
    say("c-bwd bitwise")
    q, k, v, g = race.make_inputs(5, 3000, 4, 16, 64, seed=25, grad_out=True)
    first = forward_backward(race, q, k, v, g, cuda)
    for _ in range(2):
        again = forward_backward(race, q, k, v, g, cuda)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


def test_future_gradients_do_not_reach_past_queries(race, cuda):
    # dQ at token t depends on dOut at t only: zeroing dOut after t leaves
    # dQ[:t] bitwise unchanged.
    say("c-bwd dq locality")
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, 900, 4, 16, 64, seed=26, grad_out=True))
    g2 = g.clone()
    g2[:, 600:] = 0
    dq1, _, _ = race.race_causal_backward(q, k, v, g, need=(True, False, False))
    dq2, _, _ = race.race_causal_backward(q, k, v, g2, need=(True, False, False))
    torch.cuda.synchronize()
    assert torch.equal(dq1[:, :600], dq2[:, :600])


def test_mfma_backward_needs_its_specialization(race, cuda):
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(1, 64, 2, 8, 32, seed=29, grad_out=True))
    with pytest.raises(RuntimeError, match="race_causal_bwd"):
        race.race_causal_backward(q, k, v, g, kernel="mfma")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d", [(8, 32, 128), (4, 32, 128), (8, 32, 64), (2, 32, 128)])
def test_matrix_core_blocks_agree_with_the_vector_alu(race, oracle, cuda, dtype, L, R, d):
    # S, d multiples of 64 above 64 run the matrix-core kernels in 64 x 64
    # blocks; the vector-ALU walks (forced) compute the same gradients.
    say("c-bwd blocks", L, R, d, dtype)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, 777, L, R, d, seed=50 + d, dtype=dtype,
                                                       grad_out=True))
    got = race.race_causal_backward(q, k, v, g, kernel="mfma")
    ref = race.race_causal_backward(q, k, v, g, kernel="valu")
    out = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    check_grads(oracle, q, k, v, g, out, *got, tol_for(dtype))
    for name, a, b in (("dQ", got[0], ref[0]), ("dV", got[2], ref[2])):
        assert per_stream_rel_err(to_np(a), to_np(b).astype(np.float64)) <= 2 * tol_for(dtype), name


def test_unsupported_shape_raises(race, cuda):
    # S = 512: past the library's 256 buckets.
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(1, 64, 4, 128, 8, seed=27, grad_out=True))
    with pytest.raises(RuntimeError, match="race_causal_backward: no kernel takes"):
        race.race_causal_backward(q, k, v, g)


def test_cfg5_shape_backward(race, oracle, cuda):
    # cfg5 (N = 128, L = 8, R = 32, d = 128, T = 16384, bf16) through
    # autograd and from the inputs: the walks over two 128 x 128 blocks (N x 2
    # blocks covers the CUs of an MI355X, so the forward walks go through
    # whole streams); 16 streams against the oracle VJP.
    say("c-bwd cfg5")
    q, k, v = race.make_inputs(128, 16384, 8, 32, 128, seed=5, dtype=torch.bfloat16, device=cuda,
                               gen_device="cuda")
    g = torch.randn(v.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(6)).to(v.dtype)
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    race.race_fused_fwd(qg, kg, vg, causal=True).backward(g)
    inputs = race.race_causal_backward(q, k, v, g)
    torch.cuda.synchronize()
    # 16 streams spread over the batch, heads and both ends of the stream range.
    pick = [0, 9, 17, 26, 34, 41, 50, 58, 67, 75, 86, 93, 101, 110, 119, 127]
    qn, kn, vn, gn = (to_np(x[pick]) for x in (q, k, v, g))
    rq, rk, rv = oracle.causal_bwd(qn, kn, vn, gn, nthreads=16)
    for how, (dq, dk, dv) in (("autograd", (qg.grad, kg.grad, vg.grad)), ("inputs", inputs)):
        errs = [per_stream_rel_err(to_np(x[pick]), r) for x, r in ((dq, rq), (dk, rk), (dv, rv))]
        say("c-bwd cfg5 errors", how, *(f"{e:.2e}" for e in errs))
        assert max(errs) <= tol_for(torch.bfloat16)
        # Against the rounding floor of the bf16 gradients, stream by stream.
        for name, x, r in (("dQ", dq, rq), ("dV", dv, rv)):
            got = to_np(x[pick])
            for j in range(len(pick)):
                assert_bf16_floor(got[j], r[j], float(np.abs(r[j]).max()), f"cfg5 {how} {name} stream {pick[j]}",
                                  factors=CFG5_BWD_FLOOR_FACTORS)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d, T", [(4, 16, 64, 3000), (2, 8, 32, 700), (3, 5, 7, 200),
                                        (4, 32, 128, 1500), (8, 32, 128, 1100)])
def test_backward_from_saved_records_equals_recomputing_them(race, ext, cuda, dtype, L, R, d, T):
    # Autograd keeps the forward's scanned tile records and the backward
    # starts from them; recomputing them at the same tile length runs the
    # same sums and scan, so the gradients are bitwise equal.
    say("c-bwd records", L, R, d, T, dtype)
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(2, T, L, R, d, seed=40 + T, dtype=dtype,
                                                       grad_out=True))
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    race.race_fused_fwd(qg, kg, vg, causal=True).backward(g)
    _, records, tile = ext.forward_with_records(q, k, v)
    dq, dk, dv = race.race_causal_backward(q, k, v, g, tile_tokens=tile)
    torch.cuda.synchronize()
    assert records.shape == (2, -(-T // tile), records.shape[2])
    for got, want in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
        assert torch.equal(got, want)


def test_saved_records_must_match_the_tile_length(race, ext, cuda):
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(1, 1000, 4, 16, 64, seed=41, grad_out=True))
    _, records, tile = ext.forward_with_records(q, k, v, tile_tokens=128)
    with pytest.raises(RuntimeError, match="fwd_records has 8 tiles; the tile length 256 gives 4"):
        ext.causal_backward(q, k, v, g, True, True, True, 256, 0, records)
    with pytest.raises(RuntimeError, match="tile length"):
        ext.causal_backward(q, k, v, g, True, True, True, 0, 0, records)
    # Records written for another (S, d) at the same tile count are refused on
    # the host, before any kernel would index them with this shape's record size.
    q2, k2, v2, g2 = (x.to(cuda) for x in race.make_inputs(1, 1000, 4, 16, 32, seed=41,
                                                           grad_out=True))
    with pytest.raises(RuntimeError, match="records of .* floats; this \\(S, d\\) needs"):
        ext.causal_backward(q2, k2, v2, g2, True, True, True, 128, 0, records)


@pytest.mark.parametrize("N, T", [(0, 5), (2, 0), (0, 0)])
def test_autograd_backward_of_empty_inputs(race, cuda, N, T):
    # Empty inputs: the forward keeps (empty) records with the tile count the
    # backward expects, and the gradients come back empty.
    q, k, v, g = (x.to(cuda) for x in race.make_inputs(N, T, 4, 16, 64, seed=3, grad_out=True))
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    race.race_fused_fwd(qg, kg, vg, causal=True).backward(g)
    torch.cuda.synchronize()
    for x, grad in ((q, qg.grad), (k, kg.grad), (v, vg.grad)):
        assert grad.shape == x.shape
