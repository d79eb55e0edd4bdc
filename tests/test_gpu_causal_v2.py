"""GPU parity of the Algorithm-1 forward (hashing inside, global
normalization), the drop-in for the reference's causal v2 extension.

The cases follow the reference's own suite (src/causal_v2/tests/
test_forward_cuda.py:79-318): every head dim, plane and table count over
ragged sequence lengths and three betas, the two rounding variants against
each other, forced tile lengths, exact closed forms (constant V, T = 1),
bitwise causality and reproducibility, the prefix states of forward_debug,
stream isolation, beta on either device, automatic tiles, the empty
sequence and the rejected inputs.  The reference is the fp64 oracle
(oracle.alg1_causal, pinned on the CPU in tests/test_oracle_alg1.py) on the
same bf16 inputs.

Output tolerance, after the reference's (src/causal_v2/tests/
causal_numerics.py:1-30): with F = max|bf16(ref) - ref| and F_rms the RMS of
the same rounding errors, max|o - ref| <= k F + 1e-5 max(1, beta) max|v| and
rms|o - ref| <= k_rms F_rms + 1e-7 max|v|, with (k, k_rms) = (1.1, 1.05) for
the fp32 variant and (2.5, 2.0) for the bf16 one.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu

FACTORS = {"fp32": (1.1, 1.05), "bf16": (2.5, 2.0)}
ATOL_FACTOR = 1e-5
RMS_ATOL_FACTOR = 1e-7
STATE_RTOL = {"fp32": 3e-5, "bf16": 2.0 ** -8 + 3e-5}
STATE_MASS_ATOL = 1e-6


@pytest.fixture(params=["fp32", "bf16"])
def variant(request) -> str:
    return request.param


def tc(variant: str) -> bool:
    return variant == "bf16"


def make_inputs(seed, batch, heads, T, D, L, P, device="cuda"):
    """bf16 q, k, v [B, H, T, D] and fp32 planes W [L, P, D], all N(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(batch, heads, T, D, generator=g).to(torch.bfloat16) for _ in range(3))
    W = torch.randn(L, P, D, generator=g)
    return q.to(device), k.to(device), v.to(device), W.to(device)


def reference(oracle, q, k, v, W, beta, **kw):
    """fp64 oracle on the bf16 values; [B, H, T, D] like q."""
    B, H, T, D = q.shape
    res = oracle.alg1_causal(*(x.float().cpu().numpy().reshape(B * H, T, D) for x in (q, k, v)),
                             W.float().cpu().numpy(), float(beta), nthreads=16, **kw)
    if isinstance(res, tuple):
        return (res[0].reshape(B, H, T, D),) + res[1:]
    return res.reshape(B, H, T, D)


def rounding_floor(ref: np.ndarray):
    r = torch.from_numpy(ref).to(torch.bfloat16).double().numpy()
    e = np.abs(r - ref)
    return e.max(), math.sqrt(float((e ** 2).mean()))


def check_error(err: np.ndarray, F, F_rms, k, k_rms, atol, rms_atol, label):
    emax, erms = float(err.max()), math.sqrt(float((err ** 2).mean()))
    assert emax <= k * F + atol, f"{label}: max {emax:.3e} > {k * F + atol:.3e} ({emax / max(F, 1e-30):.3f} F)"
    assert erms <= k_rms * F_rms + rms_atol, (
        f"{label}: rms {erms:.3e} > {k_rms * F_rms + rms_atol:.3e} ({erms / max(F_rms, 1e-30):.3f} F_rms)")


def assert_within_floor(out, ref, v, beta, variant):
    k, k_rms = FACTORS[variant]
    F, F_rms = rounding_floor(ref)
    vmax = float(v.float().abs().max())
    o = out.double().cpu().numpy()
    say("error", variant, f"{np.abs(o - ref).max() / max(F, 1e-30):.3f} F")
    check_error(np.abs(o - ref), F, F_rms, k, k_rms, ATOL_FACTOR * max(1.0, beta) * vmax,
                RMS_ATOL_FACTOR * vmax, variant)


def skip_unless_fits(race, D, P, L, variant):
    if not race.causal_v2.fits_on_device(D, P, L, tc(variant)):
        pytest.skip(f"output pass needs {race.causal_v2.output_pass_smem_bytes(D, P, L, tc(variant))} bytes")


def betas_for(D):
    return [1.0 / math.sqrt(D), 1.0, 2.0]


@pytest.mark.parametrize("bh", [(1, 1), (2, 4)])
@pytest.mark.parametrize("T", [1, 63, 64, 65, 2047, 2049, 4097])
@pytest.mark.parametrize("L", [1, 2, 4])
@pytest.mark.parametrize("P", [1, 2, 4, 5])
@pytest.mark.parametrize("D", [64, 128])
def test_forward_matches_reference(race, oracle, variant, D, P, L, T, bh):
    skip_unless_fits(race, D, P, L, variant)
    say("alg1", variant, D, P, L, T, bh)
    q, k, v, W = make_inputs(D * 1000 + P * 100 + L * 10 + T + bh[1], *bh, T, D, L, P)
    for beta in betas_for(D):
        out = race.causal_v2.forward(q, k, v, W, torch.tensor(beta, device="cuda"), tensor_cores=tc(variant))
        assert out.dtype == torch.bfloat16 and out.shape == q.shape
        assert torch.isfinite(out).all()
        assert_within_floor(out, reference(oracle, q, k, v, W, beta), v, beta, variant)


@pytest.mark.parametrize("D, P, L", [(64, 4, 4), (128, 5, 2), (64, 1, 1), (128, 3, 3)])
def test_long_sequence(race, oracle, variant, D, P, L):
    # T = 20000: several tiles per stream at the automatic tile length.
    say("alg1 long", variant, D, P, L)
    q, k, v, W = make_inputs(D + P + L, 1, 2, 20000, D, L, P)
    beta = 1.0 / math.sqrt(D)
    out = race.causal_v2.forward(q, k, v, W, torch.tensor(beta), tensor_cores=tc(variant))
    assert_within_floor(out, reference(oracle, q, k, v, W, beta), v, beta, variant)


@pytest.mark.parametrize("T", [1, 65, 2049, 20000])
@pytest.mark.parametrize("D, P, L", [(64, 4, 4), (128, 4, 4), (64, 1, 1), (64, 5, 3), (128, 5, 2)])
def test_variants_agree(race, oracle, D, P, L, T):
    # Each variant is checked against the reference above; against each other
    # the bound is the sum of the two (triangle inequality).
    say("alg1 agree", D, P, L, T)
    q, k, v, W = make_inputs(T + D + P + L, 1, 3, T, D, L, P)
    for beta in betas_for(D):
        a = race.causal_v2.forward(q, k, v, W, torch.tensor(beta))
        b = race.causal_v2.forward(q, k, v, W, torch.tensor(beta), tensor_cores=True)
        ref = reference(oracle, q, k, v, W, beta)
        F, F_rms = rounding_floor(ref)
        vmax = float(v.float().abs().max())
        err = np.abs(b.double().cpu().numpy() - a.double().cpu().numpy())
        check_error(err, F, F_rms, 2.5 + 1.1, 2.0 + 1.05, 2 * ATOL_FACTOR * max(1.0, beta) * vmax,
                    2 * RMS_ATOL_FACTOR * vmax, "bf16 vs fp32")


@pytest.mark.parametrize("T", [1, 2, 15, 17, 127, 129, 2047, 2049, 3 * 2048 + 17, 10000])
@pytest.mark.parametrize("D, P, L", [(64, 4, 4), (128, 4, 4), (64, 5, 3), (64, 3, 3), (128, 3, 2)])
def test_forced_tile_lengths_agree(race, oracle, variant, D, P, L, T):
    say("alg1 tiles", variant, D, P, L, T)
    chunk = race.causal_v2.sub_chunk_tokens(D, P, tc(variant))
    q, k, v, W = make_inputs(T * 7 + D + P, 1, 3, T, D, L, P)
    beta = 0.5
    ref = reference(oracle, q, k, v, W, beta)
    outs = []
    for tile in (chunk, 2 * chunk, 2048):
        out = race.causal_v2.forward(q, k, v, W, torch.tensor(beta), tile_tokens=tile, tensor_cores=tc(variant))
        assert_within_floor(out, ref, v, beta, variant)
        outs.append(out.double())
    allowance = ATOL_FACTOR * max(1.0, beta) * float(v.float().abs().max())
    for other in outs[1:]:
        ulp = torch.maximum(outs[0].abs(), other.abs()) * 2.0 ** -7
        assert ((outs[0] - other).abs() <= ulp + allowance).all()


@pytest.mark.parametrize("T", [1, 65, 2049, 20000])
@pytest.mark.parametrize("beta", [0.125, 1.0, 2.0])
@pytest.mark.parametrize("D, P, L", [(64, 4, 4), (128, 5, 2), (64, 1, 1)])
def test_constant_values_come_back_exactly(race, variant, D, P, L, T, beta):
    # The output is a convex combination of the values: V = c returns c.
    q, k, _, W = make_inputs(T + int(beta * 8) + D, 2, 2, T, D, L, P)
    v = torch.full_like(q, 0.7)
    out = race.causal_v2.forward(q, k, v, W, torch.tensor(beta), tensor_cores=tc(variant))
    assert torch.equal(out, v)


@pytest.mark.parametrize("D, P", [(64, 4), (128, 2)])
def test_first_output_is_the_first_value(race, variant, D, P):
    q, k, v, W = make_inputs(11, 2, 3, 1, D, 2, P)
    assert torch.equal(race.causal_v2.forward(q, k, v, W, torch.tensor(1.0), tensor_cores=tc(variant)), v)


@pytest.mark.parametrize("position", [0, 31, 63, 64, 2047, 2048, 5000])
def test_future_tokens_do_not_change_the_past(race, variant, position):
    say("alg1 causality", variant, position)
    T = 6000
    q, k, v, W = make_inputs(12, 1, 2, T, 64, 4, 4)
    beta = torch.tensor(1.0)
    g = torch.Generator().manual_seed(position)
    future = torch.arange(position + 1, T)
    shuffled = future[torch.randperm(len(future), generator=g)]
    k2, v2 = k.clone(), v.clone()
    k2[:, :, future] = (3.0 * k[:, :, shuffled].float()).to(torch.bfloat16)
    v2[:, :, future] = -v[:, :, shuffled]
    for tile in (64, 2048):
        out = race.causal_v2.forward(q, k, v, W, beta, tile_tokens=tile, tensor_cores=tc(variant))
        out2 = race.causal_v2.forward(q, k2, v2, W, beta, tile_tokens=tile, tensor_cores=tc(variant))
        assert torch.equal(out[:, :, : position + 1], out2[:, :, : position + 1])
        assert not torch.equal(out[:, :, position + 1:], out2[:, :, position + 1:])


@pytest.mark.parametrize("T", [129, 10000, 70000])
def test_runs_are_bitwise_identical(race, variant, T):
    q, k, v, W = make_inputs(13, 2, 4, T, 64, 4, 4)
    beta = torch.tensor(1.0, device="cuda")
    first = race.causal_v2.forward_debug(q, k, v, W, beta, tensor_cores=tc(variant))
    for _ in range(3):
        again = race.causal_v2.forward_debug(q, k, v, W, beta, tensor_cores=tc(variant))
        for a, b in zip(first[:5], again[:5]):
            assert torch.equal(a, b)
        assert first[5] == again[5]


def assert_states_close(mass, values, ref_mass, ref_values, vmax_per_stream, T, variant):
    """A [..., L, R] and B [..., L, R, D] (fp32) against fp64 references:
    |X - X_ref| <= rtol |A_ref| + 1e-6 T (times max|v| of the stream for B)."""
    mass = mass.double().cpu().numpy()
    values = values.double().cpu().numpy()
    bound = STATE_RTOL[variant] * np.abs(ref_mass) + STATE_MASS_ATOL * T
    assert (np.abs(mass - ref_mass) / bound).max() <= 1.0
    vb = bound[..., None] * vmax_per_stream
    assert (np.abs(values - ref_values) / vb).max() <= 1.0


@pytest.mark.parametrize("T, tile", [(1, 0), (777, 64), (5000, 128), (20000, 0), (20000, 2048)])
@pytest.mark.parametrize("D, P, L", [(64, 4, 4), (128, 5, 2), (64, 2, 3)])
def test_debug_prefix_states_match_oracle(race, oracle, variant, D, P, L, T, tile):
    skip_unless_fits(race, D, P, L, variant)
    say("alg1 debug", variant, D, P, L, T, tile)
    q, k, v, W = make_inputs(T + D * 3 + P + L, 1, 2, T, D, L, P)
    beta = 1.0
    out, pA, pB, fA, fB, used = race.causal_v2.forward_debug(q, k, v, W, torch.tensor(beta), tile_tokens=tile,
                                                            tensor_cores=tc(variant))
    chunk = race.causal_v2.sub_chunk_tokens(D, P, tc(variant))
    assert used % chunk == 0 and (tile == 0 or used == tile)
    tiles = -(-T // used)
    R = 1 << P
    S = L * R
    assert pA.shape == (1, 2, tiles, L, R) and pB.shape == (1, 2, tiles, L, R, D)
    assert fA.shape == (1, 2, L, R) and fB.shape == (1, 2, L, R, D)
    ref, pref, fin = reference(oracle, q, k, v, W, beta, tile=used)
    assert not pA[:, :, 0].any() and not pB[:, :, 0].any()
    vmax = v.float().abs().amax(dim=(2, 3)).double().cpu().numpy().reshape(1, 2, 1, 1, 1)
    ref_pB = pref[..., : S * D].reshape(1, 2, tiles, L, R, D)
    ref_pA = pref[..., S * D:].reshape(1, 2, tiles, L, R)
    assert_states_close(pA, pB, ref_pA, ref_pB, vmax[..., None], T, variant)
    ref_fB = fin[..., : S * D].reshape(1, 2, L, R, D)
    ref_fA = fin[..., S * D:].reshape(1, 2, L, R)
    assert_states_close(fA, fB, ref_fA, ref_fB, vmax.reshape(1, 2, 1, 1, 1), T, variant)
    assert_within_floor(out, ref, v, beta, variant)
    assert torch.equal(out, race.causal_v2.forward(q, k, v, W, torch.tensor(beta), tile_tokens=used,
                                                   tensor_cores=tc(variant)))


@pytest.mark.parametrize("T0, T1, tile", [(0, 65, 0), (63, 1, 0), (777, 300, 64), (2049, 4000, 0),
                                          (5000, 1, 128), (64, 64, 64)])
@pytest.mark.parametrize("D, P, L", [(64, 4, 4), (128, 5, 2), (64, 2, 3)])
def test_carried_state_continues_the_sequence(race, oracle, variant, D, P, L, T0, T1, tile):
    # The hand-off: forward_debug's final state over the first T0 tokens, then
    # forward_carry over the next T1 from it.  The continued outputs and the
    # state after them are the unsplit run's (fp64 oracle over all T0 + T1).
    skip_unless_fits(race, D, P, L, variant)
    say("alg1 carry", variant, D, P, L, T0, T1, tile)
    q, k, v, W = make_inputs(T0 * 3 + T1 + D + P + L, 1, 2, T0 + T1, D, L, P)
    beta = 1.0
    bt = torch.tensor(beta)
    head = [x[:, :, :T0].contiguous() for x in (q, k, v)]
    tail = [x[:, :, T0:].contiguous() for x in (q, k, v)]
    _, _, _, fA, fB, _ = race.causal_v2.forward_debug(*head, W, bt, tile_tokens=tile, tensor_cores=tc(variant))
    out, gA, gB = race.causal_v2.forward_carry(*tail, W, bt, fA, fB, tile_tokens=tile, tensor_cores=tc(variant))
    assert out.shape == tail[0].shape and out.dtype == torch.bfloat16
    ref, _, fin = reference(oracle, q, k, v, W, beta, tile=64)
    assert_within_floor(out, np.ascontiguousarray(ref[:, :, T0:]), tail[2], beta, variant)
    R, S = 1 << P, L << P
    vmax = v.float().abs().amax(dim=(2, 3)).double().cpu().numpy().reshape(1, 2, 1, 1)
    assert_states_close(gA, gB, fin[..., S * D:].reshape(1, 2, L, R), fin[..., : S * D].reshape(1, 2, L, R, D),
                        vmax[..., None], T0 + T1, variant)
    # A zero state is no state: the carry from zeros is the plain forward.
    z, _, _ = race.causal_v2.forward_carry(*tail, W, bt, torch.zeros_like(fA), torch.zeros_like(fB),
                                           tile_tokens=tile, tensor_cores=tc(variant))
    assert torch.equal(z, race.causal_v2.forward(*tail, W, bt, tile_tokens=tile, tensor_cores=tc(variant)))


def test_carry_rejects_bad_states(race, variant):
    q, k, v, W = make_inputs(3, 1, 2, 10, 64, 2, 3)
    A = torch.zeros(1, 2, 2, 8, device="cuda")
    Bs = torch.zeros(1, 2, 2, 8, 64, device="cuda")
    with pytest.raises(RuntimeError, match="state_A"):
        race.causal_v2.forward_carry(q, k, v, W, torch.tensor(1.0), A[:, :, :1], Bs, tensor_cores=tc(variant))
    with pytest.raises(RuntimeError, match="state_B"):
        race.causal_v2.forward_carry(q, k, v, W, torch.tensor(1.0), A, Bs.double(), tensor_cores=tc(variant))


def test_other_streams_cannot_leak_into_a_stream(race, oracle, variant):
    T = 3000
    q, k, v, W = make_inputs(14, 1, 3, T, 64, 4, 4)
    for t in (q, k, v):
        t[:, 1:] = float("nan")
    out = race.causal_v2.forward(q, k, v, W, torch.tensor(1.0), tile_tokens=128, tensor_cores=tc(variant))
    assert torch.isfinite(out[:, 0]).all()
    ref = reference(oracle, q[:, :1], k[:, :1], v[:, :1], W, 1.0)
    assert_within_floor(out[:, :1], ref, v[:, :1], 1.0, variant)


def test_beta_on_cpu_matches_beta_on_gpu(race, variant):
    q, k, v, W = make_inputs(15, 1, 1, 777, 128, 2, 2)
    on_gpu = race.causal_v2.forward(q, k, v, W, torch.tensor(0.5, device="cuda"), tensor_cores=tc(variant))
    on_cpu = race.causal_v2.forward(q, k, v, W, torch.tensor(0.5, dtype=torch.float64), tensor_cores=tc(variant))
    assert torch.equal(on_gpu, on_cpu)


def test_large_beta_stays_finite(race, oracle, variant):
    # sigma(+-2 beta u) is formed from exp(-|2 beta u|): no overflow at large beta.
    q, k, v, W = make_inputs(19, 1, 2, 500, 64, 2, 3)
    for beta in (30.0, 100.0):
        out = race.causal_v2.forward(q, k, v, W, torch.tensor(beta), tensor_cores=tc(variant))
        assert torch.isfinite(out).all()


def test_automatic_tile_lengths(race, variant):
    for D, P in ((64, 4), (128, 5)):
        if not race.causal_v2.fits_on_device(D, P, 2, tc(variant)):
            continue
        chunk = race.causal_v2.sub_chunk_tokens(D, P, tc(variant))
        assert race.causal_v2.select_tile_tokens(1, 100, D, P, 2, tc(variant)) == chunk
        large = race.causal_v2.select_tile_tokens(8, 1 << 21, D, P, 2, tc(variant))
        assert large % chunk == 0 and chunk <= large <= 4096


def test_empty_sequence(race, variant):
    q, k, v, W = make_inputs(16, 1, 2, 0, 64, 2, 2)
    out, pA, pB, fA, fB, tile = race.causal_v2.forward_debug(q, k, v, W, torch.tensor(1.0),
                                                            tensor_cores=tc(variant))
    assert out.shape == q.shape and tile == 0
    assert pA.shape[2] == 0 and not fA.any() and not fB.any()


def test_rejects_invalid_inputs(race, variant):
    q, k, v, W = make_inputs(17, 1, 1, 64, 64, 2, 2)
    q96, k96, v96, W96 = make_inputs(17, 1, 1, 64, 96, 2, 2)
    mis = torch.empty(1, 1, 64 * 64 + 1, dtype=torch.bfloat16, device="cuda")[..., 1:].view(1, 1, 64, 64)
    beta = torch.tensor(1.0)
    bad = {
        "fp32 q": ((q.float(), k, v, W, beta), {}),
        "cpu k": ((q, k.cpu(), v, W, beta), {}),
        "non-contiguous v": ((q, k, v.transpose(2, 3).contiguous().transpose(2, 3), W, beta), {}),
        "misaligned q": ((mis, k, v, W, beta), {}),
        "head_dim 96": ((q96, k96, v96, W96, beta), {}),
        "bf16 W": ((q, k, v, W.to(torch.bfloat16), beta), {}),
        "P = 6": ((q, k, v, torch.randn(2, 6, 64, device="cuda"), beta), {}),
        "L = 5": ((q, k, v, torch.randn(5, 2, 64, device="cuda"), beta), {}),
        "shape mismatch": ((q, k[:, :, :32].contiguous(), v, W, beta), {}),
        "tile not a multiple of C": ((q, k, v, W, beta), {"tile_tokens": 48}),
        "negative tile": ((q, k, v, W, beta), {"tile_tokens": -64}),
    }
    for label, (args, kwargs) in bad.items():
        with pytest.raises(RuntimeError):
            race.causal_v2.forward(*args, **kwargs, tensor_cores=tc(variant))
            pytest.fail(f"accepted {label}")
