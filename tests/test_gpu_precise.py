"""GPU parity of the precise bf16 path (kernel="mfma_precise",
RACE_KERNEL_MFMA_PRECISE): the workgroup matrix-core kernels with every
product fp32-accurate for bf16 tokens.  The default bf16 kernels round W =
q / (Abar + eps), the masked scores and the carried state to bf16 for their
products (the rounding points of the reference's bf16 tensor-core variant,
src/causal_v2/kernels/race_causal_fwd_tc.cu); with those carried as bf16
hi + lo pairs, a bf16 output differs from the fp64 oracle's by about its own
rounding (F = max|bf16(ref) - ref|), which is what is checked here, against
the same oracle on the same bf16 values as every other bf16 test."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import assert_bf16_floor, per_stream_rel_err, say, to_np

pytestmark = pytest.mark.gpu

# max <= k F + atol, rms <= k_rms F_rms + rms_atol: the precise path adds
# about 2^-17 relative per product to the output's own rounding.
PRECISE_FLOOR_FACTORS = (1.05, 1.05)


def run(race, q, k, v, kernel="mfma_precise", tile=0):
    out = race.race_fused_fwd(q, k, v, causal=True, tile_tokens=tile, kernel=kernel)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("L, R, d", [(4, 16, 64), (4, 16, 128), (8, 16, 64), (4, 32, 128), (8, 32, 64),
                                     (8, 32, 128)])
@pytest.mark.parametrize("T", [1, 63, 65, 700, 3000])
def test_shapes_against_the_oracle(race, oracle, cuda, L, R, d, T):
    # Every (S, d) specialization of the workgroup kernels, ragged lengths.
    say("precise shape", L, R, d, T)
    q, k, v = (x.to(cuda) for x in race.make_inputs(3, T, L, R, d, seed=T + d + 7, dtype=torch.bfloat16))
    out = run(race, q, k, v)
    assert out.dtype == torch.bfloat16
    o = to_np(out)
    vn = to_np(v)
    ref = oracle.causal_recurrence(to_np(q), to_np(k), vn, nthreads=16)
    assert per_stream_rel_err(o, ref) <= 2e-2
    assert_bf16_floor(o, ref, float(np.abs(vn).max()), f"precise S={L * R} d={d} T={T}",
                      factors=PRECISE_FLOOR_FACTORS)


def test_cfg3_length(race, oracle, cuda):
    # The cfg3 shape (N = 8, S = d = 64, bf16) at T = 2^17, all 8 streams.
    T = 1 << 17
    say("precise cfg3", T)
    q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=T, dtype=torch.bfloat16, device=cuda, gen_device="cuda")
    o = to_np(run(race, q, k, v))
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    ref = oracle.causal_recurrence(qn, kn, vn, nthreads=16)
    assert per_stream_rel_err(o, ref) <= 2e-2
    assert_bf16_floor(o, ref, float(np.abs(vn).max()), "precise cfg3", factors=PRECISE_FLOOR_FACTORS)
    # The default kernels on the same inputs stay within their own bound.
    od = to_np(run(race, q, k, v, kernel="auto"))
    assert_bf16_floor(od, ref, float(np.abs(vn).max()), "default cfg3")


def test_cfg5_shape(race, oracle, cuda):
    # cfg5 (N = 128, S = 256, d = 128, T = 16384, bf16): 16 streams.
    say("precise cfg5")
    q, k, v = race.make_inputs(128, 16384, 8, 32, 128, seed=5, dtype=torch.bfloat16, device=cuda,
                               gen_device="cuda")
    out = run(race, q, k, v)
    pick = list(range(0, 128, 8))
    o = to_np(out[pick])
    vn = to_np(v[pick])
    ref = oracle.causal_recurrence(to_np(q[pick]), to_np(k[pick]), vn, nthreads=16)
    assert per_stream_rel_err(o, ref) <= 2e-2
    assert_bf16_floor(o, ref, float(np.abs(vn).max()), "precise cfg5", factors=PRECISE_FLOOR_FACTORS)


def test_fp32_tokens_take_the_workgroup_kernels_unchanged(race, cuda):
    # For fp32 tokens every product is already split: the precise choice is
    # the workgroup kernel, bit for bit.
    q, k, v = (x.to(cuda) for x in race.make_inputs(2, 2000, 4, 16, 64, seed=9))
    assert torch.equal(run(race, q, k, v), run(race, q, k, v, kernel="mfma_wg"))


def test_bitwise_reproducible_and_causal(race, cuda):
    q, k, v = (x.to(cuda) for x in race.make_inputs(2, 3000, 8, 32, 128, seed=10, dtype=torch.bfloat16))
    a = run(race, q, k, v)
    assert torch.equal(a, run(race, q, k, v))
    v2 = v.clone()
    v2[:, 1500:] += 1
    b = run(race, q, k, v2)
    assert torch.equal(a[:, :1500], b[:, :1500])


def test_precise_is_refused_where_it_has_no_kernel(race, cuda):
    q, k, v = (x.to(cuda) for x in race.make_inputs(1, 64, 3, 5, 7, seed=11, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        run(race, q, k, v)  # S = 15, d = 7: no matrix-core kernel
    q, k, v = (x.to(cuda) for x in race.make_inputs(1, 64, 4, 16, 64, seed=11, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        race.race_fused_fwd(q, k, v, causal=False, kernel="mfma_precise")
