"""GPU parity of the causal op continued from a carried state (race_fwd_carry).

The reference hands the per-bucket sums off as final_state
(src/causal_v2/kernels/race_causal_fwd.h:20-21) and its chunked forward
carries A_state, B_state into the next chunk (src/race_chunked.py:54-63); the
reference's equivalence tests hold that chunked equals unchunked
(src/test_equivalence.py:47-65).  Here every case runs a prefix through
race_fused_fwd_with_state, continues from the returned state on the GPU (the
decode kernel, or the tile path with the scan seeded), and compares the
continued outputs and the final state with the fp64 oracle's unsplit run over
all the tokens.  Tolerances: max |out - ref| / max |ref| per stream, fp32
1e-4, bf16 outputs 2e-2; the fp32 state 1e-4 for either input dtype.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, per_stream_rel_err, say, to_np, tol_for

pytestmark = pytest.mark.gpu


def part(x, a, b):
    return x[:, a:b].contiguous()


def prefill(race, q, k, v, T0):
    """(out, state) of the first T0 tokens."""
    out, st = race.race_fused_fwd_with_state(part(q, 0, T0), part(k, 0, T0), part(v, 0, T0), True)
    return out, st


def has_mfma(ext, L, R, d):
    return ext.shape_supported(L, R, d)[1]


@pytest.mark.parametrize("kernel", ["auto", "decode", "valu", "mfma"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d", [(4, 16, 64), (1, 1, 1), (3, 5, 7), (2, 8, 32), (8, 32, 128),
                                     (4, 16, 128), (16, 16, 96)])
@pytest.mark.parametrize("T0, T1", [(0, 1), (300, 1), (300, 5), (1000, 16), (129, 17), (64, 300)])
def test_carry_matches_oracle(race, ext, oracle, cuda, kernel, dtype, L, R, d, T0, T1):
    if kernel == "mfma" and not has_mfma(ext, L, R, d):
        pytest.skip(f"no MFMA specialization for S={L * R}, d={d}")
    say("carry", kernel, dtype, L, R, d, "T0", T0, "T1", T1)
    N = 3
    q, k, v = race.make_inputs(N, T0 + T1, L, R, d, seed=T0 * 7 + T1 + d, dtype=dtype)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    _, st0 = prefill(race, qg, kg, vg, T0)
    out, st = race.race_fused_fwd_carry(part(qg, T0, T0 + T1), part(kg, T0, T0 + T1),
                                        part(vg, T0, T0 + T1), st0, kernel=kernel)
    torch.cuda.synchronize()
    ref, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True, nthreads=16)
    err = per_stream_rel_err(to_np(out), ref[:, T0:])
    serr = per_stream_rel_err(st.cpu().numpy(), fin)
    say("carry", kernel, dtype, L, R, d, "T0", T0, "T1", T1, f"out {err:.3e} state {serr:.3e}")
    assert out.dtype == dtype and out.shape == (N, T1, d)
    assert err <= tol_for(dtype)
    assert serr <= FP32_TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d", [(4, 16, 64), (8, 32, 128), (3, 5, 7)])
def test_decode_steps_in_place(race, oracle, cuda, dtype, L, R, d):
    # A prompt through the forward, then 24 one-token steps that advance the
    # same state tensor in place.
    say("decode in place", dtype, L, R, d)
    N, T0, steps = 4, 200, 24
    q, k, v = race.make_inputs(N, T0 + steps, L, R, d, seed=d + L, dtype=dtype)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    _, st = prefill(race, qg, kg, vg, T0)
    outs = []
    for t in range(T0, T0 + steps):
        o, st2 = race.race_fused_fwd_carry(part(qg, t, t + 1), part(kg, t, t + 1), part(vg, t, t + 1),
                                           st, inplace=True)
        assert st2.data_ptr() == st.data_ptr()
        outs.append(o)
    out = torch.cat(outs, dim=1)
    torch.cuda.synchronize()
    ref, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True, nthreads=16)
    err = per_stream_rel_err(to_np(out), ref[:, T0:])
    serr = per_stream_rel_err(st.cpu().numpy(), fin)
    say("decode in place", dtype, L, R, d, f"out {err:.3e} state {serr:.3e}")
    assert err <= tol_for(dtype)
    assert serr <= FP32_TOL


def test_cfg5_decode_step(race, oracle, cuda):
    # The LM-scale shape (N=128, S=256, d=128, bf16): a 64-token prompt, then
    # one decode step for every stream.
    say("cfg5 decode")
    N, T0 = 128, 64
    q, k, v = race.make_inputs(N, T0 + 1, 8, 32, 128, seed=5, dtype=torch.bfloat16)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    _, st = prefill(race, qg, kg, vg, T0)
    out, st = race.race_fused_fwd_carry(part(qg, T0, T0 + 1), part(kg, T0, T0 + 1),
                                        part(vg, T0, T0 + 1), st, inplace=True)
    torch.cuda.synchronize()
    ref, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True, nthreads=16)
    err = per_stream_rel_err(to_np(out), ref[:, T0:])
    serr = per_stream_rel_err(st.cpu().numpy(), fin)
    say("cfg5 decode", f"out {err:.3e} state {serr:.3e}")
    assert err <= tol_for(torch.bfloat16)
    assert serr <= FP32_TOL


@pytest.mark.parametrize("split", [1, 4096, 40000, 65535])
def test_cfg2_split_anywhere_equals_unsplit(race, cuda, split):
    # Size-independent property at cfg2's full length (N=8, T=65536, fp32):
    # the forward over [0, split) and the carry over [split, T) give the
    # unsplit outputs and final state.
    say("cfg2 split", split)
    T = 65536
    q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=split, device=cuda, gen_device="cuda")
    full, fin = race.race_fused_fwd_with_state(q, k, v, True)
    out0, st0 = prefill(race, q, k, v, split)
    out1, st1 = race.race_fused_fwd_carry(part(q, split, T), part(k, split, T), part(v, split, T), st0)
    torch.cuda.synchronize()
    got = torch.cat([out0, out1], dim=1)
    err = per_stream_rel_err(got.cpu().numpy(), full.cpu().numpy())
    serr = per_stream_rel_err(st1.cpu().numpy(), fin.cpu().numpy())
    say("cfg2 split", split, f"out {err:.3e} state {serr:.3e}")
    assert err <= FP32_TOL
    assert serr <= FP32_TOL


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_zero_carried_state_is_the_forward_bitwise(race, cuda, kernel):
    # Seeding the tile scan with zeros adds 0 to every running sum, which
    # changes no bit: the tile path then returns race_fused_fwd's result.
    q, k, v = race.make_inputs(5, 3000, 4, 16, 64, seed=3, device=cuda)
    want, fin = race.race_fused_fwd_with_state(q, k, v, True, kernel=kernel, tile_tokens=512)
    zero = torch.zeros_like(fin)
    got, st = race.race_fused_fwd_carry(q, k, v, zero, kernel=kernel, tile_tokens=512)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(st, fin)
    assert not zero.any()


def test_decode_is_deterministic_and_leaves_init_alone(race, cuda):
    q, k, v = race.make_inputs(6, 10, 4, 16, 64, seed=4, device=cuda)
    _, st = race.race_fused_fwd_with_state(q, k, v, True)
    keep = st.clone()
    a, sa = race.race_fused_fwd_carry(q, k, v, st)
    b, sb = race.race_fused_fwd_carry(q, k, v, st)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(sa, sb)
    assert torch.equal(st, keep)
    assert sa.data_ptr() != st.data_ptr()


def test_decode_and_tile_paths_agree(race, cuda):
    # The same 16 tokens through the decode kernel and the two tile paths.
    q, k, v = race.make_inputs(8, 2000, 4, 16, 64, seed=6, device=cuda)
    _, st = prefill(race, q, k, v, 1984)
    rest = [part(x, 1984, 2000) for x in (q, k, v)]
    runs = {kern: race.race_fused_fwd_carry(*rest, st, kernel=kern) for kern in ("decode", "valu", "mfma")}
    torch.cuda.synchronize()
    o_dec, s_dec = runs["decode"]
    for kern in ("valu", "mfma"):
        o, s = runs[kern]
        assert per_stream_rel_err(o.cpu().numpy(), o_dec.cpu().numpy()) <= FP32_TOL
        assert per_stream_rel_err(s.cpu().numpy(), s_dec.cpu().numpy()) <= FP32_TOL


def test_empty_carry_copies_the_state(race, cuda):
    q, k, v = race.make_inputs(3, 0, 4, 16, 64, device=cuda)
    st = torch.randn(3, 64 * 64 + 64, device=cuda)
    for kernel in ("auto", "decode", "valu"):
        out, st2 = race.race_fused_fwd_carry(q, k, v, st, kernel=kernel)
        torch.cuda.synchronize()
        assert out.shape == (3, 0, 64)
        assert torch.equal(st2, st) and st2.data_ptr() != st.data_ptr()


def test_carry_rejects_bad_states(race, cuda):
    q, k, v = race.make_inputs(2, 4, 4, 16, 64, device=cuda)
    with pytest.raises(RuntimeError, match="race_fused_fwd_carry: state has shape"):
        race.race_fused_fwd_carry(q, k, v, torch.zeros(2, 64 * 64, device=cuda))
    with pytest.raises(RuntimeError, match="race_fused_fwd_carry: state must be float32"):
        race.race_fused_fwd_carry(q, k, v, torch.zeros(2, 64 * 65, device=cuda, dtype=torch.float64))
    with pytest.raises(RuntimeError, match="race_fused_fwd_carry: state lives on the CPU"):
        race.race_fused_fwd_carry(q, k, v, torch.zeros(2, 64 * 65))


def test_c_abi_carry_direct_call(race, cuda):
    # race_fwd_carry through ctypes on raw device addresses, as a non-Python
    # host would call it, against the binding's result.
    from race_attention_kernel_amd import abi

    q, k, v = race.make_inputs(3, 9, 4, 16, 64, seed=8, device=cuda)
    init = torch.randn(3, 64 * 65, device=cuda).abs()
    want, want_st = race.race_fused_fwd_carry(q, k, v, init)
    sh = abi.shape(3, 9, 4, 16, 64, abi.RACE_F32)
    st, nbytes = abi.fwd_carry_workspace_bytes(sh, None)
    assert st == 0 and nbytes == 0
    out = torch.empty_like(v)
    state = init.clone()
    stream = torch.cuda.current_stream().cuda_stream
    st = abi.fwd_carry(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), state.data_ptr(),
                       state.data_ptr(), sh, None, None, 0, stream)
    assert st == 0, abi.status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    assert torch.equal(state, want_st)
