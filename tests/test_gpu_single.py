"""GPU parity of the one-read causal forward (kernel "single", single_pass.hip).

The same per-bucket causal function of src/race_baseline.py:45-51 as the
three-launch path, computed in one persistent launch (tiles of 128 tokens,
prefixes from four scanner workgroups per stream).  Checked against the fp64
oracle on full and ragged lengths, fp32 and bf16, one and two streams per XCD;
bitwise repeatable across runs (the scan adds tile totals in a fixed order);
the final state and a carried continuation against the oracle's unsplit run;
the kernel's error word (set when a bounded wait gives up) clear after every
call; and the conditions the path refuses.  Tolerances (north star): fp32 max
rel err 1e-4, bf16 inputs 2e-2, max |out - ref| / max |ref| per stream.
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import FP32_TOL, per_stream_rel_err, say, to_np, tol_for

pytestmark = pytest.mark.gpu

TILE = 128
CTL_ERROR = 8  # control word of the error flag (after the per-XCD counters)


def full_gpu():
    return torch.cuda.get_device_properties(0).multi_processor_count == 256


@pytest.fixture(autouse=True)
def _needs_full_gpu(cuda):
    if not full_gpu():
        pytest.skip("the one-read forward runs on a full MI355X (256 CUs)")


def run(race, q, k, v):
    out = race.race_fused_fwd(q, k, v, causal=True, kernel="single")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N, T", [(8, 1), (8, 31), (8, 127), (8, 128), (8, 129), (8, 1000),
                                  (16, 3000), (16, 777), (16, 2048), (8, 4096)])


def test_single_matches_oracle(race, oracle, cuda, dtype, N, T):
    say("single", dtype, "N", N, "T", T)
    q, k, v = race.make_inputs(N, T, 4, 16, 64, seed=N * 100003 + T, dtype=dtype)
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda))
    assert out.dtype == dtype and out.shape == v.shape
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), nthreads=16)
    err = per_stream_rel_err(to_np(out), ref)
    say("single", dtype, "N", N, "T", T, f"max rel err {err:.3e}")
    assert err <= tol_for(dtype)


def test_single_cfg2_full_size(race, ext, oracle, cuda):
    # cfg2: N=8, L=4, R=16, d=64, T=65536, fp32 (512 tiles per stream).  The
    # torch binding runs the one-read path: its records come in 128-token
    # tiles, the same output as the op.
    say("single cfg2")
    q, k, v = race.make_inputs(8, 65536, 4, 16, 64, seed=65536)
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda))
    dbg = ext.forward_debug(q.to(cuda), k.to(cuda), v.to(cuda), True, 0, race.ops.KERNELS["single"])
    torch.cuda.synchronize()
    assert dbg[-1] == TILE and torch.equal(dbg[0], out)
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), nthreads=16)
    err = per_stream_rel_err(to_np(out), ref)
    say("single cfg2", f"max rel err {err:.3e}")
    assert err <= FP32_TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_single_is_bitwise_repeatable(race, cuda, dtype):
    say("single repeat", dtype)
    q, k, v = race.make_inputs(16, 20000, 4, 16, 64, seed=7, dtype=dtype)
    q, k, v = q.to(cuda), k.to(cuda), v.to(cuda)
    first = run(race, q, k, v)
    for _ in range(3):
        assert torch.equal(run(race, q, k, v), first)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_single_state_and_carry(race, ext, oracle, cuda, dtype):
    # The final state of the one-read forward, and a continuation from a
    # carried state (the scanner starts from it), against the unsplit oracle.
    say("single carry", dtype)
    N, T0, T1 = 8, 1500, 2100
    q, k, v = race.make_inputs(N, T0 + T1, 4, 16, 64, seed=11, dtype=dtype)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    sl = lambda x, a, b: x[:, a:b].contiguous()
    out0, st0 = ext.forward(sl(qg, 0, T0), sl(kg, 0, T0), sl(vg, 0, T0), True, 0, 5, True)
    out1, st1 = race.race_fused_fwd_carry(sl(qg, T0, T0 + T1), sl(kg, T0, T0 + T1), sl(vg, T0, T0 + T1),
                                          st0, kernel="single")
    torch.cuda.synchronize()
    ref, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True, nthreads=16)
    _, fin0 = oracle.causal_recurrence(to_np(q)[:, :T0], to_np(k)[:, :T0], to_np(v)[:, :T0], want_state=True)
    errs = (per_stream_rel_err(to_np(out0), ref[:, :T0]), per_stream_rel_err(to_np(out1), ref[:, T0:]),
            per_stream_rel_err(st0.cpu().numpy(), fin0), per_stream_rel_err(st1.cpu().numpy(), fin))
    say("single carry", dtype, "errors", " ".join(f"{e:.3e}" for e in errs))
    assert errs[0] <= tol_for(dtype) and errs[1] <= tol_for(dtype)
    assert errs[2] <= FP32_TOL and errs[3] <= FP32_TOL


def test_single_through_the_c_abi_leaves_the_error_word_clear(race, oracle, cuda):
    # race_fwd with RACE_KERNEL_SINGLE on raw pointers and a caller-owned
    # workspace: the records, then one flag per (stream, tile), then the
    # control words; the error word stays zero and the records end as the
    # exclusive prefixes (the first tile's is zero, the last plus its own
    # totals is the final state).
    from race_attention_kernel_amd import abi

    N, T = 16, 5000
    q, k, v = race.make_inputs(N, T, 4, 16, 64, seed=3)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    out = torch.empty_like(vg)
    state = torch.empty(N, 64 * 64 + 64, device=cuda)
    sh = abi.shape(N, T, 4, 16, 64, abi.RACE_F32)
    opts = abi.options(0, abi.RACE_KERNEL_SINGLE)
    st, nbytes, tiles, rec = abi.fwd_workspace_bytes(sh, True, opts)
    assert st == 0 and tiles == (T + TILE - 1) // TILE
    flag_words = ((N * tiles + 63) // 64) * 64
    assert nbytes == (N * tiles * rec + flag_words + 64) * 4
    ws = torch.full((nbytes // 4,), -1, dtype=torch.int32, device=cuda)
    assert abi.fwd(qg.data_ptr(), kg.data_ptr(), vg.data_ptr(), out.data_ptr(), state.data_ptr(), sh, True,
                   opts, ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    words = ws[N * tiles * rec:].cpu()
    ctl = words[flag_words:]
    assert int(ctl[CTL_ERROR]) == 0
    assert (words[:N * tiles] == 5).all()  # totals flag + one per scanner part: every prefix whole
    recs = ws[:N * tiles * rec].view(torch.float32).view(N, tiles, rec)[:, :, :64 * 64 + 64].cpu()
    assert torch.count_nonzero(recs[:, 0]) == 0
    ref, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True, nthreads=16)
    assert per_stream_rel_err(to_np(out), ref) <= FP32_TOL
    assert per_stream_rel_err(state.cpu().numpy(), fin) <= FP32_TOL


def test_single_refuses_what_it_does_not_take(race, ext, cuda):
    from race_attention_kernel_amd import abi

    say("single refusals")
    bad = [abi.shape(4, 1000, 4, 16, 64),      # N not a multiple of 8
           abi.shape(24, 1000, 4, 16, 64),     # more than two streams per XCD
           abi.shape(8, 1000, 2, 16, 64),      # S = 32
           abi.shape(8, 1000, 4, 16, 128)]     # d = 128
    for sh in bad:
        st, _, _, _ = abi.fwd_workspace_bytes(sh, True, abi.options(0, abi.RACE_KERNEL_SINGLE))
        assert st == abi.RACE_ERROR_INVALID_VALUE
    sh = abi.shape(8, 1000, 4, 16, 64)
    assert abi.fwd_workspace_bytes(sh, True, abi.options(64, abi.RACE_KERNEL_SINGLE))[0] == abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd_workspace_bytes(sh, False, abi.options(0, abi.RACE_KERNEL_SINGLE))[0] == abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd_workspace_bytes(sh, True, abi.options(128, abi.RACE_KERNEL_SINGLE))[0] == 0


def test_single_through_autograd(race, oracle, cuda):
    # The one-read forward keeps its records (128-token tiles) for the
    # backward, which starts from them: the gradients against the oracle VJP,
    # dK relative to the scale of its cancelling terms as in the causal
    # backward suite.
    from test_gpu_causal_bwd import check_grads
    say("single autograd")
    q, k, v, g = race.make_inputs(8, 1000, 4, 16, 64, seed=12, grad_out=True)
    qg, kg, vg = (x.to(cuda).requires_grad_(True) for x in (q, k, v))
    out = race.race_fused_fwd(qg, kg, vg, causal=True, kernel="single")
    out.backward(g.to(cuda))
    torch.cuda.synchronize()
    check_grads(oracle, q, k, v, g, out.detach(), qg.grad, kg.grad, vg.grad, FP32_TOL)


def test_single_give_up_is_visible(race, oracle, cuda):
    # With the test hook on, the arming kernel presets the error word, so every
    # bounded wait gives up at its first poll and every workgroup exits
    # normally.  No tile's prefix arrives: every output row is NaN, the state
    # is NaN, and race_fwd_single_status reports the give-up; with the hook
    # off the next call on the same workspace is correct and reports success.
    import math

    from race_attention_kernel_amd import abi

    N, T = 8, 3000
    q, k, v = race.make_inputs(N, T, 4, 16, 64, seed=21)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    sh = abi.shape(N, T, 4, 16, 64, abi.RACE_F32)
    opts = abi.options(0, abi.RACE_KERNEL_SINGLE)
    st, nbytes, _, _ = abi.fwd_workspace_bytes(sh, True, opts)
    assert st == 0
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    out = torch.zeros_like(vg)
    state = torch.zeros(N, 64 * 64 + 64, device=cuda)

    def call():
        return abi.fwd(qg.data_ptr(), kg.data_ptr(), vg.data_ptr(), out.data_ptr(), state.data_ptr(), sh,
                       True, opts, ws.data_ptr(), nbytes, stream)

    say("single give-up preset", N, T)
    assert abi.single_pass_test_give_up(True) == 0
    try:
        assert call() == 0  # the launch itself succeeds
        got = abi.fwd_single_status(sh, opts, ws.data_ptr(), nbytes, stream)
    finally:
        abi.single_pass_test_give_up(False)
    assert got == abi.RACE_ERROR_SINGLE_PASS_GAVE_UP
    assert "gave up" in abi.status_string(got)
    assert torch.isnan(out).all()
    assert torch.isnan(state).all()

    say("single after the preset", N, T)
    assert call() == 0
    assert abi.fwd_single_status(sh, opts, ws.data_ptr(), nbytes, stream) == 0
    ref, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True, nthreads=16)
    assert per_stream_rel_err(out.cpu().numpy(), ref) <= FP32_TOL
    assert per_stream_rel_err(state.cpu().numpy(), fin) <= FP32_TOL
    assert not math.isnan(float(out.abs().max()))
    # The status call refuses arguments that do not name a one-read call.
    assert abi.fwd_single_status(sh, abi.options(0, 0), ws.data_ptr(), nbytes, stream) == \
        abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd_single_status(sh, opts, ws.data_ptr(), nbytes - 4, stream) == abi.RACE_ERROR_INVALID_VALUE
