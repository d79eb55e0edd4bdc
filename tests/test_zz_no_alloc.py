"""race_fwd_noalloc: the forward for callers that cannot allocate (graph
capture, serving loops), whose workspace is the library's per-GPU scratch
array.  It runs race_fwd's kernels at race_fwd's tile length, so its outputs
and state equal race_fwd's bitwise.  Two calls in a row, the second smaller,
check that the array's leftover contents from one call never leak into the
next.  Collected last (the file name), so a failure here hides no other test."""
from __future__ import annotations

import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu


def _noalloc(abi, q, k, v, causal, tile, kernel, with_state):
    N, T = q.shape[0], q.shape[1]
    L, R = (q.shape[2], q.shape[3]) if q.dim() == 4 else (1, q.shape[2])
    d = v.shape[2]
    dt = abi.RACE_BF16 if q.dtype == torch.bfloat16 else abi.RACE_F32
    sh = abi.shape(N, T, L, R, d, dt)
    out = torch.full_like(v, float("nan"))
    state = torch.full((N, L * R * d + L * R), float("nan"), device=v.device) if with_state else None
    stream = torch.cuda.current_stream().cuda_stream
    st = abi.fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                         state.data_ptr() if with_state else None, sh, causal,
                         abi.options(tile, kernel), stream)
    assert st == 0, abi.status_string(st)
    return out, state


@pytest.mark.parametrize("causal", [True, False])
def test_noalloc_equals_race_fwd_on_two_calls_in_a_row(race, ext, cuda, causal):
    from race_attention_kernel_amd import abi

    cases = [  # (N, T, L, R, d, dtype, tile, kernel): the second is smaller
        (8, 65536, 4, 16, 64, torch.float32, 0, 0),   # cfg2 at full length, automatic tile
        (3, 1000, 4, 16, 64, torch.bfloat16, 128, 0),
    ]
    if not causal:
        cases = [(384, 1024, 4, 16, 64, torch.float32, 0, 0),  # cfg4
                 (5, 700, 2, 8, 32, torch.float32, 64, 0)]
    for i, (N, T, L, R, d, dtype, tile, kernel) in enumerate(cases):
        say("noalloc", "causal" if causal else "non-causal", "call", i, N, T, L, R, d, dtype, tile)
        q, k, v = race.make_inputs(N, T, L, R, d, seed=70 + i, dtype=dtype, device=cuda,
                                   gen_device="cuda")
        got, got_state = _noalloc(abi, q, k, v, causal, tile, kernel, True)
        want, want_state = ext.forward(q, k, v, causal, tile, kernel, True)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert torch.equal(got_state, want_state)
        # Without the optional state the output is the same.
        got2, _ = _noalloc(abi, q, k, v, causal, tile, kernel, False)
        torch.cuda.synchronize()
        assert torch.equal(got2, want)


def test_noalloc_one_read_forward_rearms_its_flags(race, ext, cuda):
    # RACE_KERNEL_SINGLE keeps ticket counters and tile flags in the scratch
    # array after its records; every call re-arms them (zeroes them ahead of
    # the main kernel).  Two calls in a row, the second smaller, on the array
    # the earlier tests left behind: both equal race_fwd bitwise and leave
    # the error word clear.
    from race_attention_kernel_amd import abi

    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the one-read forward runs on a full MI355X (256 CUs)")
    kernel = abi.RACE_KERNEL_SINGLE
    stream = torch.cuda.current_stream().cuda_stream
    for i, (N, T, dtype) in enumerate([(16, 4096, torch.float32), (8, 1500, torch.bfloat16)]):
        say("noalloc single call", i, N, T, dtype)
        q, k, v = race.make_inputs(N, T, 4, 16, 64, seed=90 + i, dtype=dtype, device=cuda,
                                   gen_device="cuda")
        got, got_state = _noalloc(abi, q, k, v, True, 0, kernel, True)
        sh = abi.shape(N, T, 4, 16, 64, abi.RACE_BF16 if dtype == torch.bfloat16 else abi.RACE_F32)
        assert abi.fwd_single_status(sh, abi.options(0, kernel), None, 0, stream) == 0
        want, want_state = ext.forward(q, k, v, True, 0, kernel, True)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert torch.equal(got_state, want_state)


def test_noalloc_refuses_calls_past_its_scratch(race, cuda):
    from race_attention_kernel_amd import abi

    # 2^20 fp32 tokens at 64-token tiles: 16384 tiles of 16.6 KB per stream,
    # far past 32 MiB.  Refused on the host, before any launch, so the
    # placeholder addresses are never read.
    sh = abi.shape(8, 1 << 20, 4, 16, 64, abi.RACE_F32)
    opts = abi.options(64, 0)
    st, need, _, _ = abi.fwd_workspace_bytes(sh, True, opts)
    assert st == 0 and need > abi.RACE_NOALLOC_SCRATCH_BYTES
    stream = torch.cuda.current_stream().cuda_stream
    assert abi.fwd_noalloc(16, 16, 16, 16, None, sh, True, opts, stream) == \
        abi.RACE_ERROR_SCRATCH_TOO_SMALL
    assert "scratch too small" in abi.status_string(abi.RACE_ERROR_SCRATCH_TOO_SMALL)
    # Shape errors are still reported as such.
    assert abi.fwd_noalloc(16, 16, 16, 16, None, abi.shape(8, 64, 4, 16, 300), True, None,
                           stream) == abi.RACE_ERROR_INVALID_VALUE
