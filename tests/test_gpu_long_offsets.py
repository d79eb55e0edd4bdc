"""GPU parity at the longest sequences: the cfg2 shape in fp32 at T = 2^24
(137 GB of tensors) and a bf16 case whose tensors hold 2^32 elements, past
the 2^31 that a 32-bit element offset can reach.

Restates the reference's test_offsets_past_2_to_the_31
(src/causal_v2/tests/test_forward_cuda.py:306-318): the last stream's last
4096 outputs, where every offset is largest, are checked against the fp64
oracle (oracle.causal_tail: the state before them from blocked fp64 sums,
then the per-token scan, pinned against the full scan in
tests/test_oracle.py).  Inputs are generated on the GPU a stream at a time,
with the distribution of the BASELINE configurations.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, assert_bf16_floor, per_stream_rel_err, say, to_np

pytestmark = pytest.mark.gpu

TAIL = 4096


def fill_streams(N, T, L, R, d, dtype, seed, device, chunk=1 << 22):
    """probsQ, probsK [N, T, L, R] (softmax over R of N(0,1)*4 logits) and V
    [N, T, d] ~ N(0,1), generated in chunks of tokens (no full-size
    temporaries)."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.empty((N, T, L, R), dtype=dtype, device=device)
    k = torch.empty_like(q)
    v = torch.empty((N, T, d), dtype=dtype, device=device)
    for n in range(N):
        for c in range(0, T, chunk):
            e = min(T, c + chunk)
            for x in (q, k):
                x[n, c:e] = torch.softmax(torch.randn((e - c, L, R), generator=g, device=device) * 4.0, -1)
            v[n, c:e] = torch.randn((e - c, d), generator=g, device=device)
    return q, k, v


def tensor_bytes(N, T, S, d, es):
    return (2 * S + 2 * d) * N * T * es


def skip_unless_room(N, T, S, d, es):
    free, _ = torch.cuda.mem_get_info()
    need = tensor_bytes(N, T, S, d, es) * 1.1
    if free < need:
        pytest.skip(f"needs {need / 2**30:.0f} GiB of device memory, {free / 2**30:.0f} GiB free")


def last_stream_tail(race, oracle, q, k, v, out):
    """(GPU tail, fp64 oracle tail) of the last stream, [1, TAIL, d]."""
    n = q.shape[0] - 1
    got = to_np(out[n:n + 1, -TAIL:])
    qn, kn, vn = (to_np(x[n:n + 1]) for x in (q, k, v))
    ref = oracle.causal_tail(qn, kn, vn, TAIL, nthreads=16)
    return got, ref, float(np.abs(vn).max())


def test_cfg2_fp32_at_T_2_to_the_24(race, oracle, cuda):
    N, T, L, R, d = 8, 1 << 24, 4, 16, 64
    skip_unless_room(N, T, L * R, d, 4)
    say("cfg2 fp32 T=2^24")
    q, k, v = fill_streams(N, T, L, R, d, torch.float32, 24, cuda)
    out = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    got, ref, _ = last_stream_tail(race, oracle, q, k, v, out)
    del q, k, v, out
    torch.cuda.empty_cache()
    err = per_stream_rel_err(got, ref)
    say("cfg2 fp32 T=2^24 last-stream tail max rel err", f"{err:.3e}")
    assert err <= FP32_TOL


def test_bf16_offsets_past_2_to_the_31(race, oracle, cuda):
    # 8 streams x 2^23 tokens x 64 values: 2^32 elements in each of probsQ,
    # probsK, V and out.
    N, T, L, R, d = 8, 1 << 23, 4, 16, 64
    assert N * T * L * R > 2 ** 31 and N * T * d > 2 ** 31
    skip_unless_room(N, T, L * R, d, 2)
    say("bf16 N*T*d = 2^32")
    q, k, v = fill_streams(N, T, L, R, d, torch.bfloat16, 31, cuda)
    out = race.race_fused_fwd(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    got, ref, vmax = last_stream_tail(race, oracle, q, k, v, out)
    del q, k, v, out
    torch.cuda.empty_cache()
    err = per_stream_rel_err(got, ref)
    say("bf16 2^32 elements last-stream tail max rel err", f"{err:.3e}")
    assert err <= 2e-2
    assert_bf16_floor(got, ref, vmax, "bf16 2^32 elements tail")
