"""GPU parity of the bucket-probability front end (src/race_baseline.py:41-44).

race_hash_probs against the fp64 oracle (oracle.hash_probs, pinned on the CPU
by the product-form identity and invariants in tests/test_oracle.py), over
head dims, table counts, corner counts, ragged row counts and both dtypes,
and the drop-in BatchedACE module end to end against the reference formula
(hashing + the causal recurrence, fp64).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, per_stream_rel_err, say, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dk, L, K", [(64, 4, 4), (8, 1, 1), (128, 8, 5), (16, 1, 8), (32, 3, 3)])
@pytest.mark.parametrize("rows", [1, 63, 65, 1000])
def test_hash_probs_match_oracle(race, oracle, cuda, dtype, dk, L, K, rows):
    say("hash", dtype, dk, L, K, rows)
    g = torch.Generator().manual_seed(dk * 131 + L * 7 + K + rows)
    x = torch.randn(rows, dk, generator=g).to(dtype)
    planes_T = torch.randn(dk, L * K, generator=g)
    got = race.race_hash_probs(x.to(cuda), planes_T.to(cuda), L, K)
    torch.cuda.synchronize()
    assert got.shape == (rows, L, 1 << K) and got.dtype == dtype
    want = oracle.hash_probs(x.float().numpy(), planes_T.numpy(), L, K)
    err = np.abs(got.float().cpu().numpy() - want).max()
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-6
    assert err <= tol, err
    if dtype == torch.float32:
        np.testing.assert_allclose(got.sum(-1).cpu().numpy(), 1.0, atol=1e-6)


def test_hash_probs_batched_shape(race, oracle, cuda):
    # Leading dimensions are kept: [N, T, d_k] -> [N, T, L, 2^K].
    x = torch.randn(3, 40, 64)
    planes_T = torch.randn(64, 16)
    got = race.race_hash_probs(x.to(cuda), planes_T.to(cuda), 4, 4)
    assert got.shape == (3, 40, 4, 16)
    want = oracle.hash_probs(x.numpy(), planes_T.numpy(), 4, 4)
    assert np.abs(got.cpu().numpy() - want).max() <= 1e-6


@pytest.mark.parametrize("dk, L, K", [(64, 4, 9), (64, 2, 8), (129, 4, 4), (64, 17, 4)])
def test_hash_probs_rejects_unsupported_shapes(race, cuda, dk, L, K):
    x = torch.randn(4, dk, device=cuda)
    planes_T = torch.randn(dk, L * K, device=cuda)
    with pytest.raises(RuntimeError, match="race_hash_probs"):
        race.race_hash_probs(x, planes_T, L, K)


def test_batched_ace_end_to_end(race, oracle, cuda):
    # The module's forward (permutes, hashing kernel, op) against the reference
    # formula of src/race_baseline.py:34-52 in fp64.
    say("batched-ace end to end")
    torch.manual_seed(77)
    ace = race.BatchedACE(64, 4, 4, 1).to(cuda)
    g = torch.Generator().manual_seed(5)
    K, V, Q = (torch.randn(1, 2, 500, 4, 64, generator=g) for _ in range(3))
    out = ace(K.to(cuda), V.to(cuda), Q.to(cuda))
    torch.cuda.synchronize()
    N = 8
    planes_T = ace.planes_T.cpu().numpy()
    k2 = K.permute(0, 1, 3, 2, 4).reshape(N, 500, 64).numpy()
    q2 = Q.permute(0, 1, 3, 2, 4).reshape(N, 500, 64).numpy()
    v2 = V.permute(0, 1, 3, 2, 4).reshape(N, 500, 64).numpy()
    pk = oracle.hash_probs(k2, planes_T, 4, 4).reshape(N, 500, 64)
    pq = oracle.hash_probs(q2, planes_T, 4, 4).reshape(N, 500, 64)
    ref = oracle.causal_recurrence(pq.astype(np.float32), pk.astype(np.float32), v2)
    got = out.permute(0, 1, 3, 2, 4).reshape(N, 500, 64)
    assert per_stream_rel_err(to_np(got), ref) <= FP32_TOL
