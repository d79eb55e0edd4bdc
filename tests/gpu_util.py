"""Helpers shared by the GPU parity tests (no test functions here)."""
from __future__ import annotations

import numpy as np
import torch

# max |out - ref| / max |ref|, per stream, worst stream.
FP32_TOL = 1e-4
BF16_TOL = 2e-2


def tol_for(dtype: torch.dtype) -> float:
    return BF16_TOL if dtype == torch.bfloat16 else FP32_TOL


def per_stream_rel_err(got, ref) -> float:
    """max over streams of max|got - ref| / max|ref| (streams with ref == 0 use 1)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    N = ref.shape[0]
    num = np.abs(got - ref).reshape(N, -1).max(1)
    den = np.abs(ref).reshape(N, -1).max(1)
    den = np.where(den > 0, den, 1.0)
    return float((num / den).max())


def to_np(t: torch.Tensor) -> np.ndarray:
    """GPU/CPU tensor -> float32 numpy, [N, T, L, R] flattened to [N, T, S]."""
    t = t.detach().float().cpu()
    if t.dim() == 4:
        t = t.flatten(2)
    return t.contiguous().numpy()


def say(*parts) -> None:
    print("[case]", *parts, flush=True)
