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


# bf16 outputs against the rounding floor (the model of
# src/causal_v2/tests/causal_numerics.py:1-30): with F = max|bf16(ref) - ref|
# and F_rms the RMS of the same rounding errors -- what a kernel exact up to
# its bf16 output still makes -- max|o - ref| <= k F + atol and
# rms|o - ref| <= k_rms F_rms + rms_atol.  (2.5, 2.0) is the reference's pair
# for its bf16 tensor-core variant, whose intra-chunk scores and carried
# state are rounded to bf16 before they multiply V and W, as the bf16 MFMA
# kernels here (single hi*hi products) round theirs.
BF16_FLOOR_FACTORS = (2.5, 2.0)


def rounding_floor(ref: np.ndarray) -> tuple[float, float]:
    """(F, F_rms) of rounding the fp64 reference to bf16."""
    r = torch.from_numpy(np.asarray(ref, np.float64)).to(torch.bfloat16).double().numpy()
    e = np.abs(r - ref)
    return float(e.max()), float(np.sqrt((e ** 2).mean()))


def assert_bf16_floor(got, ref, vmax: float, label: str, factors=BF16_FLOOR_FACTORS) -> tuple[float, float]:
    """The k F bound on bf16 outputs; returns (max err / F, rms err / F_rms)."""
    k, k_rms = factors
    F, F_rms = rounding_floor(ref)
    err = np.abs(np.asarray(got, np.float64) - ref)
    emax, erms = float(err.max()), float(np.sqrt((err ** 2).mean()))
    atol, rms_atol = 1e-5 * vmax, 1e-7 * vmax
    say(label, f"{emax / max(F, 1e-300):.3f} F", f"{erms / max(F_rms, 1e-300):.3f} F_rms")
    assert emax <= k * F + atol, f"{label}: max {emax:.3e} > {k * F + atol:.3e} ({emax / max(F, 1e-300):.3f} F)"
    assert erms <= k_rms * F_rms + rms_atol, (
        f"{label}: rms {erms:.3e} > {k_rms * F_rms + rms_atol:.3e} ({erms / max(F_rms, 1e-300):.3f} F_rms)")
    return emax / max(F, 1e-300), erms / max(F_rms, 1e-300)


def say(*parts) -> None:
    print("[case]", *parts, flush=True)
