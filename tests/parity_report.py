#!/usr/bin/env python3
"""Achieved parity of the hot path at the full BASELINE configurations, as a
markdown table (written to stdout; profiles/parity.md holds a run).

Not a test (pytest does not collect it); the bounds live in the tests.  Run
on one MI355X from the repository root:

    python tests/parity_report.py > parity.md

Every figure is measured against the fp64 CPU oracle (oracle/) on the same
inputs (bf16 cases: the bf16-rounded values):
  - rel: max over streams of max|out - ref| / max|ref| (the north star's
    definition; fp32 bound 1e-4, bf16 2e-2);
  - F units (bf16 outputs): max|out - ref| / F and rms|out - ref| / F_rms,
    with F = max|bf16(ref) - ref| and F_rms the RMS of the same rounding
    errors: the error a perfect kernel with a bf16 output still makes
    (src/causal_v2/tests/causal_numerics.py:1-30 defines the model).
"""
from __future__ import annotations

import math
import pathlib
import sys
import time

import numpy as np
import torch

REPO = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "tests"))

import __graft_entry__ as entry  # noqa: E402
from gpu_util import per_stream_rel_err, rounding_floor, to_np  # noqa: E402


def f_units(out: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    """(max err / F, rms err / F_rms) over all elements."""
    F, F_rms = rounding_floor(ref)
    e = np.abs(out.astype(np.float64) - ref)
    return float(e.max()) / max(F, 1e-300), math.sqrt(float((e ** 2).mean())) / max(F_rms, 1e-300)


def main() -> int:
    race = entry.load_package()
    oracle = entry.load_oracle()
    oracle.build()
    dev = torch.device("cuda:0")
    rows = []

    def add(case, shape, streams, rel, fmax=None, frms=None):
        rows.append((case, shape, streams, rel, fmax, frms))
        print(f"# {case} {shape}: rel {rel:.2e}" + (f", {fmax:.3f} F, {frms:.3f} F_rms" if fmax else ""),
              file=sys.stderr, flush=True)

    t0 = time.time()
    # cfg2: every T x kernel family, all 8 streams, fp32.
    for kernel in ("valu", "mfma", "mfma_wg", "single"):
        for T in (512, 2048, 8192, 32768, 65536):
            q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=T)
            out = race.race_fused_fwd(q.to(dev), k.to(dev), v.to(dev), causal=True, kernel=kernel)
            torch.cuda.synchronize()
            ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), nthreads=16)
            add(f"cfg2 causal fwd fp32, {kernel}", f"N=8 T={T}", "8/8", per_stream_rel_err(to_np(out), ref))
    # cfg3: bf16, every stream.
    for T in (1 << 17, 1 << 18, 1 << 20):
        q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=T, dtype=torch.bfloat16, device=dev,
                                   gen_device="cuda")
        out = race.race_fused_fwd(q, k, v, causal=True)
        torch.cuda.synchronize()
        o = to_np(out)
        qn, kn, vn = to_np(q), to_np(k), to_np(v)
        del q, k, v, out
        torch.cuda.empty_cache()
        ref = oracle.causal_recurrence(qn, kn, vn, nthreads=16)
        fm, fr = f_units(o, ref)
        add("cfg3 causal fwd bf16", f"N=8 T={T}", "8/8", per_stream_rel_err(o, ref), fm, fr)
    # cfg3 shape through the one-read forward (kernel "single"), bf16.
    T = 1 << 18
    q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=T, dtype=torch.bfloat16, device=dev, gen_device="cuda")
    out = race.race_fused_fwd(q, k, v, causal=True, kernel="single")
    torch.cuda.synchronize()
    o = to_np(out)
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), nthreads=16)
    fm, fr = f_units(o, ref)
    add("cfg3 causal fwd bf16, single", f"N=8 T={T}", "8/8", per_stream_rel_err(o, ref), fm, fr)
    # The same inputs through the fp32-accurate bf16 forward (kernel "mfma_precise").
    out = race.race_fused_fwd(q, k, v, causal=True, kernel="mfma_precise")
    torch.cuda.synchronize()
    o = to_np(out)
    fm, fr = f_units(o, ref)
    add("cfg3 causal fwd bf16, mfma_precise", f"N=8 T={T}", "8/8", per_stream_rel_err(o, ref), fm, fr)
    del q, k, v, out
    torch.cuda.empty_cache()
    # cfg5: bf16, S = 256, d = 128; 16 of the 128 streams.  Then the
    # backward through autograd (forward walks over both value groups),
    # 4 streams against the oracle's VJP.
    q, k, v = race.make_inputs(128, 16384, 8, 32, 128, seed=5, dtype=torch.bfloat16, device=dev,
                               gen_device="cuda")
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = race.race_fused_fwd(qg, kg, vg, causal=True)
    torch.cuda.synchronize()
    pick = list(range(0, 128, 8))
    o = to_np(out[pick])
    ref = oracle.causal_recurrence(to_np(q[pick]), to_np(k[pick]), to_np(v[pick]), nthreads=16)
    fm, fr = f_units(o, ref)
    add("cfg5 causal fwd bf16", "N=128 T=16384 S=256 d=128", "16/128", per_stream_rel_err(o, ref), fm, fr)
    with torch.no_grad():
        o = to_np(race.race_fused_fwd(q, k, v, causal=True, kernel="mfma_precise")[pick])
    torch.cuda.synchronize()
    fm, fr = f_units(o, ref)
    add("cfg5 causal fwd bf16, mfma_precise", "N=128 T=16384 S=256 d=128", "16/128",
        per_stream_rel_err(o, ref), fm, fr)
    g = torch.randn(v.shape, device=dev, generator=torch.Generator(device=dev).manual_seed(6)).to(v.dtype)
    out.backward(g)
    torch.cuda.synchronize()
    pick = [0, 41, 86, 127]
    rq, rk, rv = oracle.causal_bwd(*(to_np(x[pick]) for x in (q, k, v, g)), nthreads=16)
    for name, got, want in (("dQ", qg.grad, rq), ("dK", kg.grad, rk), ("dV", vg.grad, rv)):
        gn = to_np(got[pick])
        fm, fr = f_units(gn, want)
        add(f"cfg5 causal bwd {name} bf16", "N=128 T=16384 S=256 d=128", "4/128",
            per_stream_rel_err(gn, want), fm, fr)
    del q, k, v, out, qg, kg, vg, g
    torch.cuda.empty_cache()
    # cfg4: non-causal forward and the three gradients, every stream.
    q, k, v, g = race.make_inputs(384, 1024, 4, 16, 64, seed=4, grad_out=True)
    qg, kg, vg = (x.to(dev).requires_grad_(True) for x in (q, k, v))
    out = race.race_fused_fwd(qg, kg, vg, causal=False)
    out.backward(g.to(dev))
    torch.cuda.synchronize()
    ref_out, _ = oracle.noncausal_fwd(to_np(q), to_np(k), to_np(v), nthreads=16)
    rq, rk, rv = oracle.noncausal_bwd(to_np(q), to_np(k), to_np(v), to_np(g), nthreads=16)
    for name, got, want in (("out", out.detach(), ref_out), ("dQ", qg.grad, rq), ("dK", kg.grad, rk),
                            ("dV", vg.grad, rv)):
        add(f"cfg4 non-causal {name} fp32", "N=384 T=1024", "384/384", per_stream_rel_err(to_np(got), want))
    # Causal backward at the cfg2 shape (T = 16384): through autograd.
    q, k, v, g = race.make_inputs(8, 16384, 4, 16, 64, seed=21, grad_out=True)
    qg, kg, vg = (x.to(dev).requires_grad_(True) for x in (q, k, v))
    race.race_fused_fwd(qg, kg, vg, causal=True).backward(g.to(dev))
    torch.cuda.synchronize()
    rq, rk, rv = oracle.causal_bwd(to_np(q), to_np(k), to_np(v), to_np(g), nthreads=16)
    for name, got, want in (("dQ", qg.grad, rq), ("dK", kg.grad, rk), ("dV", vg.grad, rv)):
        add(f"causal bwd {name} fp32", "N=8 T=16384", "8/8", per_stream_rel_err(to_np(got), want))
    # The module's hot span with the hashing inside (race_fused_fwd_hashed).
    for dtype, T in ((torch.float32, 65536), (torch.bfloat16, 1 << 18)):
        gen = torch.Generator(device=dev).manual_seed(9)
        kx, qx, vx = (torch.randn(8, T, 64, generator=gen, device=dev).to(dtype) for _ in range(3))
        planes = torch.randn(16, 64, generator=gen, device=dev)
        out = race.race_fused_fwd_hashed(kx, qx, vx, planes, 4)
        torch.cuda.synchronize()
        pt = planes.double().cpu().numpy().T
        pk = oracle.hash_probs(to_np(kx).astype(np.float64), pt, 4, 4).reshape(8, T, 64)
        pq = oracle.hash_probs(to_np(qx).astype(np.float64), pt, 4, 4).reshape(8, T, 64)
        ref = oracle.causal_recurrence(pq, pk, to_np(vx), nthreads=16)
        o = to_np(out)
        if dtype == torch.bfloat16:
            fm, fr = f_units(o, ref)
            add("hashed module bf16", f"N=8 T={T} L=4 K=4 d=64", "8/8", per_stream_rel_err(o, ref), fm, fr)
        else:
            add("hashed module fp32", f"N=8 T={T} L=4 K=4 d=64", "8/8", per_stream_rel_err(o, ref))
        del kx, qx, vx, out
        torch.cuda.empty_cache()

    print("| case | shape | streams checked | max rel err | max err / F | rms err / F_rms |")
    print("|---|---|---|---|---|---|")
    for case, shape, streams, rel, fm, fr in rows:
        fm_s = f"{fm:.3f}" if fm is not None else ""
        fr_s = f"{fr:.3f}" if fr is not None else ""
        print(f"| {case} | {shape} | {streams} | {rel:.2e} | {fm_s} | {fr_s} |")
    print(f"\n({time.time() - t0:.0f} s)", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
