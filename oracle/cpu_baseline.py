#!/usr/bin/env python3
"""One point of the CPU baseline, in a fresh process -- TEST INFRASTRUCTURE.

bench.py's cpu_baseline leg runs this script once per sequence length, so
that each point's peak resident set is its own (the method of the
reference's src/bench_cpu_memory.py:18-36: a new interpreter per T,
resource.getrusage at the end).  What is timed is the reference's CPU path,
the fp32 torch cumsum + bmm composition of src/race_baseline.py:45-51
(oracle.torch_reference_path), on inputs of the BASELINE distribution:
probsQ, probsK = softmax over R of N(0,1)*4 logits, V ~ N(0,1).

Timing: 1 warmup call, then the median of ``--reps`` calls
(time.perf_counter).  Prints one JSON line:
    {"N", "T", "S", "d", "threads", "ms", "ms_min_max", "m_tokens_per_s",
     "peak_rss_bytes", "input_bytes", "predicted_peak_bytes"}

Usage: python oracle/cpu_baseline.py --N 8 --T 4096 --L 4 --R 16 --d 64
                                     --threads 16 [--reps 3]
"""
from __future__ import annotations

import argparse
import json
import pathlib
import resource
import statistics
import sys
import time


def predicted_peak_bytes(N: int, T: int, S: int, d: int) -> int:
    """The composition's live fp32 tensors: about 2.2 N T S d (the k v
    products, their prefix sums and the quotient, with the allocator's
    overlap) plus the inputs and the output."""
    return int(2.2 * N * T * S * d * 4 + (2 * N * T * S + 2 * N * T * d) * 4)


def main() -> int:
    ap = argparse.ArgumentParser()
    for name in ("N", "T", "L", "R", "d", "threads"):
        ap.add_argument(f"--{name}", type=int, required=True)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--seed", type=int, default=1)
    a = ap.parse_args()

    import torch

    sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
    import oracle

    torch.set_num_threads(a.threads)
    S = a.L * a.R
    g = torch.Generator().manual_seed(a.seed)
    q = torch.softmax(torch.randn((a.N, a.T, a.L, a.R), generator=g) * 4.0, -1).reshape(a.N, a.T, S)
    k = torch.softmax(torch.randn((a.N, a.T, a.L, a.R), generator=g) * 4.0, -1).reshape(a.N, a.T, S)
    v = torch.randn((a.N, a.T, a.d), generator=g)
    times = []
    with torch.no_grad():
        oracle.torch_reference_path(q, k, v)  # warmup
        for _ in range(a.reps):
            t0 = time.perf_counter()
            oracle.torch_reference_path(q, k, v)
            times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    print(json.dumps({
        "N": a.N, "T": a.T, "S": S, "d": a.d, "threads": torch.get_num_threads(),
        "ms": round(med * 1e3, 3),
        "ms_min_max": [round(min(times) * 1e3, 3), round(max(times) * 1e3, 3)],
        "m_tokens_per_s": round(a.N * a.T / med / 1e6, 5),
        "peak_rss_bytes": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024,
        "input_bytes": (2 * a.N * a.T * S + a.N * a.T * a.d) * 4,
        "predicted_peak_bytes": predicted_peak_bytes(a.N, a.T, S, a.d),
    }), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
