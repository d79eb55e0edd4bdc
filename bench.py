#!/usr/bin/env python3
"""Benchmark of race_fused_fwd on one MI355X; prints ONE JSON line.

Default workload (cfg2, the configuration the headline metric is quoted on):
causal forward, N = 8 streams, L = 4, R = 16 (S = 64), d = 64, T = 65536,
fp32, synthetic inputs (softmax probabilities of N(0,1)*4 logits, N(0,1)
values) generated on the GPU and resident in HBM before the timed region.  A "step" is one
race_fused_fwd pass over that batch: every kernel of the op, through the C
ABI (include/race_mi355x.h), with caller-owned output and workspace.

Timing: W untimed warmup steps, then two timed regions, each of K steps
bracketed by torch.cuda.synchronize() on both sides.  The first runs plain
race_fwd steps back to back on the stream between two HIP events: `value` =
N*T / (mean step time) in M tokens/s.  The second runs race_fwd_profiled,
which records a HIP event on the launch stream before the first kernel and
after every kernel; the per-kernel durations behind `roofline` come from it
(its step time, with the extra events, is `profiled_ms_per_step`).

roofline: the dominant kernel's algorithmic HBM bytes per launch (each
operand it streams read once, its output written once: bytes per
stream-token * N * T; workspace records excluded) / its mean duration,
against MI355X's 8 TB/s.  traffic: HBM bytes per launch measured with
rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (scaled by the same counters on a
plain copy of known size, --calibrate-copy), read from profiles/traffic.json
when a measurement for this workload exists, else null.

cpu_baseline: the reference's CPU path -- the fp32 torch cumsum + bmm
composition of src/race_baseline.py:45-51, as restated in oracle/ -- timed on
this host's cores on the bench workload itself (cfg2: N = 8, T = 65536; a
shorter T when the host has too little free memory for its 5-D tensors):
1 warmup, median of 3.

Other workloads and passes (--workload, --pass bwd|fwdbwd) print the same
line for that configuration; the CPU baseline belongs to the headline
(cfg2 forward) only.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2|cfg3|cfg4|cfg5]
                       [--pass fwd|bwd|fwdbwd|module] [--T T] [--kernel auto|valu|mfma|mfma_wg]
                       [--tile N] [--no-cpu-baseline] [--calibrate-copy MIB]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import statistics
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

import __graft_entry__ as entry  # noqa: E402

METRIC = "causal fwd M tokens/s at N=8,S=64,d_k=64,T=64K on 1 GPU; max T that fits"
UNIT = "M tokens/s"
PEAK_HBM_GBPS = 8000.0
# The reference's published number for this shape: its PyTorch cumsum + bmm
# path at T = 65536 on an A100-SXM4-40GB (README.md:65-77 of the reference).
REFERENCE_MTOKS_T65536 = 5.25

WORKLOADS = {
    # name: (config key, default T)
    "cfg2": ("cfg2_causal_fp32", 65536),
    "cfg3": ("cfg3_causal_bf16", 1 << 20),
    "cfg4": ("cfg4_noncausal_fp32", 1024),
    "cfg5": ("cfg5_causal_bf16_S256", 16384),
}

# Kernel names of each launch sequence, by (causal, kernel family).
PHASES = {
    (True, "valu"): ["tile_sums", "tile_scan", "output_pass_valu"],
    (False, "valu"): ["tile_sums", "tile_reduce", "token_map"],
    (True, "mfma"): ["tile_sums_mfma", "tile_scan", "output_pass_mfma"],
    (True, "hashed"): ["hashed_sums", "tile_scan", "hashed_output"],
}
# Non-causal forwards with at most this many tiles per stream add the tile
# records inside the map (no tile_reduce launch), as race_api.hip does.
NONCAUSAL_FOLD_TILES = 4
# Backward launch sequences (every gradient requested).
BWD_PHASES = {
    True: ["bwd_tile_sums", "tile_scan", "bwd_dq", "suffix_scan", "bwd_dkv"],
    False: ["token_map_dq", "tile_sums_dE", "bwd_finalize", "token_map_dk", "token_map_dv"],
}


class HipEvents:
    """hipEvent_t handles from the HIP runtime torch already loaded."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.created = []

    def record(self, h, stream) -> None:
        if self.lib.hipEventRecord(h, stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def array(self, n):
        arr = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            if self.lib.hipEventCreate(ctypes.byref(h)) != 0:
                raise RuntimeError("hipEventCreate failed")
            arr[i] = h
            self.created.append(h)
        return arr

    def elapsed_ms(self, a, b) -> float:
        ms = ctypes.c_float()
        if self.lib.hipEventSynchronize(b) != 0:
            raise RuntimeError("hipEventSynchronize failed")
        if self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self):
        for h in self.created:
            self.lib.hipEventDestroy(h)
        self.created = []


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="cfg2")
    ap.add_argument("--pass", dest="pass_",
                    choices=["fwd", "bwd", "fwdbwd", "module", "module_twostep", "alg1", "decode"],
                    default="fwd",
                    help="what one step runs: the forward (default), the backward (from the "
                         "forward's inputs and a synthetic dOut), both, the module's hot "
                         "span (hashing of Q and K rows, then the forward), the "
                         "Algorithm-1 forward with the hashing inside (race_alg1_fwd), or "
                         "one decode step (race_fwd_carry of --T tokens per stream, default 1, "
                         "advancing the carried state in place) at the workload's N, S, d")
    ap.add_argument("--alg1-variant", choices=["fp32", "bf16"], default="bf16",
                    help="rounding variant of --pass alg1 (fp32-accurate or bf16 features)")
    ap.add_argument("--T", type=int, default=0)
    ap.add_argument("--kernel", choices=["auto", "valu", "mfma", "mfma_wg", "decode"], default="auto")
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB before timing (rocprofv3 counter scale)")
    return ap.parse_args()


def phase_bytes(name: str, cfg, T: int, es: int, tiles: int, rec: int) -> float:
    """Algorithmic HBM bytes of one launch of kernel `name` (each operand once)."""
    NT = cfg.N * T
    S, d = cfg.S, cfg.d
    state = 4.0 * cfg.N * tiles * rec
    small = 4.0 * cfg.N * (S * d + S) * 3
    return {
        "tile_sums": es * (S + d) * NT,
        "tile_sums_mfma": es * (S + d) * NT,
        "tile_scan": 2 * state,
        "tile_reduce": state,
        "output_pass_valu": es * (2 * S + 2 * d) * NT,
        "output_pass_mfma": es * (2 * S + 2 * d) * NT,
        "token_map": es * (S + d) * NT,
        # backward: each launch's own operands (reads) and outputs (writes)
        "bwd_tile_sums": es * (S + d) * NT,
        "bwd_dq": es * (3 * S + 2 * d) * NT,       # q, k, v, dOut -> dQ
        "suffix_scan": 2 * state,
        "bwd_dkv": es * (3 * S + 3 * d) * NT,      # q, k, v, dOut -> dK, dV
        "token_map_dq": es * (d + S) * NT,
        "tile_sums_dE": es * (S + d) * NT,
        "bwd_finalize": state + small,             # dE tile records, state -> dB, dA
        "token_map_dk": es * (d + S) * NT,
        "token_map_dv": es * (S + d) * NT,
        "hash_q": es * (d + S) * NT,               # rows of d_k = d -> probabilities
        "hash_k": es * (d + S) * NT,
        "hashed_sums": es * 2 * d * NT,            # K rows, V (hashing inside)
        "hashed_output": es * 4 * d * NT,          # Q, K, V rows -> out
    }.get(name, es * (2 * S + 2 * d) * NT)


def op_bytes(pass_: str, cfg, T: int, es: int) -> float:
    """Algorithmic bytes of one step: the forward reads Q, K, V and writes out;
    the backward reads Q, K, V, dOut and writes dQ, dK, dV.  The module's
    hot span (hashing + forward, src/race_baseline.py:41-51) reads the Q, K
    and V rows and writes out: 4 d values per stream-token, whichever path
    runs it (the two-step path's probability round trip is its own cost)."""
    S, d, NT = cfg.S, cfg.d, cfg.N * T
    fwd, bwd = es * (2 * S + 2 * d) * NT, es * (4 * S + 3 * d) * NT
    module = es * 4 * d * NT
    return {"fwd": fwd, "bwd": bwd, "fwdbwd": fwd + bwd, "module": module,
            "module_twostep": module}[pass_]


def traffic_for(workload_key: str, kernel_name: str):
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        table = json.loads(path.read_text())
    except ValueError:
        return None
    entry_ = table.get(f"{workload_key}:{kernel_name}")
    return None if entry_ is None else entry_.get("hbm_bytes_per_launch")


def cpu_baseline():
    """The reference CPU path (torch fp32 cumsum + bmm) on the cfg2 workload.

    Its 5-D prefix tensors need about 2.2 * N * T * S * d * 4 bytes
    (src/race_baseline.py:46-47); T is halved until that fits in a third of
    the host's available memory."""
    import torch

    race = entry.load_package()
    oracle = entry.load_oracle()
    N, T, L, R, d = 8, 65536, 4, 16, 64
    try:
        import psutil

        avail = psutil.virtual_memory().available
    except ImportError:
        avail = 64 << 30
    while T > 1024 and 3 * 2.2 * N * T * L * R * d * 4 > avail:
        T //= 2
    q, k, v = race.make_inputs(N, T, L, R, d, seed=1)
    q, k = q.flatten(2), k.flatten(2)
    threads = torch.get_num_threads()
    with torch.no_grad():
        oracle.torch_reference_path(q, k, v)  # warmup
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.torch_reference_path(q, k, v)
            times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(N * T / med / 1e6, 4),
        "unit": UNIT,
        "cores": threads,
        "kind": "port",
        "sample": (f"causal N={N} T={T} L={L} R={R} d={d} fp32 (the cfg2 workload"
                   f"{'' if T == 65536 else ', T reduced to fit host memory'}), the torch-CPU "
                   f"cumsum+bmm composition of src/race_baseline.py:45-51 (oracle/oracle.py "
                   f"torch_reference_path), {threads} threads, median of 3 after 1 warmup: "
                   f"{med * 1e3:.1f} ms per call"),
    }


# The reference's own benchmark of its causal v2 forward
# (src/causal_v2/bench/bench_causal.py:37-39): B*H = 8 streams, d = 64,
# P = 4, L = 4, beta = 1/sqrt(d); its "2M-token" job is T = 2^21.
ALG1_JOB = {"BH": 8, "T": 1 << 21, "D": 64, "P": 4, "L": 4}
# Its published times for that job on an H100 80GB (benchmarks/h100_run.md:63-69);
# context only, a different GPU.
ALG1_REFERENCE_H100_MS = {"bf16": 14.7, "fp32": 55.0}


def bench_alg1(args) -> int:
    """--pass alg1: race_alg1_fwd on the reference's causal v2 job."""
    import torch

    race = entry.load_package()
    from race_attention_kernel_amd import abi

    BH, D, P, L = ALG1_JOB["BH"], ALG1_JOB["D"], ALG1_JOB["P"], ALG1_JOB["L"]
    T = args.T or ALG1_JOB["T"]
    S = L << P
    variant = abi.RACE_ALG1_BF16 if args.alg1_variant == "bf16" else abi.RACE_ALG1_FP32
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(BH, T, D, device=dev, generator=gen).to(torch.bfloat16) for _ in range(3))
    W = torch.randn(L, P, D, device=dev, generator=gen)
    beta = torch.tensor([1.0 / D ** 0.5], device=dev)
    out = torch.empty_like(v)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    sh = abi.alg1_shape(BH, T, D, P, L)
    st, ws_bytes, tiles, rec = abi.alg1_workspace_bytes(sh, variant, args.tile)
    if st != 0:
        raise RuntimeError(abi.status_string(st))
    tile = race.causal_v2.select_tile_tokens(BH, T, D, P, L, variant == abi.RACE_ALG1_BF16) \
        if args.tile == 0 else args.tile
    ws = torch.empty(max(ws_bytes // 4, 1), device=dev, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), W.data_ptr(), beta.data_ptr(), out.data_ptr())

    def check(st_):
        if st_ != 0:
            raise RuntimeError(abi.status_string(st_))

    def plain():
        check(abi.alg1_fwd(*ptrs, None, sh, args.tile, variant, ws.data_ptr(), ws_bytes, stream))

    if args.calibrate_copy:
        src = torch.ones(args.calibrate_copy << 18, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    events = HipEvents()
    per_step = [events.array(8) for _ in range(args.steps)]
    warm = events.array(8)
    for _ in range(args.warmup):
        plain()
        check(abi.alg1_fwd_profiled(*ptrs, None, sh, args.tile, variant, ws.data_ptr(), ws_bytes,
                                    stream, warm)[0])
    torch.cuda.synchronize()
    bracket = events.array(2)
    t0 = time.perf_counter()
    events.record(bracket[0], stream)
    for _ in range(args.steps):
        plain()
    events.record(bracket[1], stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = events.elapsed_ms(bracket[0], bracket[1]) / args.steps
    n = 0
    for i in range(args.steps):
        st_, n = abi.alg1_fwd_profiled(*ptrs, None, sh, args.tile, variant, ws.data_ptr(), ws_bytes,
                                       stream, per_step[i])
        check(st_)
    torch.cuda.synchronize()
    names = ["alg1_sums", "tile_scan", "alg1_output"]
    gaps = [statistics.fmean(events.elapsed_ms(ev[j], ev[j + 1]) for ev in per_step) for j in range(n - 1)]
    if len(gaps) != len(names):
        names = [f"kernel{j}" for j in range(len(gaps))]
    NT = BH * T
    state = 4.0 * BH * tiles * rec
    kbytes = {"alg1_sums": 2 * 2 * D * NT, "tile_scan": 2 * state, "alg1_output": 4 * 2 * D * NT}
    dom = max(range(len(gaps)), key=lambda j: gaps[j])
    dom_bytes = kbytes.get(names[dom], 0.0)
    achieved = dom_bytes / (gaps[dom] * 1e-3) / 1e9
    peak_bytes = torch.cuda.max_memory_allocated(dev)
    events.destroy()
    value = NT / (ms_per_step * 1e-3) / 1e6
    # Whole-op algorithmic bytes: read q, k, v once and write out once (8 d
    # bytes per stream-token, the reference's "minimum" model,
    # bench_causal.py:11-17).
    op_min = 8 * D * NT
    result = {
        "metric": f"causal Algorithm-1 fwd (hashing inside) M tokens/s at BH={BH},d={D},P={P},L={L},T={T} on 1 GPU",
        "value": round(value, 3),
        "unit": UNIT,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"alg1: causal Algorithm 1 with hashing, BH={BH} T={T} d={D} P={P} L={L} "
                        f"beta=1/sqrt(d) bf16, {args.alg1_variant} variant",
            "BH": BH, "T": T, "D": D, "P": P, "L": L, "S": S, "variant": args.alg1_variant,
            "tile_tokens": tile, "launches_per_step": len(gaps),
            "kernel_ms": {names[j]: round(gaps[j], 5) for j in range(len(gaps))},
            "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
            "peak_hbm_bytes_per_token": round(peak_bytes / T, 1),
            "alg_bytes_per_stream_token": 8 * D,
            "whole_op_frac": round(op_min / (ms_per_step * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "reference_h100_ms_same_job": ALG1_REFERENCE_H100_MS[args.alg1_variant] if T == 1 << 21 else None,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": names[dom],
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": traffic_for(f"alg1_{args.alg1_variant}", names[dom]),
        },
        "cpu_baseline": None,
    }
    print(json.dumps(result))
    return 0


def bench_decode(args) -> int:
    """--pass decode: race_fwd_carry steps on a state carried in place."""
    import torch

    race = entry.load_package()
    from race_attention_kernel_amd import abi

    cfg = race.CONFIGS[WORKLOADS[args.workload][0]]
    T = args.T or 1
    N, S, d = cfg.N, cfg.L * cfg.R, cfg.d
    es = 2 if cfg.dtype == torch.bfloat16 else 4
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v = race.config_inputs(cfg, T, seed=0, device=dev, gen_device="cuda")
    # The state of a 4096-token prompt of the same distribution.
    pq, pk, pv = race.config_inputs(cfg, 4096, seed=1, device=dev, gen_device="cuda")
    _, state = race.race_fused_fwd_with_state(pq, pk, pv, True)
    del pq, pk, pv
    out = torch.empty_like(v)
    sh = abi.shape(N, T, cfg.L, cfg.R, d, abi.RACE_BF16 if es == 2 else abi.RACE_F32)
    kernel_id = race.ops.KERNELS["decode" if args.kernel == "auto" else args.kernel]
    opts = abi.options(args.tile, kernel_id)
    st, ws_bytes = abi.fwd_carry_workspace_bytes(sh, opts)
    if st != 0:
        raise RuntimeError(abi.status_string(st))
    ws = torch.empty(max(ws_bytes // 4, 1), device=dev, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), state.data_ptr(), state.data_ptr())
    if args.calibrate_copy:
        src = torch.ones(args.calibrate_copy << 18, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        del src, dst
    torch.cuda.synchronize()

    def check(st_):
        if st_ != 0:
            raise RuntimeError(abi.status_string(st_))

    def plain():
        check(abi.fwd_carry(*ptrs, sh, opts, ws.data_ptr(), ws_bytes, stream))

    events = HipEvents()
    per_step = [events.array(8) for _ in range(args.steps)]
    for _ in range(args.warmup):
        plain()
    torch.cuda.synchronize()
    bracket = events.array(2)
    t0 = time.perf_counter()
    events.record(bracket[0], stream)
    for _ in range(args.steps):
        plain()
    events.record(bracket[1], stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = events.elapsed_ms(bracket[0], bracket[1]) / args.steps
    n = 0
    for i in range(args.steps):
        st_, n = abi.fwd_carry_profiled(*ptrs, sh, opts, ws.data_ptr(), ws_bytes, stream, per_step[i])
        check(st_)
    torch.cuda.synchronize()
    gaps = [statistics.fmean(events.elapsed_ms(ev[j], ev[j + 1]) for ev in per_step) for j in range(n - 1)]
    names = ["decode"] if len(gaps) == 1 else [f"kernel{j}" for j in range(len(gaps))]
    events.destroy()
    # One launch reads and writes the state (B [S][d] and A [S], fp32) once
    # and reads the tokens' q, k, v rows and writes their outputs once.
    state_bytes = 4.0 * N * (S * d + S)
    launch_bytes = 2 * state_bytes + es * N * T * (2 * S + 2 * d)
    dom = max(range(len(gaps)), key=lambda j: gaps[j])
    achieved = launch_bytes / (gaps[dom] * 1e-3) / 1e9 if len(gaps) == 1 else None
    value = N * T / (ms_per_step * 1e-3) / 1e6
    result = {
        "metric": f"causal decode step M tokens/s at N={N},S={S},d={d},{T} token(s) per stream on 1 GPU",
        "value": round(value, 3),
        "unit": UNIT,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if es == 2 else "fp32",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload} decode: race_fwd_carry of {T} token(s) per stream, N={N} "
                        f"S={S} d={d}, state carried in place from a 4096-token prompt",
            "N": N, "S": S, "d": d, "T": T, "kernel": args.kernel if args.kernel != "auto" else "decode",
            "launches_per_step": len(gaps),
            "kernel_ms": {names[j]: round(gaps[j], 6) for j in range(len(gaps))},
            "wall_ms_per_step": round(wall * 1e3 / args.steps, 6),
            "state_bytes": state_bytes,
            "alg_bytes_per_launch": launch_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": names[dom],
            "achieved": round(achieved, 1) if achieved is not None else None,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4) if achieved is not None else None,
            "traffic": traffic_for(f"decode_{args.workload}_T{T}", names[dom]),
        },
        "cpu_baseline": None,
    }
    print(json.dumps(result))
    return 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the "
              "multi-GPU sharding of the op is designed but not measured here.",
              file=sys.stderr)
        return 2
    if args.pass_ == "alg1":
        return bench_alg1(args)
    if args.pass_ == "decode":
        return bench_decode(args)
    import torch

    race = entry.load_package()
    from race_attention_kernel_amd import abi

    cfg_key, default_T = WORKLOADS[args.workload]
    cfg = race.CONFIGS[cfg_key]
    T = args.T or default_T
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    es = 2 if cfg.dtype == torch.bfloat16 else 4
    q, k, v = race.config_inputs(cfg, T, seed=0, device=dev, gen_device="cuda")
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    sh = abi.shape(cfg.N, T, cfg.L, cfg.R, cfg.d, abi.RACE_BF16 if es == 2 else abi.RACE_F32)
    kernel_id = race.ops.KERNELS[args.kernel]
    opts = abi.options(args.tile, kernel_id)
    st, ws_bytes, tiles, rec = abi.fwd_workspace_bytes(sh, cfg.causal, opts)
    if st != 0:
        raise RuntimeError(abi.status_string(st))
    tile = race.select_tile_tokens(cfg.N, T, cfg.L, cfg.R, cfg.d, bf16=(es == 2), causal=cfg.causal,
                                   tile_tokens=args.tile, kernel=kernel_id)
    family = "valu"
    if cfg.causal and (kernel_id in (2, 3) or (kernel_id == 0 and race.ops._lib.ext().shape_supported(
            cfg.L, cfg.R, cfg.d)[1])):
        family = "mfma"
    ws = torch.empty(max(ws_bytes // 4, 1), device=dev, dtype=torch.float32)
    out = torch.empty_like(v)
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr())

    def check(st_):
        if st_ != 0:
            raise RuntimeError(abi.status_string(st_))

    # One step of the chosen pass: plain(), and profiled(events) -> events used.
    run_hashed = args.pass_ == "module"
    run_hash = args.pass_ == "module_twostep"
    if run_hash or run_hashed:
        # The module's inputs: Q and K rows [N, T, d_k] and the shared planes;
        # the hashing writes the probabilities the forward then reads.
        if not cfg.causal or cfg.R & (cfg.R - 1):
            raise SystemExit("--pass module needs a causal workload with R a power of two")
        Kp = cfg.R.bit_length() - 1
        gen = torch.Generator(device=dev).manual_seed(11)
        xq = torch.randn(cfg.N, T, cfg.d, device=dev, generator=gen).to(v.dtype)
        xk = torch.randn(cfg.N, T, cfg.d, device=dev, generator=gen).to(v.dtype)
        planes_T = torch.randn(cfg.d, cfg.L * Kp, device=dev, generator=gen)
        planes = planes_T.t().contiguous()  # [L*K, d], the hashed op's layout
        hdt = abi.RACE_BF16 if es == 2 else abi.RACE_F32
        hopts = abi.options(args.tile, 0)
        st, hws_bytes, tiles, rec = abi.hashed_fwd_workspace_bytes(sh, Kp, hopts)
        check(st)
        if run_hashed:
            ws = torch.empty(max(hws_bytes // 4, 1), device=dev, dtype=torch.float32)
            ws_bytes = hws_bytes
            tile = race.select_tile_tokens(cfg.N, T, cfg.L, cfg.R, cfg.d, bf16=(es == 2), causal=True,
                                           tile_tokens=args.tile, kernel="mfma_wg")
            family = "hashed"
            hptrs = (xk.data_ptr(), xq.data_ptr(), v.data_ptr(), planes.data_ptr(), out.data_ptr())

        def hash_both():
            for x_, p_ in ((xq, q), (xk, k)):
                check(abi.hash_probs(x_.data_ptr(), planes_T.data_ptr(), p_.data_ptr(), cfg.N * T,
                                     cfg.d, cfg.L, Kp, hdt, stream))
    run_fwd = args.pass_ in ("fwd", "fwdbwd", "module_twostep")
    run_bwd = args.pass_ in ("bwd", "fwdbwd")
    state = None
    if run_bwd:
        g = torch.randn(v.shape, device=dev, dtype=torch.float32,
                        generator=torch.Generator(device=dev).manual_seed(7)).to(v.dtype)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        bptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr())
        gptrs = (dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
        bopts = abi.options(0, 0)
        if cfg.causal:
            st, bws_bytes = abi.causal_bwd_workspace_bytes(sh, bopts)
        else:
            st, bws_bytes = abi.noncausal_bwd_workspace_bytes(sh, bopts)
            state = torch.empty(cfg.N * (cfg.S * cfg.d + cfg.S), device=dev, dtype=torch.float32)
        check(st)
        bws = torch.empty(max(bws_bytes // 4, 1), device=dev, dtype=torch.float32)
        if state is not None:  # the non-causal backward consumes the forward's state
            check(abi.fwd(*ptrs, state.data_ptr(), sh, False, opts, ws.data_ptr(), ws_bytes, stream))
    sptr = state.data_ptr() if state is not None else None

    def plain():
        if run_hashed:
            check(abi.hashed_fwd(*hptrs, None, sh, Kp, hopts, ws.data_ptr(), ws_bytes, stream))
        if run_hash:
            hash_both()
        if run_fwd:
            check(abi.fwd(*ptrs, sptr, sh, cfg.causal, opts, ws.data_ptr(), ws_bytes, stream))
        if run_bwd:
            if cfg.causal:
                check(abi.causal_bwd(*bptrs, *gptrs, sh, bopts, bws.data_ptr(), bws_bytes, stream))
            else:
                check(abi.noncausal_bwd(*bptrs, sptr, *gptrs, sh, bopts, bws.data_ptr(), bws_bytes,
                                        stream))

    def profiled(evs):
        n_used = 0
        if run_hashed:
            st_, n = abi.hashed_fwd_profiled(*hptrs, None, sh, Kp, hopts, ws.data_ptr(), ws_bytes,
                                             stream, evs)
            check(st_)
            n_used += n
        if run_hash:
            events.record(evs[0], stream)
            for j, (x_, p_) in enumerate(((xq, q), (xk, k))):
                check(abi.hash_probs(x_.data_ptr(), planes_T.data_ptr(), p_.data_ptr(), cfg.N * T,
                                     cfg.d, cfg.L, Kp, hdt, stream))
                events.record(evs[j + 1], stream)
            n_used = 3
        if run_fwd:
            tail = (ctypes.c_void_p * (len(evs) - n_used)).from_buffer(evs, n_used * ctypes.sizeof(ctypes.c_void_p))
            st_, n = abi.fwd_profiled(*ptrs, sptr, sh, cfg.causal, opts, ws.data_ptr(), ws_bytes,
                                      stream, tail)
            check(st_)
            n_used += n
        if run_bwd:
            tail = (ctypes.c_void_p * (len(evs) - n_used)).from_buffer(evs, n_used * ctypes.sizeof(ctypes.c_void_p))
            if cfg.causal:
                st_, n = abi.causal_bwd_profiled(*bptrs, *gptrs, sh, bopts, bws.data_ptr(), bws_bytes,
                                                 stream, tail)
            else:
                st_, n = abi.noncausal_bwd_profiled(*bptrs, sptr, *gptrs, sh, bopts, bws.data_ptr(),
                                                    bws_bytes, stream, tail)
            check(st_)
            n_used += n
        return n_used

    fwd_names = PHASES.get((cfg.causal, family), [])
    if not cfg.causal and tiles <= NONCAUSAL_FOLD_TILES:
        fwd_names = [n for n in fwd_names if n != "tile_reduce"]
    names = []
    if run_hashed:
        names += PHASES[(True, "hashed")]
    if run_hash:
        names += ["hash_q", "hash_k"]
    if run_fwd:
        names += fwd_names
    if run_bwd:
        names += BWD_PHASES[cfg.causal]

    if args.calibrate_copy:
        # A plain copy of known size: its FETCH_SIZE / WRITE_SIZE counters give
        # the scale of those counters on this device.
        src = torch.ones(args.calibrate_copy << 18, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    events = HipEvents()
    max_launches = 16
    per_step = [events.array(max_launches + 2) for _ in range(args.steps)]
    warm = events.array(max_launches + 2)

    for _ in range(args.warmup):
        plain()
        profiled(warm)
    torch.cuda.synchronize()

    # Timed region 1 (`value`): K plain steps, back to back on one stream,
    # between two events.
    bracket = events.array(2)
    t0 = time.perf_counter()
    events.record(bracket[0], stream)
    for _ in range(args.steps):
        plain()
    events.record(bracket[1], stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = events.elapsed_ms(bracket[0], bracket[1]) / args.steps

    # Timed region 2 (per-kernel durations): K profiled steps, which put an
    # event before the first launch and after every launch.
    n_events = 0
    for i in range(args.steps):
        n_events = profiled(per_step[i])
    torch.cuda.synchronize()

    profiled_ms = events.elapsed_ms(per_step[0][0], per_step[-1][n_events - 1]) / args.steps
    # Intervals between consecutive events; the forward's last event and the
    # backward's first one bracket nothing and are dropped below.
    n_gaps = n_events - 1
    gaps = [statistics.fmean(events.elapsed_ms(ev[j], ev[j + 1]) for ev in per_step)
            for j in range(n_gaps)]
    n_fwd = len(fwd_names) if run_fwd else 0
    if run_fwd and run_bwd:
        gaps = gaps[:n_fwd] + gaps[n_fwd + 1:]
    if run_hash:  # the forward's first event follows the hashing's last one
        gaps = gaps[:2] + gaps[3:]
    n_launch = len(gaps)
    phase_ms = gaps
    if len(names) != n_launch:
        names = [f"kernel{j}" for j in range(n_launch)]
    dom = max(range(n_launch), key=lambda j: phase_ms[j])
    dom_bytes = phase_bytes(names[dom], cfg, T, es, tiles, rec)
    achieved = dom_bytes / (phase_ms[dom] * 1e-3) / 1e9
    peak_bytes = torch.cuda.max_memory_allocated(dev)
    events.destroy()

    NT = cfg.N * T
    value = NT / (ms_per_step * 1e-3) / 1e6
    headline = args.workload == "cfg2" and args.pass_ == "fwd"
    metric = METRIC if headline else (
        f"{'causal' if cfg.causal else 'non-causal'} {args.pass_} M tokens/s at N={cfg.N},"
        f"S={cfg.S},d_k={cfg.d},T={T} on 1 GPU")
    total_mem = torch.cuda.get_device_properties(dev).total_memory
    bytes_per_token = peak_bytes / T
    result = {
        "metric": metric,
        "value": round(value, 3),
        "unit": UNIT,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (round(value / REFERENCE_MTOKS_T65536, 2)
                        if (headline and T == 65536) else None),
        "dtype": "bf16" if es == 2 else "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: {'causal' if cfg.causal else 'non-causal'} {args.pass_} N={cfg.N} "
                        f"L={cfg.L} R={cfg.R} d={cfg.d} T={T} {'bf16' if es == 2 else 'fp32'}",
            "N": cfg.N, "T": T, "L": cfg.L, "R": cfg.R, "d": cfg.d, "causal": cfg.causal,
            "pass": args.pass_,
            "kernel": family, "tile_tokens": tile, "launches_per_step": n_launch,
            "kernel_ms": {names[j]: round(phase_ms[j], 5) for j in range(n_launch)},
            "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
            "profiled_ms_per_step": round(profiled_ms, 5),
            "peak_hbm_bytes_per_token": round(bytes_per_token, 1),
            "workspace_bytes_per_token": round(ws_bytes / T, 2),
            "max_T_fits_est": int(0.95 * total_mem / bytes_per_token),
            "alg_bytes_per_stream_token": op_bytes(args.pass_, cfg, 1, es) / cfg.N,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": names[dom],
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": traffic_for(args.workload if args.pass_ == "fwd" else
                                   f"{args.workload}/{args.pass_}", names[dom]),
            "alg_bytes_per_launch": int(dom_bytes),
            "whole_op_frac": round(op_bytes(args.pass_, cfg, T, es) / (ms_per_step * 1e-3) / 1e9
                                   / PEAK_HBM_GBPS, 4),
        },
        "cpu_baseline": None,
    }
    del q, k, v, out, ws
    if run_bwd:
        del g, dq, dk, dv, bws
    if run_hash or run_hashed:
        del xq, xk, planes_T, planes
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline and headline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    os.environ.setdefault("PYTHONUNBUFFERED", "1")
    sys.exit(main())
