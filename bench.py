#!/usr/bin/env python3
"""Benchmark of race_fused_fwd on one MI355X; prints ONE JSON line.

Default workload (cfg2, the configuration the headline metric is quoted on):
causal forward, N = 8 streams, L = 4, R = 16 (S = 64), d = 64, T = 65536,
fp32, synthetic inputs (softmax probabilities of N(0,1)*4 logits, N(0,1)
values) generated on the GPU and resident in HBM before the timed region.  A "step" is one
race_fused_fwd pass over that batch: every kernel of the op, through the C
ABI (include/race_mi355x.h), with caller-owned output and workspace.

Timing: W untimed warmup steps, then an untimed clock-settling phase (plain
steps until --settle-ms of GPU time has passed, 250 by default; reported as
config.settle_ms and config.settle_steps), then timed regions, each of K
steps bracketed by torch.cuda.synchronize() on both sides.  The first runs plain
race_fwd steps back to back on the stream between two HIP events: `value` =
N*T / (mean step time) in M tokens/s.  Every step reads the same inputs
(--input-sets R cycles through R sets instead), so part of them may still sit
in the 256 MB memory-side cache from the step before.  The second runs
race_fwd_profiled, which records a HIP event on the launch stream before the
first kernel and after every kernel; the per-kernel durations behind
`roofline` come from it (its step time, with the extra events, is
`profiled_ms_per_step`).  For the forward pass a third region runs K plain
steps alternating two input sets, which no step finds left over from the
step before: config.fresh_inputs.  For the causal backward on the matrix
cores a fourth region times K backward steps started, as autograd starts
them, from a forward call's scanned tile records (the backward's own tile
sums and scan skipped): config.bwd_from_saved_records.

roofline: the dominant kernel's algorithmic HBM bytes per launch (each
operand it streams read once, its output written once: bytes per
stream-token * N * T; workspace records excluded) / its mean duration,
against MI355X's 8 TB/s.  traffic: HBM bytes per launch measured with
rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (scaled by the same counters on a
plain copy of known size, --calibrate-copy), read from profiles/traffic.json
when a measurement for this workload exists, else null.

cpu_baseline: the reference's CPU path -- the fp32 torch cumsum + bmm
composition of src/race_baseline.py:45-51, as restated in oracle/ -- timed on
this host's cores (os.cpu_count() bounded by the CPUs this job may use),
each T in a fresh process (oracle/cpu_baseline.py, which also reports its
peak RSS): cfg1 (T = 4096) and the cfg2 shape at T = 512 ... 65536 while the
predicted peak fits in half the available memory; 1 warmup, median of 3.
`value` is the T = 65536 point.  The CPU points run before the GPU is
touched.

config.max_T_measured: the headline also runs the cfg2 forward at the
longest T (a multiple of 2^20) whose tensors fit the free device memory and
reports its T and M tokens/s.

Other workloads and passes (--workload, --pass bwd|fwdbwd) print the same
line for that configuration; the CPU baseline belongs to the headline
(cfg2 forward) only.  --sweep prints a markdown table over T = 512 ... 65536
instead of the JSON line.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2|cfg3|cfg4|cfg5]
                       [--pass fwd|bwd|fwdbwd|module] [--T T] [--kernel auto|valu|mfma|mfma_wg|single]
                       [--tile N] [--no-cpu-baseline] [--no-max-t] [--sweep]
                       [--calibrate-copy MIB] [--settle-ms MS]
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
    (True, "single"): ["single_arm", "single_pass"],
}
# Non-causal forwards with at most this many tiles per stream add the tile
# records inside the map (no tile_reduce launch), as race_api.hip does.
NONCAUSAL_FOLD_TILES = 4
# Backward launch sequences (every gradient requested).
BWD_PHASES = {
    True: ["bwd_tile_sums", "tile_scan", "bwd_dq", "suffix_scan", "bwd_dkv"],
    False: ["token_map_dq", "tile_sums_dE", "bwd_finalize", "token_map_dk", "token_map_dv"],
}


def causal_bwd_phases(S: int, d: int, es: int, whole_streams: bool = False) -> list:
    """The causal backward's launches as race_api.hip issues them (starting
    from the inputs): one 64 x 64 block at S = d = 64; with bf16 tokens, d =
    128 and S = 128 or 256, the forward walks of every 128-bucket block
    (pair of 64-bucket groups) in one launch, one reverse scan of all their
    records, then a backward walk per block; other shapes get generic
    names.  With `whole_streams` (the streams times the blocks fill the
    device's CUs, or one tile per stream) the forward walks go through whole
    streams and the forward's tile sums and scan are not run."""
    if S == 64 and d == 64:
        return BWD_PHASES[True]
    if es == 2 and d == 128 and S in (128, 256):
        names = [] if whole_streams else ["bwd_tile_sums", "tile_scan"]
        names += ["bwd_dq_walks", "suffix_scan_blocks"]
        return names + [f"bwd_dkv_pair{mp}" for mp in range(S // 128)]
    return []


def noncausal_bwd_phases(S: int, d: int, tiles: int) -> list:
    """The non-causal backward's launches as race_api.hip issues them: at
    S = d = 64 the query side and the key side, with the finalize between
    them past NONCAUSAL_FOLD_TILES tiles per stream; the five passes
    otherwise."""
    if S == 64 and d == 64:
        mid = ["bwd_finalize"] if tiles > NONCAUSAL_FOLD_TILES else []
        return ["query_grad"] + mid + ["key_grad"]
    return BWD_PHASES[False]


# Steps of the per-kernel (event-marked) region: each holds up to 66 HIP
# events, so it does not grow with --steps.
PROFILED_STEPS = 50

# Untimed clock-settling phase run after the warmup steps and right before
# the timed regions: plain steps until this much GPU time has passed.  The
# GPU sits idle while the CPU baseline runs, and its clock then ramps over
# several milliseconds of load; without this phase a window of 20 steps
# (about 3.6 ms at cfg2) measured mostly that ramp.
SETTLE_MS = 250.0
# Input sets the forward steps cycle through by default (--input-sets).
INPUT_SETS = 1
SETTLE_MAX_STEPS = 200000


def settle(plain, stream, events, target_ms: float) -> dict:
    """Runs plain() steps back to back, in batches that double, until the
    batches' GPU time (HIP events on `stream`) reaches target_ms; returns
    {"settle_ms": GPU ms spent, "settle_steps": steps run}.  Untimed: nothing
    here enters `value`."""
    import torch

    if target_ms <= 0:
        return {"settle_ms": 0.0, "settle_steps": 0}
    ev = events.array(2)
    spent, steps, batch = 0.0, 0, 4
    while spent < target_ms and steps < SETTLE_MAX_STEPS:
        events.record(ev[0], stream)
        for _ in range(batch):
            plain()
        events.record(ev[1], stream)
        torch.cuda.synchronize()
        dt = events.elapsed_ms(ev[0], ev[1])
        spent += dt
        steps += batch
        # Aim the next batch at the time still missing, at most doubling.
        per_step = max(dt / batch, 1e-4)
        batch = int(min(2 * batch, max(4, (target_ms - spent) / per_step + 1)))
    return {"settle_ms": round(spent, 2), "settle_steps": steps}


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
    # 2000 timed steps (about 0.3 s at cfg2): after a host-side pause the
    # GPU's clock ramps up over several milliseconds, which a window of a few
    # steps would mostly measure (cfg2 forward, 20 steps: 3190-3220 M tokens/s;
    # 200 after 2000 warmup, or 2000 after 5: 3345).
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
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
    ap.add_argument("--kernel", choices=["auto", "valu", "mfma", "mfma_wg", "decode", "single", "mfma_precise"],
                    default="auto")
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-max-t", action="store_true",
                    help="skip the headline's run at the longest T that fits (config.max_T_measured)")
    ap.add_argument("--sweep", action="store_true",
                    help="measure the pass at T = 512 ... 65536 and print a markdown table instead")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB before timing (rocprofv3 counter scale)")
    ap.add_argument("--input-sets", type=int, default=INPUT_SETS, metavar="R",
                    help="the forward's steps cycle through R input sets (probsQ, probsK, V, out); "
                         "with R >= 2 no step finds the previous step's operands in the 256 MB "
                         "memory-side cache; reported as config.input_sets")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="GPU milliseconds of untimed plain steps between the warmup and the timed "
                         "regions, so the clock has settled (0 turns the phase off); reported as "
                         "config.settle_ms and config.settle_steps")
    return ap.parse_args()


def phase_bytes(name: str, cfg, T: int, es: int, tiles: int, rec: int) -> float:
    """Algorithmic HBM bytes of one launch of kernel `name` (each operand once)."""
    NT = cfg.N * T
    S, d = cfg.S, cfg.d
    state = 4.0 * cfg.N * tiles * rec
    small = 4.0 * cfg.N * (S * d + S) * 3
    # Walks over 128-bucket blocks: the forward walks of every block (each
    # block's Q, K and dQ columns, every value column once), a backward walk
    # per block (its Q, K, dK columns, every value column, dV); the reverse
    # scan of four 64 x 64 record arrays per block.
    if name == "bwd_dq_walks":
        return es * (3 * S + 2 * d) * NT
    if name.startswith("bwd_dkv_pair"):
        return es * (3 * 128 + 3 * d) * NT
    if name == "suffix_scan_blocks":
        return 2 * 4.0 * 4 * (S // 128) * cfg.N * tiles * (64 * 64 + 64)
    return {
        "tile_sums": es * (S + d) * NT,
        "tile_sums_mfma": es * (S + d) * NT,
        "tile_scan": 2 * state,
        "tile_reduce": state,
        "output_pass_valu": es * (2 * S + 2 * d) * NT,
        "output_pass_mfma": es * (2 * S + 2 * d) * NT,
        "single_arm": 4.0 * cfg.N * tiles,         # zeroes one flag per tile
        "single_pass": es * (2 * S + 2 * d) * NT,  # q, k, v read once -> out
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
        "query_grad": es * (2 * S + d) * NT,       # q, dOut -> dQ (and the dE records)
        "key_grad": es * (2 * S + 2 * d) * NT,     # k, v -> dK, dV
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


def host_cpu_info() -> dict:
    """os.cpu_count(), the CPUs this process may run on (affinity and the
    cgroup quota), the thread count the baseline uses, the CPU model and
    the available host memory."""
    info = {"cpu_count": os.cpu_count()}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["affinity_cpus"] = os.cpu_count()
    quota = None
    try:
        q, period = pathlib.Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    info["cgroup_cpus"] = quota
    # Every core this job may use: os.cpu_count() (as BASELINE's plan asks),
    # bounded by the affinity mask, the cgroup quota and the OMP_NUM_THREADS
    # share the GPU box assigns to one GPU.
    threads = os.cpu_count() or 1
    for cap in (info["affinity_cpus"], quota, os.environ.get("OMP_NUM_THREADS")):
        try:
            if cap and int(cap) > 0:
                threads = min(threads, int(cap))
        except ValueError:
            pass
    info["threads"] = threads
    model = None
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, ValueError):
        pass
    if model is None:
        try:
            for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    info["cpu_model"] = model
    try:
        for line in pathlib.Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemAvailable:"):
                info["mem_available_bytes"] = int(line.split()[1]) * 1024
    except (OSError, ValueError):
        info["mem_available_bytes"] = None
    return info


# The CPU sweep of the cfg2 shape (BASELINE's CPU plan): every T whose
# predicted peak stays under half the available host memory; T = 4096 is
# also cfg1, the reference's CPU-runnable configuration.
CPU_SWEEP_T = [512, 1024, 2048, 4096, 8192, 16384, 32768, 65536]


def cpu_point(N, T, L, R, d, threads, timeout=600) -> dict:
    """One CPU point in a fresh interpreter (oracle/cpu_baseline.py)."""
    import subprocess

    cmd = [sys.executable, str(REPO / "oracle" / "cpu_baseline.py"), "--N", str(N), "--T", str(T),
           "--L", str(L), "--R", str(R), "--d", str(d), "--threads", str(threads)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if res.returncode != 0:
        raise RuntimeError(f"cpu baseline at T={T} failed ({res.returncode}): {res.stderr[-2000:]}")
    return json.loads(res.stdout.strip().splitlines()[-1])


def cpu_baseline():
    """The reference CPU path (torch fp32 cumsum + bmm) on this host.

    cfg1 (N = 8, T = 4096) always, then the cfg2 shape swept over T while its
    predicted peak fits in half the available memory; each point in a fresh
    process (its own peak RSS), 1 warmup + median of 3.  `value` is the
    bench workload's T = 65536 point (the largest measured T if that one
    does not fit)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("race_cpu_baseline", REPO / "oracle" / "cpu_baseline.py")
    cb = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(cb)
    info = host_cpu_info()
    N, L, R, d = 8, 4, 16, 64
    avail = info.get("mem_available_bytes") or (64 << 30)
    sweep, skipped = [], []
    for T in CPU_SWEEP_T:
        if cb.predicted_peak_bytes(N, T, L * R, d) > avail / 2:
            skipped.append(T)
            continue
        pt = cpu_point(N, T, L, R, d, info["threads"])
        print(f"# cpu T={T}: {pt['ms']:.1f} ms, {pt['m_tokens_per_s']:.4f} {UNIT}, peak RSS "
              f"{pt['peak_rss_bytes'] / 2**30:.2f} GiB", file=sys.stderr, flush=True)
        sweep.append({"T": T, "ms": pt["ms"], "ms_min_max": pt["ms_min_max"],
                      "m_tokens_per_s": pt["m_tokens_per_s"],
                      "peak_rss_bytes": pt["peak_rss_bytes"],
                      "predicted_peak_bytes": pt["predicted_peak_bytes"]})
    if not sweep:
        raise RuntimeError("cpu baseline: no T fits in half the available host memory")
    cfg1 = next((x for x in sweep if x["T"] == 4096), None)
    head = next((x for x in sweep if x["T"] == 65536), sweep[-1])
    return {
        "value": head["m_tokens_per_s"],
        "unit": UNIT,
        "cores": info["threads"],
        "kind": "port",
        "sample": (f"causal N={N} T={head['T']} L={L} R={R} d={d} fp32 (the cfg2 workload), the "
                   f"torch-CPU cumsum+bmm composition of src/race_baseline.py:45-51 "
                   f"(oracle/oracle.py torch_reference_path) in a fresh process per T, "
                   f"{info['threads']} threads, median of 3 after 1 warmup: {head['ms']:.1f} ms per "
                   f"call, peak RSS {head['peak_rss_bytes'] / 2**30:.2f} GiB"),
        "host": info,
        "cfg1": cfg1,
        "sweep": sweep,
        "skipped_host_memory": skipped,
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
    n_prof = min(args.steps, PROFILED_STEPS)
    per_step = [events.array(8) for _ in range(n_prof)]
    warm = events.array(8)
    for _ in range(args.warmup):
        plain()
        check(abi.alg1_fwd_profiled(*ptrs, None, sh, args.tile, variant, ws.data_ptr(), ws_bytes,
                                    stream, warm)[0])
    torch.cuda.synchronize()
    settled = settle(plain, stream, events, args.settle_ms)
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
    for i in range(n_prof):
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
            "tile_tokens": tile, "launches_per_step": len(gaps), **settled,
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
    n_prof = min(args.steps, PROFILED_STEPS)
    per_step = [events.array(8) for _ in range(n_prof)]
    for _ in range(args.warmup):
        plain()
    torch.cuda.synchronize()
    settled = settle(plain, stream, events, args.settle_ms)
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
    for i in range(n_prof):
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
            "launches_per_step": len(gaps), **settled,
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


def measure(args, T: int) -> dict:
    """One bench line (without cpu_baseline) for args' workload and pass at T."""
    import torch

    race = entry.load_package()
    from race_attention_kernel_amd import abi

    cfg_key, _ = WORKLOADS[args.workload]
    cfg = race.CONFIGS[cfg_key]
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
    if cfg.causal and (kernel_id in (2, 3, 6) or (kernel_id == 0 and race.ops._lib.ext().shape_supported(
            cfg.L, cfg.R, cfg.d)[1])):
        family = "mfma"
    if cfg.causal and kernel_id == race.ops.KERNELS["single"]:
        family = "single"
    ws = torch.empty(max(ws_bytes // 4, 1), device=dev, dtype=torch.float32)
    out = torch.empty_like(v)
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr())
    # The forward's steps cycle through `input_sets` sets of operands (other
    # seeds), so that with two or more a step never re-reads the previous
    # step's bytes from the memory-side cache.  Their memory is left out of
    # the peak-HBM figure, which describes one call.
    # A third timed region (`config.fresh_inputs`) alternates two sets, so its
    # figure never profits from the previous call's operands.
    n_sets = max(1, args.input_sets) if args.pass_ == "fwd" else 1
    n_alloc = max(n_sets, 2) if args.pass_ == "fwd" else 1
    sets = [(q, k, v, out)]
    extra_bytes = 0
    for j in range(1, n_alloc):
        qj, kj, vj = race.config_inputs(cfg, T, seed=j, device=dev, gen_device="cuda")
        sets.append((qj, kj, vj, torch.empty_like(vj)))
        extra_bytes += sum(x.numel() * x.element_size() for x in sets[-1])
    ptr_sets = [tuple(x.data_ptr() for x in st_) for st_ in sets]
    turn = [0]
    active = [n_sets]

    def fwd_ptrs():
        p_ = ptr_sets[turn[0] % active[0]]
        turn[0] += 1
        return p_

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
            check(abi.fwd(*fwd_ptrs(), sptr, sh, cfg.causal, opts, ws.data_ptr(), ws_bytes, stream))
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
            st_, n = abi.fwd_profiled(*fwd_ptrs(), sptr, sh, cfg.causal, opts, ws.data_ptr(), ws_bytes,
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
        whole = tiles == 1 or cfg.N * (cfg.S // 128) >= torch.cuda.get_device_properties(dev).multi_processor_count
        names += (causal_bwd_phases(cfg.S, cfg.d, es, whole) if cfg.causal
                  else noncausal_bwd_phases(cfg.S, cfg.d, tiles))

    if args.calibrate_copy:
        # A plain copy of known size: its FETCH_SIZE / WRITE_SIZE counters give
        # the scale of those counters on this device.
        src = torch.ones(args.calibrate_copy << 18, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    events = HipEvents()
    max_launches = 64
    n_prof = min(args.steps, PROFILED_STEPS)
    per_step = [events.array(max_launches + 2) for _ in range(n_prof)]
    warm = events.array(max_launches + 2)

    for _ in range(args.warmup):
        plain()
        profiled(warm)
    torch.cuda.synchronize()
    settled = settle(plain, stream, events, args.settle_ms)

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

    # Timed region 2 (per-kernel durations): min(K, PROFILED_STEPS) profiled
    # steps, which put an event before the first launch and after every launch.
    n_events = 0
    for i in range(n_prof):
        n_events = profiled(per_step[i])
    torch.cuda.synchronize()

    profiled_ms = events.elapsed_ms(per_step[0][0], per_step[-1][n_events - 1]) / n_prof

    # Timed region 3 (forward only): K plain steps alternating two input sets.
    fresh = None
    if args.pass_ == "fwd":
        active[0] = 2
        events.record(bracket[0], stream)
        for _ in range(args.steps):
            plain()
        events.record(bracket[1], stream)
        torch.cuda.synchronize()
        active[0] = n_sets
        fresh_ms = events.elapsed_ms(bracket[0], bracket[1]) / args.steps
        fresh = {"input_sets": 2, "ms_per_step": round(fresh_ms, 5),
                 "m_tokens_per_s": round(cfg.N * T / (fresh_ms * 1e-3) / 1e6, 3),
                 "whole_op_frac": round(op_bytes(args.pass_, cfg, T, es) / (fresh_ms * 1e-3) / 1e9
                                        / PEAK_HBM_GBPS, 4)}
    # Timed region 4 (causal backward on the matrix cores): the backward as
    # autograd runs it, from a forward call's scanned tile records (the
    # backward's own tile sums and scan skipped), K steps after W warmup
    # steps.  Its workspace is left out of the peak-HBM figure.
    peak_bytes = torch.cuda.max_memory_allocated(dev) - extra_bytes
    from_records = None
    if args.pass_ == "bwd" and cfg.causal and family == "mfma":
        check(abi.fwd(*ptrs, None, sh, True, opts, ws.data_ptr(), ws_bytes, stream))
        ropts = abi.options(tile, 0)
        st_, rws_bytes = abi.causal_bwd_from_records_workspace_bytes(sh, ropts)
        check(st_)
        rws = torch.empty(max(rws_bytes // 4, 1), device=dev, dtype=torch.float32)

        def from_rec():
            check(abi.causal_bwd_from_records(*bptrs, ws.data_ptr(), *gptrs, sh, ropts, rws.data_ptr(),
                                              rws_bytes, stream))

        for _ in range(args.warmup):
            from_rec()
        events.record(bracket[0], stream)
        for _ in range(args.steps):
            from_rec()
        events.record(bracket[1], stream)
        torch.cuda.synchronize()
        rec_ms = events.elapsed_ms(bracket[0], bracket[1]) / args.steps
        from_records = {"ms_per_step": round(rec_ms, 5),
                        "m_tokens_per_s": round(cfg.N * T / (rec_ms * 1e-3) / 1e6, 3),
                        "tile_tokens": tile}
        del rws
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
    # The extra input sets are left out of the peak (taken above): it
    # describes one call.
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
            "kernel": family, "tile_tokens": tile, "launches_per_step": n_launch, **settled,
            "input_sets": n_sets,
            "fresh_inputs": fresh,
            "bwd_from_saved_records": from_records,
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
    del q, k, v, out, ws, sets, ptr_sets
    if run_bwd:
        del g, dq, dk, dv, bws
    if run_hash or run_hashed:
        del xq, xk, planes_T, planes
    torch.cuda.empty_cache()
    return result


def max_t_leg(steps: int = 3) -> dict:
    """The cfg2 forward (fp32, N = 8, S = d = 64) at the longest T whose four
    tensors and workspace fit in 92% of the free device memory, T a multiple
    of 2^20: 1 warmup step, then `steps` timed ones between two HIP events.
    Inputs are filled a chunk of tokens at a time (no full-size
    temporaries) with the BASELINE distribution."""
    import torch

    race = entry.load_package()
    from race_attention_kernel_amd import abi

    N, L, R, d = 8, 4, 16, 64
    S = L * R
    dev = torch.device("cuda:0")
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info(dev)
    per_token = N * (2 * S + 2 * d) * 4
    opts = abi.options(0, 0)
    T = int(0.92 * free / per_token) >> 20 << 20
    while T > 0:
        sh = abi.shape(N, T, L, R, d, abi.RACE_F32)
        st, ws_bytes, tiles, _ = abi.fwd_workspace_bytes(sh, True, opts)
        if st != 0:
            raise RuntimeError(abi.status_string(st))
        if T * per_token + ws_bytes <= 0.92 * free:
            break
        T -= 1 << 20
    if T <= 0:
        return {"T": 0, "note": "no 2^20-token multiple fits"}
    torch.cuda.reset_peak_memory_stats(dev)
    q = torch.empty((N, T, L, R), device=dev, dtype=torch.float32)
    k = torch.empty_like(q)
    v = torch.empty((N, T, d), device=dev, dtype=torch.float32)
    out = torch.empty_like(v)
    ws = torch.empty(max(ws_bytes // 4, 1), device=dev, dtype=torch.float32)
    g = torch.Generator(device=dev).manual_seed(3)
    chunk = 1 << 22
    for n in range(N):
        for c in range(0, T, chunk):
            e = min(T, c + chunk)
            for x in (q, k):
                x[n, c:e] = torch.softmax(torch.randn((e - c, L, R), generator=g, device=dev) * 4.0, -1)
            v[n, c:e] = torch.randn((e - c, d), generator=g, device=dev)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr())

    def step():
        st_ = abi.fwd(*ptrs, None, sh, True, opts, ws.data_ptr(), ws_bytes, stream)
        if st_ != 0:
            raise RuntimeError(abi.status_string(st_))

    step()
    torch.cuda.synchronize()
    events = HipEvents()
    ev = events.array(2)
    events.record(ev[0], stream)
    for _ in range(steps):
        step()
    events.record(ev[1], stream)
    torch.cuda.synchronize()
    ms = events.elapsed_ms(ev[0], ev[1]) / steps
    events.destroy()
    peak = torch.cuda.max_memory_allocated(dev)
    del q, k, v, out, ws
    torch.cuda.empty_cache()
    return {
        "T": T, "N": N, "dtype": "f32", "steps": steps, "ms_per_step": round(ms, 3),
        "m_tokens_per_s": round(N * T / (ms * 1e-3) / 1e6, 1),
        "peak_hbm_bytes": peak, "hbm_total_bytes": total, "tile_tokens": T // tiles,
    }


# The GPU sweep of the cfg2 shape (T = 512 to
# 65536, powers of two).
GPU_SWEEP_T = [512, 1024, 2048, 4096, 8192, 16384, 32768, 65536]


def sweep(args) -> int:
    """--sweep: one measurement per T of the workload's pass; prints a
    markdown table (and no JSON line)."""
    rows = []
    for T in GPU_SWEEP_T:
        r = measure(args, T)
        print(f"# T={T}: {r['value']:.1f} {UNIT}", file=sys.stderr, flush=True)
        rows.append(r)
    print(f"{rows[0]['metric'].split(' at ')[0]} sweep, workload {args.workload}, "
          f"{args.steps} timed steps after {args.warmup} warmup\n")
    print("| T | M tokens/s | ms / step | peak HBM bytes / token (T) | whole-op HBM frac "
          "| dominant kernel | its frac | kernel ms |")
    print("|---|---|---|---|---|---|---|---|")
    for r in rows:
        c, rf = r["config"], r["roofline"]
        kms = ", ".join(f"{k_}: {v_:.4f}" for k_, v_ in c["kernel_ms"].items())
        print(f"| {c['T']} | {r['value']:.1f} | {r['ms_per_step']:.4f} | {c['peak_hbm_bytes_per_token']:.0f} "
              f"| {rf['whole_op_frac']:.3f} | {rf['kernel']} | {rf['frac']:.3f} | {kms} |")
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
    if args.sweep:
        return sweep(args)
    T = args.T or WORKLOADS[args.workload][1]
    headline = args.workload == "cfg2" and args.pass_ == "fwd"
    # The CPU points run first, in child processes started before this
    # process touches the GPU.
    cpu = cpu_baseline() if (headline and not args.no_cpu_baseline) else None
    result = measure(args, T)
    if headline and not args.no_max_t:
        result["config"]["max_T_measured"] = max_t_leg()
    result["cpu_baseline"] = cpu
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    os.environ.setdefault("PYTHONUNBUFFERED", "1")
    sys.exit(main())
