"""The host side of bench.py's CPU baseline (no GPU): the per-T point in a
fresh process reports its time, threads and peak RSS, and the host
description holds what the CPU plan asks for (os.cpu_count(), the threads
used, the CPU model)."""
from __future__ import annotations

import importlib.util
import os
import pathlib

REPO = pathlib.Path(__file__).resolve().parents[1]


def load_bench():
    spec = importlib.util.spec_from_file_location("race_bench", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_host_info_names_cores_threads_and_model():
    info = load_bench().host_cpu_info()
    assert info["cpu_count"] == os.cpu_count()
    assert 1 <= info["threads"] <= os.cpu_count()
    assert info["affinity_cpus"] >= 1
    assert "cpu_model" in info and "mem_available_bytes" in info


def test_cpu_point_runs_in_a_fresh_process():
    b = load_bench()
    pt = b.cpu_point(2, 256, 2, 4, 16, 2, timeout=300)
    assert pt["N"] == 2 and pt["T"] == 256 and pt["S"] == 8 and pt["d"] == 16
    assert pt["threads"] == 2
    assert pt["ms"] > 0 and pt["m_tokens_per_s"] > 0
    lo, hi = pt["ms_min_max"]
    assert lo <= pt["ms"] <= hi
    # The child's own peak: at least its inputs, and a fresh interpreter's.
    assert pt["peak_rss_bytes"] >= pt["input_bytes"]
    assert pt["predicted_peak_bytes"] > pt["input_bytes"]


def test_sweep_lengths_cover_cfg1_and_cfg2():
    b = load_bench()
    assert 4096 in b.CPU_SWEEP_T and b.CPU_SWEEP_T[-1] == 65536
    assert b.GPU_SWEEP_T == [512 << i for i in range(8)]


def test_noncausal_backward_launch_names_follow_the_library():
    # race_api.hip: at S = d = 64 the query side and the key side (with the
    # finalize between them past 4 tiles per stream); five passes otherwise.
    b = load_bench()
    assert b.noncausal_bwd_phases(64, 64, 2) == ["query_grad", "key_grad"]
    assert b.noncausal_bwd_phases(64, 64, 8) == ["query_grad", "bwd_finalize", "key_grad"]
    assert b.noncausal_bwd_phases(256, 128, 2) == b.BWD_PHASES[False]


def test_causal_backward_launch_names_follow_the_library():
    # race_api.hip: one 64 x 64 block at S = d = 64; bf16 with d = 128 and S
    # = 128 or 256, after the forward's tile sums and scan the forward walks
    # of every 128-bucket block in one launch, one reverse scan, then a
    # backward walk per block; other shapes get generic names.
    b = load_bench()
    assert b.causal_bwd_phases(64, 64, 4) == b.BWD_PHASES[True]
    assert b.causal_bwd_phases(256, 128, 2) == [
        "bwd_tile_sums", "tile_scan", "bwd_dq_walks", "suffix_scan_blocks", "bwd_dkv_pair0",
        "bwd_dkv_pair1"]
    assert len(b.causal_bwd_phases(128, 128, 2)) == 5
    assert b.causal_bwd_phases(256, 128, 4) == []
    # Streams that fill the device: whole-stream forward walks, no tile sums or scan.
    assert b.causal_bwd_phases(256, 128, 2, True) == [
        "bwd_dq_walks", "suffix_scan_blocks", "bwd_dkv_pair0", "bwd_dkv_pair1"]



class _FakeEvents:
    """Stands in for HipEvents: each plain() step 'takes' 0.5 ms of GPU time."""

    def __init__(self):
        self.pending = 0

    def array(self, n):
        return [None] * n

    def record(self, h, stream):
        pass

    def elapsed_ms(self, a, b):
        dt, self.pending = 0.5 * self.pending, 0
        return dt


def test_settle_runs_until_the_gpu_time_is_reached(monkeypatch):
    b = load_bench()
    import torch
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    ev = _FakeEvents()
    ran = []

    def plain():
        ran.append(1)
        ev.pending += 1

    got = b.settle(plain, 0, ev, 250.0)
    assert got["settle_steps"] == len(ran)
    # The last batch aims at the time still missing, so it overshoots by at most a step or two.
    assert 250.0 <= got["settle_ms"] <= 251.0
    assert b.settle(plain, 0, ev, 0.0) == {"settle_ms": 0.0, "settle_steps": 0}
