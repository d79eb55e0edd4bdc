"""GPU parity of the causal forward against the CPU oracle (fp64).

Mirrors the reference's causal GPU suite (src/causal_v2/tests/test_forward_cuda.py):
parameter grids over shapes and ragged T, forced tile lengths, prefix states
against an emulation of the decomposition, bitwise reproducibility and
causality, NaN stream isolation, empty sequences and invalid-input
rejection -- restated for the per-bucket function of src/race_baseline.py:45-51.
Tolerances (north star): fp32 max rel err 1e-4, bf16 inputs 2e-2, defined as
max |out - ref| / max |ref| per stream.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, assert_bf16_floor, per_stream_rel_err, say, to_np, tol_for

pytestmark = pytest.mark.gpu

KERNELS = ["valu", "mfma", "mfma_wg"]


def has_mfma(ext, L, R, d):
    return ext.shape_supported(L, R, d)[1]


def skip_unless_kernel(ext, kernel, L, R, d):
    if kernel in ("mfma", "mfma_wg") and not has_mfma(ext, L, R, d):
        pytest.skip(f"no MFMA specialization for S={L * R}, d={d}")


def run(race, q, k, v, kernel="auto", tile=0):
    out = race.race_fused_fwd(q, k, v, causal=True, kernel=kernel, tile_tokens=tile)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("T", [512, 1024, 2048, 4096, 8192, 16384, 32768, 65536])
def test_cfg2_sweep_matches_oracle(race, ext, oracle, cuda, kernel, T):
    # cfg2: N=8, L=4, R=16, d=64, fp32, every T in 512..65536.
    skip_unless_kernel(ext, kernel, 4, 16, 64)
    say("cfg2", kernel, "T", T)
    q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=T)
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda), kernel)
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), nthreads=16)
    err = per_stream_rel_err(to_np(out), ref)
    say("cfg2", kernel, "T", T, "max rel err", f"{err:.3e}")
    assert err <= FP32_TOL


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L, R, d", [(1, 1, 1), (1, 2, 16), (2, 8, 32), (4, 16, 64), (3, 5, 7),
                                     (8, 32, 128), (16, 16, 128), (4, 16, 128), (8, 16, 64),
                                     (16, 16, 64)])
@pytest.mark.parametrize("T", [1, 63, 65, 300])
def test_shapes_and_ragged_lengths(race, ext, oracle, cuda, kernel, dtype, L, R, d, T):
    skip_unless_kernel(ext, kernel, L, R, d)
    say("shape", kernel, dtype, L, R, d, T)
    q, k, v = race.make_inputs(3, T, L, R, d, seed=L * 1000 + R * 10 + d + T, dtype=dtype)
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda), kernel)
    assert out.dtype == dtype and out.shape == v.shape
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v))
    assert per_stream_rel_err(to_np(out), ref) <= tol_for(dtype)


@pytest.mark.parametrize("T, tile", [(1, 64), (31, 64), (33, 64), (95, 64), (96, 128), (1000, 64),
                                     (1000, 128), (4097, 2048), (5000, 1024)])
def test_s256_bf16_sub_chunks_and_tiles(race, ext, oracle, cuda, T, tile):
    # S = 256, d = 128, bf16 (the cfg5 shape's eight-wave workgroup output
    # pass, 32-token sub-chunks): ragged last sub-chunks, one-sub-chunk tiles
    # and several tiles per stream, against the oracle and against the fp32
    # path on the same values.
    skip_unless_kernel(ext, "mfma_wg", 8, 32, 128)
    say("s256 bf16", T, tile)
    q, k, v = race.make_inputs(2, T, 8, 32, 128, seed=T + 3 * tile, dtype=torch.bfloat16)
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda), "mfma_wg", tile)
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v))
    assert per_stream_rel_err(to_np(out), ref) <= tol_for(torch.bfloat16)
    f32 = run(race, q.float().to(cuda), k.float().to(cuda), v.float().to(cuda), "mfma_wg", tile)
    assert per_stream_rel_err(to_np(out), to_np(f32).astype(np.float64)) <= tol_for(torch.bfloat16)


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 127, 129, 2047, 2049, 3 * 2048 + 17, 10000])
def test_forced_tile_lengths_agree(race, ext, oracle, cuda, kernel, T):
    skip_unless_kernel(ext, kernel, 4, 16, 64)
    say("tiles", kernel, T)
    q, k, v = race.make_inputs(2, T, 4, 16, 64, seed=T + 5)
    qd, kd, vd = q.to(cuda), k.to(cuda), v.to(cuda)
    ref = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v))
    outs = []
    for tile in (64, 128, 2048):
        out = run(race, qd, kd, vd, kernel, tile)
        assert per_stream_rel_err(to_np(out), ref) <= FP32_TOL
        outs.append(to_np(out).astype(np.float64))
    for other in outs[1:]:
        assert per_stream_rel_err(other, outs[0]) <= 2 * FP32_TOL


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("T, tile", [(1, 64), (777, 64), (5000, 128), (20000, 2048), (4096, 1024)])
@pytest.mark.parametrize("L, R, d", [(4, 16, 64), (2, 4, 24), (8, 32, 128)])
def test_prefix_states_match_oracle_decomposition(race, ext, oracle, cuda, kernel, T, tile, L, R, d):
    skip_unless_kernel(ext, kernel, L, R, d)
    say("prefix", kernel, T, tile, L, R, d)
    q, k, v = race.make_inputs(2, T, L, R, d, seed=T + tile)
    out, records, state, used = ext.forward_debug(q.to(cuda), k.to(cuda), v.to(cuda), True, tile,
                                                  race.ops.KERNELS[kernel])
    torch.cuda.synchronize()
    assert used == tile
    S = L * R
    o_out, o_pref, o_fin = oracle.causal_tiled(to_np(q), to_np(k), to_np(v), tile, 64)
    rec = records[..., : S * d + S].cpu().double().numpy()
    assert rec.shape == o_pref.shape
    assert not rec[:, 0].any()
    scale = np.abs(o_fin).max()
    assert np.abs(rec - o_pref).max() <= 1e-5 * scale
    assert np.abs(state.cpu().double().numpy() - o_fin).max() <= 1e-5 * scale
    assert per_stream_rel_err(to_np(out), o_out) <= FP32_TOL


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("T", [129, 10000, 70000])
def test_runs_are_bitwise_identical(race, ext, cuda, kernel, T):
    skip_unless_kernel(ext, kernel, 4, 16, 64)
    say("bitwise", kernel, T)
    q, k, v = (x.to(cuda) for x in race.make_inputs(4, T, 4, 16, 64, seed=13))
    first = ext.forward_debug(q, k, v, True, 0, race.ops.KERNELS[kernel])
    for _ in range(3):
        again = ext.forward_debug(q, k, v, True, 0, race.ops.KERNELS[kernel])
        for a, b in zip(first[:3], again[:3]):
            assert torch.equal(a, b)
        assert first[3] == again[3]


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("position", [0, 31, 63, 64, 2047, 2048, 5000])
def test_future_tokens_do_not_change_the_past(race, ext, cuda, kernel, position):
    skip_unless_kernel(ext, kernel, 4, 16, 64)
    say("causality", kernel, position)
    T = 6000
    q, k, v = (x.to(cuda) for x in race.make_inputs(2, T, 4, 16, 64, seed=12))
    future = torch.arange(position + 1, T, device=cuda)
    shuffled = future[torch.randperm(len(future), device=cuda)]
    k2, v2 = k.clone(), v.clone()
    k2[:, future] = k[:, shuffled]
    v2[:, future] = -3.0 * v[:, shuffled]
    for tile in (64, 2048):
        out = run(race, q, k, v, kernel, tile)
        out2 = run(race, q, k2, v2, kernel, tile)
        assert torch.equal(out[:, : position + 1], out2[:, : position + 1])
        assert not torch.equal(out[:, position + 1:], out2[:, position + 1:])


@pytest.mark.parametrize("kernel", KERNELS)
def test_other_streams_cannot_leak_into_a_stream(race, ext, oracle, cuda, kernel):
    skip_unless_kernel(ext, kernel, 4, 16, 64)
    say("nan-isolation", kernel)
    q, k, v = race.make_inputs(3, 3000, 4, 16, 64, seed=14)
    ref = oracle.causal_recurrence(to_np(q[:1]), to_np(k[:1]), to_np(v[:1]))
    for x in (q, k, v):
        x[1:] = float("nan")
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda), kernel, 128)
    assert torch.isfinite(out[0]).all()
    assert torch.isnan(out[1:]).all()
    assert per_stream_rel_err(to_np(out[:1]), ref) <= FP32_TOL


def test_empty_sequence_and_no_streams(race, ext, cuda):
    say("empty")
    for N, T in ((2, 0), (0, 5), (0, 0)):
        q, k, v = (x.to(cuda) for x in race.make_inputs(N, T, 4, 16, 64))
        out, state = ext.forward(q, k, v, True, 0, 0, True)
        torch.cuda.synchronize()
        assert out.shape == (N, T, 64) and state.shape == (N, 64 * 64 + 64)
        assert not state.any()
        out, records, state, tile = ext.forward_debug(q, k, v, True, 0, 0)
        assert records.shape[1] == 0


def test_rejects_invalid_inputs(race, ext, cuda):
    say("invalid-inputs")
    q, k, v = (x.to(cuda) for x in race.make_inputs(1, 64, 4, 16, 64))
    q2 = torch.empty(1, 64 * 64 + 1, device=cuda)[:, 1:].view(1, 64, 4, 16)
    bad_calls = {
        "mixed dtypes": (q, k.to(torch.bfloat16), v),
        "fp16": (q.half(), k.half(), v.half()),
        "cpu V": (q, k, v.cpu()),
        "non-contiguous V": (q, k, v.transpose(1, 2).contiguous().transpose(1, 2)),
        "misaligned probsQ": (q2, k, v),
        "S > 256": (torch.rand(1, 64, 16, 17, device=cuda), torch.rand(1, 64, 16, 17, device=cuda), v),
        "d > 128": (q, k, torch.rand(1, 64, 129, device=cuda)),
        "shape mismatch": (q, k[:, :32].contiguous(), v),
        "V length mismatch": (q, k, v[:, :32].contiguous()),
        "5-D probs": (q[None], k[None], v),
    }
    for label, args in bad_calls.items():
        with pytest.raises(RuntimeError):
            ext.forward(*args, True)
            pytest.fail(f"accepted {label}")
    for tile in (48, -64):
        with pytest.raises(RuntimeError):
            ext.forward(q, k, v, True, tile, 0)


def test_first_output_closed_form(race, cuda):
    # T = 1: out_0 = v_0 * sum_s q_s k_s / (k_s + eps).
    say("first-output")
    q, k, v = race.make_inputs(4, 1, 4, 16, 64, seed=11)
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda))
    q0, k0 = q[:, 0].flatten(1).double(), k[:, 0].flatten(1).double()
    want = v[:, 0].double() * (q0 * k0 / (k0 + 1e-6)).sum(-1, keepdim=True)
    assert per_stream_rel_err(to_np(out[:, 0:1]), want[:, None].numpy()) <= FP32_TOL


@pytest.mark.parametrize("name", ["small", "one_token", "wide", "s1", "eps"])
def test_golden_vectors(race, cuda, name):
    import pathlib

    g = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "race_golden.npz")
    say("golden", name)
    q, k, v = (torch.from_numpy(g[f"{name}_{x}"]) for x in "qkv")
    out = run(race, q.to(cuda), k.to(cuda), v.to(cuda))
    assert per_stream_rel_err(to_np(out), g[f"{name}_causal"]) <= 1e-5


def test_cfg3_bf16_long_context(race, oracle, cuda):
    # cfg3: bf16 inputs, T = 2^17, 2^18 and 2^20, N = 8.  Inputs are generated
    # on the GPU; all 8 streams are copied back and checked against the fp64
    # oracle on the same bf16 values: the north-star bound and the rounding
    # floor bound (max <= 2.5 F, rms <= 2.0 F_rms).
    for T in (1 << 17, 1 << 18, 1 << 20):
        say("cfg3", T)
        q, k, v = race.make_inputs(8, T, 4, 16, 64, seed=T, dtype=torch.bfloat16, device=cuda,
                                   gen_device="cuda")
        out = run(race, q, k, v)
        assert torch.isfinite(out).all()
        o = to_np(out)
        qn, kn, vn = to_np(q), to_np(k), to_np(v)
        del q, k, v, out
        torch.cuda.empty_cache()
        ref = oracle.causal_recurrence(qn, kn, vn, nthreads=16)
        err = per_stream_rel_err(o, ref)
        say("cfg3", T, "max rel err", f"{err:.3e}")
        assert err <= 2e-2
        assert_bf16_floor(o, ref, float(np.abs(vn).max()), f"cfg3 T={T}")


def test_cfg5_bf16_large_buckets(race, oracle, cuda):
    # cfg5: N = 128, L = 8, R = 32 (S = 256), d = 128, T = 16384, bf16; 16 of
    # the 128 streams (every eighth) against the fp64 oracle.
    say("cfg5")
    q, k, v = race.make_inputs(128, 16384, 8, 32, 128, seed=5, dtype=torch.bfloat16, device=cuda,
                               gen_device="cuda")
    out = run(race, q, k, v)
    assert torch.isfinite(out).all()
    pick = list(range(0, 128, 8))
    o = to_np(out[pick])
    vn = to_np(v[pick])
    ref = oracle.causal_recurrence(to_np(q[pick]), to_np(k[pick]), vn, nthreads=16)
    err = per_stream_rel_err(o, ref)
    say("cfg5 max rel err", f"{err:.3e}")
    assert err <= 2e-2
    assert_bf16_floor(o, ref, float(np.abs(vn).max()), "cfg5")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [150, 200, 1000])
def test_s256_many_streams_ragged_tiles(race, oracle, cuda, dtype, T):
    # S = 256, d = 128 with 256 streams and 64-token tiles: odd and even tile
    # counts per stream, ragged last tiles, a grid of one to four rounds.
    # Eight streams spread over the batch against the oracle, and the final
    # state.
    say("s256 many streams", T, dtype)
    q, k, v = race.make_inputs(256, T, 8, 32, 128, seed=31 + T, dtype=dtype, device=cuda, gen_device="cuda")
    out, state = race.race_fused_fwd_with_state(q, k, v, causal=True, tile_tokens=64)
    torch.cuda.synchronize()
    pick = [0, 37, 74, 111, 148, 185, 222, 255]
    qn, kn, vn = (to_np(x[pick]) for x in (q, k, v))
    ref = oracle.causal_recurrence(qn, kn, vn, nthreads=16)
    assert per_stream_rel_err(to_np(out[pick]), ref) <= tol_for(dtype)
    # The state after the last token: B = K^T V, A = colsum K over the stream.
    kd, vd = kn.astype(np.float64), vn.astype(np.float64)
    b = np.einsum("nts,ntc->nsc", kd, vd)
    a = kd.sum(1)
    st = to_np(state[pick]).astype(np.float64)
    assert np.abs(st[:, :256 * 128] - b.reshape(len(pick), -1)).max() <= 1e-4 * np.abs(b).max()
    assert np.abs(st[:, 256 * 128:] - a).max() <= 1e-4 * np.abs(a).max()


def test_final_state_is_the_decode_handoff(race, oracle, cuda):
    say("final-state")
    q, k, v = race.make_inputs(2, 3333, 4, 16, 64, seed=21)
    out, state = race.race_fused_fwd_with_state(q.to(cuda), k.to(cuda), v.to(cuda), causal=True)
    torch.cuda.synchronize()
    _, fin = oracle.causal_recurrence(to_np(q), to_np(k), to_np(v), want_state=True)
    assert np.abs(state.cpu().double().numpy() - fin).max() <= 1e-5 * np.abs(fin).max()


def test_batched_ace_dropin(race, oracle, cuda):
    # The drop-in module's op against the oracle on the module's own probabilities.
    say("batched-ace")
    torch.manual_seed(1234)
    ace = race.BatchedACE(64, 4, 4, 1).to(cuda)
    g = torch.Generator().manual_seed(0)
    K, V, Q = (torch.randn(1, 1, 700, 8, 64, generator=g) for _ in range(3))
    out = ace(K.to(cuda), V.to(cuda), Q.to(cuda))
    torch.cuda.synchronize()
    N = 8
    k2 = K.permute(0, 1, 3, 2, 4).reshape(N, 700, 64).to(cuda)
    q2 = Q.permute(0, 1, 3, 2, 4).reshape(N, 700, 64).to(cuda)
    v2 = V.permute(0, 1, 3, 2, 4).reshape(N, 700, 64)
    pk = ace.bucket_probs(k2).flatten(2).cpu().numpy()
    pq = ace.bucket_probs(q2).flatten(2).cpu().numpy()
    ref = oracle.causal_recurrence(pq, pk, v2.numpy())
    got = out.permute(0, 1, 3, 2, 4).reshape(N, 700, 64)
    assert per_stream_rel_err(to_np(got), ref) <= FP32_TOL


def test_c_abi_direct_call_matches_the_binding(race, ext, cuda):
    # The raw C ABI through ctypes, on torch-allocated buffers and torch's stream.
    from race_attention_kernel_amd import abi

    say("c-abi")
    q, k, v = (x.to(cuda) for x in race.make_inputs(3, 1000, 4, 16, 64, seed=31))
    sh = abi.shape(3, 1000, 4, 16, 64, abi.RACE_F32)
    opts = abi.options(128, abi.RACE_KERNEL_AUTO)
    st, nbytes, tiles, rec = abi.fwd_workspace_bytes(sh, True, opts)
    assert st == 0 and tiles == 8
    ws = torch.empty(nbytes // 4, device=cuda)
    out = torch.empty_like(v)
    state = torch.empty(3, 64 * 64 + 64, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    st = abi.fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), state.data_ptr(), sh, True,
                 opts, ws.data_ptr(), nbytes, stream)
    assert st == 0, abi.status_string(st)
    torch.cuda.synchronize()
    want, want_state = ext.forward(q, k, v, True, 128, 0, True)
    torch.cuda.synchronize()
    assert torch.equal(out, want) and torch.equal(state, want_state)
    # Too small a workspace is refused without launching.
    assert abi.fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), None, sh, True, opts,
                   ws.data_ptr(), nbytes - 4, stream) == abi.RACE_ERROR_INVALID_VALUE
