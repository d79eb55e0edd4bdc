"""CPU tests of the boundary: the C-ABI library loads and exports what the header
declares, pure host logic (shape limits, workspace sizes, argument checks)
answers without touching a device, and the PyTorch binding validates its
inputs.  No kernel is launched here."""
from __future__ import annotations

import pathlib
import re

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "race_mi355x.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(race_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(race):
    from race_attention_kernel_amd import _lib, abi

    lib = _lib.cdll()
    names = declared_functions()
    assert names, "no declarations found in the header"
    for name in names:
        assert hasattr(lib, name), f"librace_mi355x.so does not export {name}"
    assert sorted(abi.EXPORTED_SYMBOLS) == names


def test_abi_version_and_status_strings(race):
    from race_attention_kernel_amd import abi

    assert abi.lib().race_abi_version() == 1
    assert abi.status_string(0) == "success"
    assert "invalid value" in abi.status_string(1)
    assert "gave up" in abi.status_string(abi.RACE_ERROR_SINGLE_PASS_GAVE_UP)


def test_single_status_refuses_other_kernels_on_the_host(race):
    # race_fwd_single_status names a RACE_KERNEL_SINGLE call; anything else is
    # refused before any device is touched.
    from race_attention_kernel_amd import abi

    sh = abi.shape(8, 4096, 4, 16, 64)
    for kernel in (abi.RACE_KERNEL_AUTO, abi.RACE_KERNEL_MFMA, abi.RACE_KERNEL_VALU):
        assert abi.fwd_single_status(sh, abi.options(0, kernel), 16, 1 << 20, 0) == \
            abi.RACE_ERROR_INVALID_VALUE
    assert abi.single_pass_test_give_up(False) == 0


@pytest.mark.parametrize("L, R, d, ok", [(4, 16, 64, True), (8, 32, 128, True), (1, 1, 1, True),
                                         (16, 16, 64, True), (16, 17, 64, False), (4, 16, 129, False),
                                         (0, 16, 64, False), (4, 16, 0, False)])
def test_shape_limits(race, L, R, d, ok):
    from race_attention_kernel_amd import abi

    supported, _ = abi.shape_supported(abi.shape(8, 1024, L, R, d))
    assert supported == ok


def test_stream_and_length_limits(race):
    from race_attention_kernel_amd import abi

    assert abi.shape_supported(abi.shape(65535, 1, 4, 16, 64))[0]
    assert not abi.shape_supported(abi.shape(65536, 1, 4, 16, 64))[0]
    assert not abi.shape_supported(abi.shape(-1, 1, 4, 16, 64))[0]
    assert not abi.shape_supported(abi.shape(8, 1, 4, 16, 64, dtype=7))[0]


def test_workspace_bytes_for_explicit_tiles(race):
    # Pure host arithmetic when the tile length is given (no device query).
    from race_attention_kernel_amd import abi

    sh = abi.shape(8, 65536, 4, 16, 64)
    st, nbytes, tiles, rec = abi.fwd_workspace_bytes(sh, True, abi.options(1024, abi.RACE_KERNEL_VALU))
    assert st == 0
    assert tiles == 64 and rec == 4160 and rec % 64 == 0
    assert nbytes == 8 * 64 * 4160 * 4
    # Ragged T: ceil division.
    st, _, tiles, _ = abi.fwd_workspace_bytes(abi.shape(2, 1025, 4, 16, 64), True, abi.options(512, 1))
    assert st == 0 and tiles == 3
    # Non-causal adds the E region.
    st, nc_bytes, _, _ = abi.fwd_workspace_bytes(sh, False, abi.options(1024, abi.RACE_KERNEL_VALU))
    assert st == 0 and nc_bytes == (8 * 64 * 4160 + 8 * 64 * 64) * 4
    st, bwd_bytes = abi.noncausal_bwd_workspace_bytes(sh, abi.options(1024, 0))
    # The dE tile records, then dB [N][S*d] and dA [N][S] (each region a
    # multiple of 64 floats).
    assert st == 0 and bwd_bytes == (8 * 64 * 4160 + 8 * 64 * 64 + 8 * 64) * 4
    # Causal backward: forward and suffix records, the running mass per 16
    # tokens and an fp32 copy of dQ.
    st, cb_bytes = abi.causal_bwd_workspace_bytes(sh, abi.options(1024, 0))
    assert st == 0
    assert cb_bytes == (2 * 8 * 64 * 4160 + 8 * 64 * (1024 // 16) * 64 + 8 * 65536 * 64) * 4
    # Starting from the forward's saved records needs no region for them, and
    # needs the forward's explicit tile length.
    st, rb_bytes = abi.causal_bwd_from_records_workspace_bytes(sh, abi.options(1024, 0))
    assert st == 0 and rb_bytes == cb_bytes - 8 * 64 * 4160 * 4
    assert abi.causal_bwd_from_records_workspace_bytes(sh, abi.options(0, 0))[0] == 1
    assert abi.causal_bwd_from_records_workspace_bytes(sh, None)[0] == 1


def test_causal_bwd_workspace_for_matrix_core_blocks(race):
    # S = 256, d = 128: 64 x 64 blocks on the matrix cores.  Forward records
    # of the full shape, suffix records of one block, the running mass every
    # 16 tokens and dq32 for one block; fp32 tokens add nothing.  bf16 tokens
    # take a forward and a backward walk per pair of bucket groups (128
    # buckets), the forward walks of every pair in one launch: per pair the
    # suffix records of its four blocks, its running mass (128 buckets every
    # 32 tokens) and dQ's bf16 remainders and bf16 part (N T x 128 x 4
    # bytes), and an fp32 running sum of dV (N T d) over the two pairs (the
    # walks write dQ and dK whole).  S = 128 is a single pair: no running sum.
    # Host arithmetic only.
    from race_attention_kernel_amd import abi

    def r64(x):
        return -(-x // 64) * 64

    N, T, S, d, tile = 2, 1000, 256, 128, 512
    tiles = -(-T // tile)
    rec_full, rec_blk = r64(S * d + S), r64(64 * 64 + 64)
    NT = N * T
    apre, dq32 = r64(N * tiles * (tile // 16) * 64), r64(NT * 64)
    base = N * tiles * rec_full + N * tiles * rec_blk + apre + dq32
    st, nbytes = abi.causal_bwd_workspace_bytes(abi.shape(N, T, 8, 32, d, abi.RACE_F32), abi.options(tile, 0))
    assert st == 0 and nbytes == base * 4
    apre_pair = r64(N * tiles * (tile // 32) * 128)
    pairs2 = N * tiles * rec_full + 8 * N * tiles * rec_blk + 2 * apre_pair + r64(2 * NT * 128)
    st, nbytes = abi.causal_bwd_workspace_bytes(abi.shape(N, T, 8, 32, d, abi.RACE_BF16), abi.options(tile, 0))
    assert st == 0 and nbytes == (pairs2 + r64(NT * d)) * 4
    rec_128 = r64(128 * d + 128)
    pair1 = N * tiles * rec_128 + 4 * N * tiles * rec_blk + apre_pair + r64(NT * 128)
    st, nbytes = abi.causal_bwd_workspace_bytes(abi.shape(N, T, 8, 16, d, abi.RACE_BF16), abi.options(tile, 0))
    assert st == 0 and nbytes == pair1 * 4
    # Forced vector-ALU walks: two column groups of 64, no block parts.
    st, vb = abi.causal_bwd_workspace_bytes(abi.shape(N, T, 8, 32, d, abi.RACE_F32),
                                            abi.options(tile, abi.RACE_KERNEL_VALU))
    assert st == 0
    assert vb == (N * tiles * rec_full + N * tiles * r64(S * 64 + S) + r64(N * tiles * (tile // 16) * S)
                  + r64(NT * S)) * 4


def test_precise_kernel_choice_on_the_host(race):
    # RACE_KERNEL_MFMA_PRECISE: the causal forward's workgroup kernels with
    # fp32-accurate products; same workspace as MFMA_WG, refused where there is
    # no matrix-core kernel, for the non-causal op and for the backward.
    from race_attention_kernel_amd import abi, ops

    assert ops.KERNELS["mfma_precise"] == abi.RACE_KERNEL_MFMA_PRECISE == 6
    for dt in (abi.RACE_BF16, abi.RACE_F32):
        sh = abi.shape(8, 4096, 8, 32, 128, dt)
        # An explicit tile: the automatic one reads the device's CU count.
        st, nb, tiles, rec = abi.fwd_workspace_bytes(sh, True, abi.options(512, abi.RACE_KERNEL_MFMA_PRECISE))
        assert st == 0 and tiles == 8
        assert (st, nb, tiles, rec) == abi.fwd_workspace_bytes(sh, True, abi.options(512, abi.RACE_KERNEL_MFMA_WG))
    bad = abi.options(512, abi.RACE_KERNEL_MFMA_PRECISE)
    assert abi.fwd_workspace_bytes(abi.shape(8, 4096, 3, 5, 7, abi.RACE_BF16), True, bad)[0] == \
        abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd_workspace_bytes(abi.shape(8, 4096, 4, 16, 64, abi.RACE_BF16), False, bad)[0] == \
        abi.RACE_ERROR_INVALID_VALUE
    assert abi.causal_bwd_workspace_bytes(abi.shape(8, 4096, 4, 16, 64, abi.RACE_BF16), bad)[0] == \
        abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd_workspace_bytes(abi.shape(8, 4096, 4, 16, 64), True, abi.options(512, 7))[0] == \
        abi.RACE_ERROR_INVALID_VALUE


def test_scratch_per_token_is_constant(race):
    # The causal workspace is O(T / tile): per token it stays at 4 * rec / tile bytes.
    from race_attention_kernel_amd import abi

    per_token = []
    for T in (1 << 17, 1 << 18, 1 << 20):
        st, nbytes, _, _ = abi.fwd_workspace_bytes(abi.shape(8, T, 4, 16, 64, abi.RACE_BF16), True,
                                                   abi.options(4096, 1))
        assert st == 0
        per_token.append(nbytes / T)
    assert max(per_token) == min(per_token) and per_token[0] <= 8 * 4160 * 4 / 4096 + 1e-9


@pytest.mark.parametrize("tile", [-64, 32, 100])
def test_invalid_tile_lengths_are_rejected(race, tile):
    from race_attention_kernel_amd import abi

    st, *_ = abi.fwd_workspace_bytes(abi.shape(8, 4096, 4, 16, 64), True, abi.options(tile, 1))
    assert st == abi.RACE_ERROR_INVALID_VALUE


def test_empty_calls_without_optional_outputs_touch_no_device(race):
    # An empty sequence with no state (or final state) asked for is a no-op:
    # nothing is launched, so it succeeds here without a GPU.  (It once
    # zero-filled the absent state through a null pointer.)
    from race_attention_kernel_amd import abi

    for causal in (True, False):
        assert abi.fwd(0, 0, 0, 0, None, abi.shape(2, 0, 4, 16, 64), causal, None, None, 0, 0) == 0
    assert abi.alg1_fwd(0, 0, 0, 0, 0, 0, None, abi.alg1_shape(2, 0, 64, 4, 4), 0, 0, None, 0,
                        0) == 0


def test_tiles_past_the_buffer_range_are_rejected(race):
    # The kernels address a tile's rows through one buffer resource, whose
    # range is a 32-bit byte count: 2^23 fp32 rows of 64 values are 2^31 bytes.
    from race_attention_kernel_amd import abi

    inv = abi.RACE_ERROR_INVALID_VALUE
    for kernel in (abi.RACE_KERNEL_VALU, abi.RACE_KERNEL_MFMA):
        big = abi.options(1 << 23, kernel)
        assert abi.fwd_workspace_bytes(abi.shape(8, 1 << 24, 4, 16, 64), True, big)[0] == inv
        assert abi.fwd_workspace_bytes(abi.shape(8, 1 << 24, 4, 16, 64), False, big)[0] == inv
        # The same tile in bf16 is 2^30 bytes, inside the range.
        assert abi.fwd_workspace_bytes(abi.shape(8, 1 << 24, 4, 16, 64, abi.RACE_BF16), True,
                                       big)[0] == 0
    # The widest operand sets the row length (S = 256 buckets here).
    assert abi.fwd_workspace_bytes(abi.shape(1, 1 << 22, 16, 16, 64), True,
                                   abi.options(1 << 21, 1))[0] == inv
    st, _ = abi.causal_bwd_workspace_bytes(abi.shape(8, 1 << 24, 4, 16, 64), abi.options(1 << 23, 0))
    assert st == inv
    assert abi.alg1_workspace_bytes(abi.alg1_shape(1, 1 << 25, 64, 4, 4), 0, 1 << 24)[0] == inv


def test_invalid_arguments_are_rejected_before_any_launch(race):
    from race_attention_kernel_amd import abi

    opts = abi.options(64, abi.RACE_KERNEL_VALU)
    bad = abi.shape(8, 1024, 4, 16, 300)
    assert abi.fwd(0, 0, 0, 0, None, bad, True, opts, None, 0, 0) == abi.RACE_ERROR_INVALID_VALUE
    good = abi.shape(8, 1024, 4, 16, 64)
    # Null inputs, misaligned pointers, missing workspace.
    assert abi.fwd(0, 0, 0, 0, None, good, True, opts, None, 0, 0) == abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd(16, 16, 16, 18, None, good, True, opts, 64, 1 << 30, 0) == abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd(16, 16, 16, 16, None, good, True, opts, None, 0, 0) == abi.RACE_ERROR_INVALID_VALUE
    assert abi.fwd(16, 16, 16, 16, None, good, True, opts, 64, 16, 0) == abi.RACE_ERROR_INVALID_VALUE
    # Bad kernel id.
    assert abi.fwd(16, 16, 16, 16, None, good, True, abi.options(64, 9), 64, 1 << 30, 0) == \
        abi.RACE_ERROR_INVALID_VALUE
    # The non-causal path has no MFMA kernel.
    assert abi.fwd(16, 16, 16, 16, None, good, False, abi.options(64, abi.RACE_KERNEL_MFMA), 64, 1 << 30,
                   0) == abi.RACE_ERROR_INVALID_VALUE
    # Backward needs the state and dOut.
    assert abi.noncausal_bwd(16, 16, 16, 0, 0, 16, 16, 16, good, opts, 64, 1 << 30, 0) == \
        abi.RACE_ERROR_INVALID_VALUE
    # Causal backward: dOut, aligned outputs and a large enough workspace; the
    # MFMA kernels only for S = d = 64.
    inv = abi.RACE_ERROR_INVALID_VALUE
    assert abi.causal_bwd(16, 16, 16, 0, 16, 16, 16, good, opts, 64, 1 << 30, 0) == inv
    assert abi.causal_bwd(16, 16, 16, 16, 16, 24, 16, good, opts, 64, 1 << 30, 0) == inv
    assert abi.causal_bwd(16, 16, 16, 16, 16, 16, 16, good, opts, 64, 64, 0) == inv
    no_mfma = abi.shape(8, 1024, 2, 8, 32)
    assert abi.causal_bwd(16, 16, 16, 16, 16, 16, 16, no_mfma, abi.options(64, abi.RACE_KERNEL_MFMA),
                          64, 1 << 30, 0) == inv
    assert abi.causal_bwd(16, 16, 16, 16, 16, 16, 16, good, abi.options(64, abi.RACE_KERNEL_MFMA_WG),
                          64, 1 << 30, 0) == inv
    # Nothing requested, or nothing to do: success without a launch.
    assert abi.causal_bwd(0, 0, 0, 0, None, None, None, good, opts, None, 0, 0) == 0
    assert abi.causal_bwd(0, 0, 0, 0, 16, 16, 16, abi.shape(8, 0, 4, 16, 64), opts, None, 0, 0) == 0


def test_carry_workspace_and_argument_checks(race):
    from race_attention_kernel_amd import abi

    inv = abi.RACE_ERROR_INVALID_VALUE
    # Decode calls (at most RACE_DECODE_TOKENS tokens, automatic choice, or the
    # decode kernel forced at any length) need no workspace.
    for T, opts in [(1, None), (abi.RACE_DECODE_TOKENS, None), (0, None),
                    (5000, abi.options(0, abi.RACE_KERNEL_DECODE))]:
        st, b = abi.fwd_carry_workspace_bytes(abi.shape(8, T, 4, 16, 64), opts)
        assert (st, b) == (0, 0), (T, st, b)
    # Longer calls use race_fwd's causal workspace for the same tile.
    sh = abi.shape(8, 4096, 4, 16, 64)
    opts = abi.options(512, abi.RACE_KERNEL_VALU)
    st, b = abi.fwd_carry_workspace_bytes(sh, opts)
    st2, b2, *_ = abi.fwd_workspace_bytes(sh, True, opts)
    assert st == st2 == 0 and b == b2 > 0
    assert abi.fwd_carry_workspace_bytes(sh, abi.options(100, abi.RACE_KERNEL_DECODE))[0] == inv
    assert abi.fwd_carry_workspace_bytes(abi.shape(8, 4, 4, 16, 300))[0] == inv
    one = abi.shape(8, 1, 4, 16, 64)
    # The carried state is required and 16-byte aligned; the advanced state
    # (when given) too; token pointers as in race_fwd.
    assert abi.fwd_carry(16, 16, 16, 16, 0, 16, one, None, None, 0, 0) == inv
    assert abi.fwd_carry(16, 16, 16, 16, 24, 16, one, None, None, 0, 0) == inv
    assert abi.fwd_carry(16, 16, 16, 16, 16, 24, one, None, None, 0, 0) == inv
    assert abi.fwd_carry(0, 16, 16, 16, 16, 16, one, None, None, 0, 0) == inv
    assert abi.fwd_carry(16, 16, 16, 18, 16, 16, one, None, None, 0, 0) == inv
    assert abi.fwd_carry(16, 16, 16, 16, 16, 16, one, abi.options(0, 9), None, 0, 0) == inv
    # The tile path wants its workspace.
    assert abi.fwd_carry(16, 16, 16, 16, 16, 16, sh, opts, None, 0, 0) == inv
    # race_fwd itself has no decode kernel.
    assert abi.fwd(16, 16, 16, 16, None, sh, True, abi.options(64, abi.RACE_KERNEL_DECODE), 64, 1 << 30,
                   0) == inv
    # Nothing to do: no streams, or no tokens and the state advanced in place.
    assert abi.fwd_carry(0, 0, 0, 0, 16, 16, abi.shape(0, 1, 4, 16, 64), None, None, 0, 0) == 0
    assert abi.fwd_carry(0, 0, 0, 0, 16, 16, abi.shape(8, 0, 4, 16, 64), None, None, 0, 0) == 0
    assert abi.fwd_carry(0, 0, 0, 0, 16, None, abi.shape(8, 0, 4, 16, 64), None, None, 0, 0) == 0


def test_torch_binding_validates_inputs_on_the_host(race, ext):
    import torch

    q, k, v = race.make_inputs(1, 64, 4, 16, 64)
    with pytest.raises(RuntimeError, match="race_fused_fwd: probsQ lives on the CPU"):
        ext.forward(q, k, v, True)
    with pytest.raises(ValueError):
        race.race_fused_fwd(q, k, v, True, kernel="tensor")
    assert ext.shape_supported(4, 16, 64)[0]
    assert not ext.shape_supported(4, 16, 256)[0]
    assert ext.abi_version() == 1
    with pytest.raises(RuntimeError):
        ext.select_tile_tokens(8, 1024, 4, 16, 64, False, True, 48, 0)
    del torch


def test_inputs_are_seeded_softmax_probabilities(race):
    import torch

    a = race.make_inputs(2, 33, 4, 16, 8, seed=3, grad_out=True)
    b = race.make_inputs(2, 33, 4, 16, 8, seed=3, grad_out=True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    q, k, v, g = a
    assert q.shape == (2, 33, 4, 16) and v.shape == (2, 33, 8) and g.shape == v.shape
    torch.testing.assert_close(q.sum(-1), torch.ones(2, 33, 4))
    assert (q > 0).all() and (k > 0).all()
    bq, _, _ = race.make_inputs(2, 33, 4, 16, 8, seed=3, dtype=torch.bfloat16)
    assert bq.dtype == torch.bfloat16 and torch.equal(bq, q.to(torch.bfloat16))


def test_configs_match_baseline(race):
    c = race.CONFIGS
    assert (c["cfg2_causal_fp32"].N, c["cfg2_causal_fp32"].S, c["cfg2_causal_fp32"].d) == (8, 64, 64)
    assert c["cfg4_noncausal_fp32"].N == 384 and not c["cfg4_noncausal_fp32"].causal
    assert (c["cfg5_causal_bf16_S256"].S, c["cfg5_causal_bf16_S256"].d) == (256, 128)


def test_product_path_never_imports_the_oracle():
    pkg = REPO / "race-attention-kernel_amd"
    for path in list(pkg.glob("*.py")) + list((pkg / "csrc").glob("*")):
        text = path.read_text(errors="ignore")
        hit = re.search(r"liboracle|race_oracle|oracle\.py|load_oracle|from oracle|import oracle", text)
        assert hit is None, f"{path.name} reaches the oracle: {hit.group(0)}"


# --- Algorithm 1 with the hashing inside (race_alg1_*) -------------------------------------

@pytest.mark.parametrize("D, P, L, ok", [(64, 4, 4, True), (128, 5, 4, True), (64, 1, 1, True),
                                         (96, 4, 4, False), (64, 6, 1, False), (64, 0, 1, False),
                                         (64, 4, 5, False), (64, 4, 0, False)])
def test_alg1_shape_limits(race, D, P, L, ok):
    from race_attention_kernel_amd import abi

    assert abi.alg1_shape_supported(abi.alg1_shape(8, 4096, D, P, L)) is ok


def test_alg1_lds_and_workspace_sizes(race):
    from race_attention_kernel_amd import abi

    sh = abi.alg1_shape(8, 5000, 64, 4, 4)
    for variant in (abi.RACE_ALG1_FP32, abi.RACE_ALG1_BF16):
        st, lds = abi.alg1_output_lds_bytes(sh, variant)
        assert st == 0 and 0 < lds <= 160 * 1024
    # The bf16-feature variant keeps single-term feature planes: less LDS.
    assert abi.alg1_output_lds_bytes(sh, abi.RACE_ALG1_BF16)[1] < abi.alg1_output_lds_bytes(sh, abi.RACE_ALG1_FP32)[1]
    # Every supported shape fits the MI355X's 160 KB of LDS per workgroup.
    for D in (64, 128):
        for P in range(1, 6):
            for L in range(1, 5):
                for variant in (0, 1):
                    st, lds = abi.alg1_output_lds_bytes(abi.alg1_shape(1, 1, D, P, L), variant)
                    assert st == 0 and lds <= 160 * 1024, (D, P, L, variant, lds)
    st, nbytes, tiles, rec = abi.alg1_workspace_bytes(sh, 0, 128)
    S = 4 * 16
    assert st == 0 and tiles == 40 and rec == -(-(S * 64 + S) // 64) * 64
    assert nbytes == 8 * tiles * rec * 4


@pytest.mark.parametrize("tile", [-64, 48, 100])
def test_alg1_invalid_tiles_and_variants(race, tile):
    from race_attention_kernel_amd import abi

    inv = abi.RACE_ERROR_INVALID_VALUE
    sh = abi.alg1_shape(8, 4096, 64, 4, 4)
    assert abi.alg1_workspace_bytes(sh, 0, tile)[0] == inv
    assert abi.alg1_workspace_bytes(sh, 2, 64)[0] == inv


def test_alg1_invalid_arguments_are_rejected_before_any_launch(race):
    from race_attention_kernel_amd import abi

    inv = abi.RACE_ERROR_INVALID_VALUE
    good = abi.alg1_shape(8, 1024, 64, 4, 4)
    bad = abi.alg1_shape(8, 1024, 96, 4, 4)
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 16, None, bad, 64, 0, 64, 1 << 30, 0) == inv
    # Null inputs, planes or beta; misaligned pointers; missing or short workspace.
    assert abi.alg1_fwd(0, 16, 16, 16, 16, 16, None, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 0, 16, 16, None, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 16, 0, 16, None, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 18, None, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 20, 16, 16, None, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 16, 20, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 16, None, good, 64, 0, None, 0, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 16, None, good, 64, 0, 64, 64, 0) == inv
    # Bad variant or tile.
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 16, None, good, 64, 3, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd(16, 16, 16, 16, 16, 16, None, good, 96, 0, 64, 1 << 30, 0) == inv
    # The continuation needs its carried state, 16-byte aligned.
    assert abi.alg1_fwd_carry(16, 16, 16, 16, 16, 16, 0, 16, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd_carry(16, 16, 16, 16, 16, 16, 24, 16, good, 64, 0, 64, 1 << 30, 0) == inv
    assert abi.alg1_fwd_carry(16, 16, 16, 16, 16, 16, 16, 16, bad, 64, 0, 64, 1 << 30, 0) == inv


def test_alg1_torch_binding_validates_inputs_on_the_host(race, ext):
    import torch

    q = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16)
    W = torch.zeros(2, 3, 64)
    with pytest.raises(RuntimeError, match="causal_v2.forward: q lives on the CPU"):
        race.causal_v2.forward(q, q, q, W, torch.tensor(1.0))
    with pytest.raises(RuntimeError, match="no Algorithm-1 kernel .* head_dim=96"):
        race.causal_v2.sub_chunk_tokens(96, 4)
    with pytest.raises(RuntimeError, match="num_planes=6"):
        race.causal_v2.output_pass_smem_bytes(64, 6, 1)
    assert race.causal_v2.sub_chunk_tokens(64, 4) == 64
    assert race.causal_v2.output_pass_smem_bytes(64, 4, 4) > 0
    assert race.causal_v2.precise_carry()


def test_hashed_forward_limits_and_workspace(race):
    # The hashed causal forward takes R = 2^K buckets, K >= 2, L*K <= 64,
    # S = L*2^K in {64, 128, 256} and d in {64, 128}; its workspace and tile
    # records are race_fwd's at the workgroup kernels' tile policy.
    from race_attention_kernel_amd import abi

    inv = abi.RACE_ERROR_INVALID_VALUE
    opts = abi.options(512, 0)
    st, nbytes, tiles, rec = abi.hashed_fwd_workspace_bytes(abi.shape(8, 65536, 4, 16, 64), 4, opts)
    assert st == 0 and tiles == 128 and rec == 4160 and nbytes == 8 * 128 * 4160 * 4
    want = abi.fwd_workspace_bytes(abi.shape(8, 65536, 4, 16, 64), True, abi.options(512, 3))
    assert (st, nbytes, tiles, rec) == want
    for L, R, K, d in [(8, 32, 5, 128), (2, 32, 5, 64), (16, 16, 4, 64), (8, 16, 4, 128), (16, 4, 2, 128),
                       (1, 256, 8, 64)]:
        assert abi.hashed_fwd_workspace_bytes(abi.shape(2, 100, L, R, d), K, opts)[0] == 0, (L, R, d)
    for L, R, K, d, why in [(4, 16, 3, 64, "R != 2^K"), (32, 2, 1, 64, "K = 1"), (4, 16, 4, 32, "d = 32"),
                            (2, 16, 4, 64, "S = 32"), (32, 4, 2, 64, "L*K = 64 but S = 128 ok?")]:
        st = abi.hashed_fwd_workspace_bytes(abi.shape(2, 100, L, R, d), K, opts)[0]
        if why.startswith("L*K = 64"):
            assert st == 0  # L = 32, K = 2: L*K = 64 and S = 128 are both in range
        else:
            assert st == inv, why
    # L*K past 64 (S = 256 at L = 64, K = 2).
    assert abi.hashed_fwd_workspace_bytes(abi.shape(2, 100, 64, 4, 128), 2, opts)[0] == inv
    # Only the matrix-core kernels hash.
    assert abi.hashed_fwd_workspace_bytes(abi.shape(2, 100, 4, 16, 64), 4,
                                          abi.options(512, abi.RACE_KERNEL_VALU))[0] == inv
    # Null or misaligned pointers are refused before any launch.
    sh = abi.shape(2, 100, 4, 16, 64)
    assert abi.hashed_fwd(0, 16, 16, 16, 16, None, sh, 4, opts, 16, 1 << 30, 0) == inv
    assert abi.hashed_fwd(16, 16, 16, 24, 16, None, sh, 4, opts, 16, 1 << 30, 0) == inv
    assert abi.hashed_fwd(16, 16, 16, 16, 16, None, sh, 4, opts, 16, 64, 0) == inv  # workspace
    # An empty sequence without a state asked for is a no-op.
    assert abi.hashed_fwd(0, 0, 0, 0, 0, None, abi.shape(2, 0, 4, 16, 64), 4, None, None, 0, 0) == 0


def test_hashed_binding_validates_inputs_on_the_host(race, ext):
    import torch

    x = torch.zeros(2, 64, 64)
    planes = torch.zeros(16, 64)
    with pytest.raises(RuntimeError, match="race_fused_fwd_hashed: K lives on the CPU"):
        ext.hashed_forward(x, x, x, planes, 4)
    assert ext.hashed_supported(4, 4, 64) and ext.hashed_supported(8, 5, 128)
    assert not ext.hashed_supported(4, 4, 32) and not ext.hashed_supported(8, 1, 64)
    assert race.hashed_supported(4, 4, 64)
