"""CPU emulation of the MFMA kernels' index math (no GPU).

Each mapping the kernels rely on is restated here from its definition in
race-attention-kernel_amd/csrc (the function or expression named in each
test) and checked the way the reference checks its own kernels' layouts
(src/causal_v2/tests/test_kernel_layout.py:96-201,317-441;
src/noncausal/tests/test_kernel_emulation.py:64-153): every mapping covers
its index space exactly once, composed mappings give the fragments the
comments promise, and the LDS accesses the comments call conflict-free touch
each bank once under the model of 64 banks of 4 bytes, a 16-lane group
served per pass.

Planted mistakes (a dropped or row-only swizzle, swapped lane roles of the
transposed read, reversed corner bits, a missing final flush, unpadded plane
rows) are shown to fail the same checks, so the checks are not vacuous.
"""
from __future__ import annotations

import itertools
import math
from collections import Counter

import numpy as np
import pytest

BANKS = 64
BANK_BYTES = 4


# ---------------------------------------------------------------------------
# mfma_common.h: fpos, Plane, OutTile


def fpos(k: int) -> int:
    """mfma_common.h fpos(): element k of an LDS operand row sits at fpos(k)."""
    return (k & ~31) | (((k >> 2) & 3) << 3) | (((k >> 4) & 1) << 2) | (k & 3)


def k_of(kk: int, g: int, e: int) -> int:
    """The permuted contraction index of step kk, lane group g, element e."""
    return 32 * kk + 4 * g + (e % 4) + 16 * (e // 4)


class Plane:
    """mfma_common.h Plane<kSplit, K>: bf16 rows of K elements (hi plane, then
    the lo plane at +2K bytes when split), chunk u of row r stored at
    u ^ sw(r), rows 32 bytes longer than the planes."""

    def __init__(self, split: bool, K: int, swizzle: bool = True, half_swap: bool = False):
        self.split, self.K = split, K
        self.lo_off = 2 * K
        self.pitch = (4 if split else 2) * K + 32
        self.mask = min(K // 8, 8) - 1
        self.swizzle = swizzle
        self.half_swap = half_swap

    def sw(self, row: int) -> int:
        return (((row >> 3) ^ ((row >> 2) & 1)) & self.mask) if self.swizzle else 0

    def hs(self, row: int) -> int:
        """Plane<..., kHalfSwap>::hs(): odd rows hold each chunk's halves swapped."""
        return (row & 1) if self.half_swap else 0

    def elem(self, row: int, k: int) -> int:   # put1
        p = fpos(k)
        return row * self.pitch + 16 * ((p >> 3) ^ self.sw(row)) + 2 * ((p & 7) ^ (self.hs(row) << 2))

    def off4(self, row: int, k0: int) -> int:  # put4 / off4
        p = fpos(k0)
        return row * self.pitch + 16 * ((p >> 3) ^ self.sw(row)) + 8 * (((p >> 2) & 1) ^ self.hs(row))

    def frag(self, row: int, kk: int, g: int) -> int:  # frag (the address; see frag_values)
        return row * self.pitch + 16 * ((4 * kk + g) ^ self.sw(row))

    def frag_values(self, mem: dict, row: int, kk: int, g: int, fix: bool = True) -> list:
        """The 8 values frag() hands lane (g, row): the 16 bytes at frag(), with
        the halves swapped back in registers for odd rows of a half-swapped
        plane (fix=False: a planted mistake that forgets the swap)."""
        a = self.frag(row, kk, g)
        vals = [mem[a + 2 * e] for e in range(8)]
        if self.half_swap and fix and (row & 1):
            vals = vals[4:] + vals[:4]
        return vals


class OutTile:
    """mfma_common.h OutTile<TIn, D, C>: [C][D] values, 16-byte chunk u of row
    r stored at u ^ swz(r), swz(r) = (r / rows per 256-byte span) & kMask.
    per_span=False gives the row-only swizzle swz(r) = r & kMask (a planted
    mistake below)."""

    def __init__(self, es: int, D: int, C: int, per_span: bool = True):
        self.es, self.D, self.C = es, D, C
        self.row_bytes = D * es
        self.chunks = self.row_bytes // 16
        self.mask = min(self.chunks, 16) - 1
        self.rows_per_span = (1 if self.row_bytes >= 256 else 256 // self.row_bytes) if per_span else 1

    def swz(self, row: int) -> int:
        return (row // self.rows_per_span) & self.mask

    def at(self, row: int, byte: int) -> int:
        return row * self.row_bytes + 16 * ((byte >> 4) ^ self.swz(row)) + (byte & 15)

    def chunk_at(self, q: int) -> int:
        row, u = divmod(q, self.chunks)
        return row * self.row_bytes + 16 * (u ^ self.swz(row))


def bank_load(accesses) -> Counter:
    """accesses: (byte offset, bytes) per lane -> dwords per bank."""
    c = Counter()
    for off, n in accesses:
        assert off % 4 == 0 and n % 4 == 0
        for j in range(n // 4):
            c[(off // BANK_BYTES + j) % BANKS] += 1
    return c


PLANE_KS = [32, 64, 128, 256]  # S, D (64..256) and the P tile's C (32, 64)


def test_fpos_permutes_each_32_block():
    for K in (32, 64, 128, 256):
        assert sorted(fpos(k) for k in range(K)) == list(range(K))
        assert all(fpos(k) // 32 == k // 32 for k in range(K))


def test_fragment_is_one_contiguous_run_and_two_accumulator_blocks():
    # Lane group g, step kk: its 8 permuted k land on 8 consecutive positions
    # (one 16-byte read), and they are exactly rows 4 g + r of two stacked
    # accumulator blocks (D[4 g + r][lr] of block b = element e = 4 b + r).
    for kk, g in itertools.product(range(4), range(4)):
        assert [fpos(k_of(kk, g, e)) for e in range(8)] == [32 * kk + 8 * g + e for e in range(8)]
        assert [k_of(kk, g, 4 * b + r) - 32 * kk for b in range(2) for r in range(4)] == \
               [16 * b + 4 * g + r for b in range(2) for r in range(4)]
    # Over the four lane groups a step covers its 32 k once.
    for kk in range(4):
        assert sorted(k_of(kk, g, e) for g in range(4) for e in range(8)) == list(range(32 * kk, 32 * kk + 32))


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", PLANE_KS)
def test_plane_places_every_element_once_inside_its_row(split, K):
    P = Plane(split, K)
    for row in range(64):
        offs = [P.elem(row, k) for k in range(K)]
        assert len(set(offs)) == K
        base = row * P.pitch
        assert min(offs) >= base and max(offs) + 2 <= base + 2 * K  # hi plane
        if split:  # the lo plane follows, inside the pitch
            assert max(offs) + P.lo_off + 2 <= base + P.pitch
        assert P.pitch >= (4 if split else 2) * K


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", PLANE_KS)
def test_plane_put4_and_frag_read_what_put1_stored(split, K):
    P = Plane(split, K)
    for row in range(48):
        for k0 in range(0, K, 4):  # put4: 4 consecutive elements, 8 contiguous bytes
            assert [P.off4(row, k0) + 2 * j for j in range(4)] == [P.elem(row, k0 + j) for j in range(4)]
        for kk, g in itertools.product(range(K // 32), range(4)):  # frag: the permuted 8
            assert [P.frag(row, kk, g) + 2 * e for e in range(8)] == \
                   [P.elem(row, k_of(kk, g, e)) for e in range(8)]


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", PLANE_KS)
def test_plane_fragment_reads_touch_each_bank_once(split, K):
    # frag(): 16 consecutive rows (lanes lr of a group), one 16-byte chunk.
    P = Plane(split, K)
    for r0, kk, g in itertools.product(range(0, 64, 16), range(K // 32), range(4)):
        load = bank_load((P.frag(r0 + lr, kk, g), 16) for lr in range(16))
        assert len(load) == BANKS and max(load.values()) == 1


def test_plane_without_swizzle_conflicts():
    # Planted mistake: without sw() the 16 rows of a fragment pile up.
    P = Plane(False, 64, swizzle=False)
    load = bank_load((P.frag(lr, 0, 0), 16) for lr in range(16))
    assert max(load.values()) > 1


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", [64, 128, 256])
def test_plane_staging_stores_spread_over_all_banks(split, K):
    # causal_geo.h KVStage::store: thread tid owns block (a, b) = divmod(tid,
    # K / E) of 4 rows x E columns and stores rows 4 a + rr, elements
    # b E + 4 h .. + 3 with put4 (8 bytes).  A wave's 64 stores (512 bytes)
    # load every bank exactly twice.
    E = 4 if split else 8  # elements per 16-byte global vector: fp32 / bf16
    P = Plane(split, K)
    for rr, h in itertools.product(range(4), range(E // 4)):
        load = bank_load((P.off4(4 * (t // (K // E)) + rr, (t % (K // E)) * E + 4 * h), 8) for t in range(64))
        assert len(load) == BANKS and max(load.values()) == 2


def ds_read_tr16_b64(mem: dict, addrs: list[int]) -> list[list]:
    """Emulation of ds_read_b64_tr_b16 for one 16-lane group: lane 4 r + q
    supplies the address of 4 bf16 values, forming row r, columns 4 q .. 4 q
    + 3 of a 4 x 16 block; lane i receives column i (rows 0..3)."""
    assert len(addrs) == 16
    M = [[None] * 16 for _ in range(4)]
    for lane, a in enumerate(addrs):
        r, q = divmod(lane, 4)
        for j in range(4):
            M[r][4 * q + j] = mem[a + 2 * j]
    return [[M[r][i] for r in range(4)] for i in range(16)]


def frag_tr(P: Plane, mem: dict, row0: int, col0: int, g: int) -> list[list]:
    """mfma_common.h Plane::frag_tr for lane group g: the 8 values of each
    lane lr (two transposed reads, rows r and r + 16, shuffled a ++ b)."""
    p0 = [P.off4(row0 + 4 * g + (lr >> 2), col0 + 4 * (lr & 3)) for lr in range(16)]
    p1 = [P.off4(row0 + 4 * g + (lr >> 2) + 16, col0 + 4 * (lr & 3)) for lr in range(16)]
    a, b = ds_read_tr16_b64(mem, p0), ds_read_tr16_b64(mem, p1)
    return [a[lr] + b[lr] for lr in range(16)]


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", PLANE_KS)
def test_frag_tr_hands_each_lane_its_transposed_fragment(split, K):
    # Lane (g, lr) gets elements (row0 + 4 g + e % 4 + 16 (e / 4), col0 + lr),
    # e = 0..7: the contraction runs over the plane's rows in the permuted
    # order, the lane's column is its lr.
    P = Plane(split, K)
    rows = 64
    mem = {P.elem(r, k) + o: (r, k) for r in range(rows) for k in range(K) for o in (0,)}
    for row0, col0, g in itertools.product(range(0, rows, 32), range(0, K, 16), range(4)):
        got = frag_tr(P, mem, row0, col0, g)
        for lr in range(16):
            assert got[lr] == [(row0 + 4 * g + e % 4 + 16 * (e // 4), col0 + lr) for e in range(8)]


def test_frag_tr_with_swapped_lane_roles_fails():
    # Planted mistake: lanes addressing column blocks by lr >> 2 and rows by
    # lr & 3 hand out a different fragment.
    P = Plane(False, 64)
    mem = {P.elem(r, k): (r, k) for r in range(64) for k in range(64)}
    p0 = [P.off4(4 * 0 + (lr & 3), 4 * (lr >> 2)) for lr in range(16)]
    got = ds_read_tr16_b64(mem, p0)
    assert any(got[lr] != [(e, lr) for e in range(4)] for lr in range(16))


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", PLANE_KS)
def test_frag_tr_reads_at_most_two_way(split, K):
    # The transposed reads (16 lanes x 8 bytes) put at most two dwords on a
    # bank: a 2-way conflict at worst, never the pile-up of an unswizzled tile.
    P = Plane(split, K)
    for row0, col0, g in itertools.product(range(0, 64, 32), range(0, K, 16), range(4)):
        load = bank_load((P.off4(row0 + 4 * g + (lr >> 2), col0 + 4 * (lr & 3)), 8) for lr in range(16))
        assert max(load.values()) <= 2


def max_ways(accesses) -> int:
    return max(bank_load(accesses).values())


def frag_tr_pass(P: Plane, row0: int, col0: int, half: int, second: int):
    """The 32 lanes of one pass of a transposed read (ds_read_b64_tr_b16: 8
    bytes per lane, 32 lanes served per pass): lane groups g = 2 half, 2 half
    + 1, rows row0 + second + 4 g + lr / 4."""
    return [(P.off4(row0 + second + 4 * g + (lr >> 2), col0 + 4 * (lr & 3)), 8)
            for g in (2 * half, 2 * half + 1) for lr in range(16)]


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("K", PLANE_KS)
def test_half_swapped_plane_hands_out_the_same_fragments(split, K):
    # put1/put4 store, frag (with the register swap) and frag_tr read back the
    # values of the plain plane: the layout change is invisible to the math.
    P = Plane(split, K, half_swap=True)
    rows = 64
    mem = {P.elem(r, k): (r, k) for r in range(rows) for k in range(K)}
    assert len(mem) == rows * K
    for r, k0 in itertools.product(range(rows), range(0, K, 4)):
        assert [mem[P.off4(r, k0) + 2 * j] for j in range(4)] == [(r, k) for k in range(k0, k0 + 4)]
    for r, kk, g in itertools.product(range(rows), range(K // 32), range(4)):
        assert P.frag_values(mem, r, kk, g) == [(r, k_of(kk, g, e)) for e in range(8)]
    for row0, col0, g in itertools.product(range(0, rows, 32), range(0, K, 16), range(4)):
        got = frag_tr(P, mem, row0, col0, g)
        for lr in range(16):
            assert got[lr] == [(row0 + 4 * g + e % 4 + 16 * (e // 4), col0 + lr) for e in range(8)]


def test_half_swapped_fragments_need_the_register_swap():
    # Planted mistake: reading a half-swapped plane's fragment without
    # swapping its halves back hands odd rows permuted contraction elements.
    P = Plane(False, 256, half_swap=True)
    mem = {P.elem(r, k): (r, k) for r in range(32) for k in range(256)}
    assert P.frag_values(mem, 1, 0, 0, fix=False) != [(1, k_of(0, 0, e)) for e in range(8)]
    assert P.frag_values(mem, 0, 0, 0, fix=False) == [(0, k_of(0, 0, e)) for e in range(8)]


def test_k_tile_transposed_reads_are_conflict_free_with_the_half_swap():
    # causal_geo.h Geo::PK for bf16 S = 256 (the cfg5 K tile): 32-lane passes
    # of the transposed reads touch each bank once with the half swap; the
    # plain plane puts every pass's 32 pieces on the 16 slots of one parity
    # (2-way), which is what the cfg5 counters measured.
    plain, swapped = Plane(False, 256), Plane(False, 256, half_swap=True)
    for row0, col0, half, second in itertools.product(range(0, 64, 32), range(0, 256, 16), range(2), (0, 16)):
        assert max_ways(frag_tr_pass(swapped, row0, col0, half, second)) == 1
        assert max_ways(frag_tr_pass(plain, row0, col0, half, second)) == 2


def test_k_tile_fragment_reads_stay_conflict_free_with_the_half_swap():
    # The 16-byte fragment reads (16-lane passes) keep their addresses.
    P = Plane(False, 256, half_swap=True)
    for base, kk, g in itertools.product(range(0, 64, 16), range(8), range(4)):
        assert max_ways((P.frag(base + lr, kk, g), 16) for lr in range(16)) == 1


def test_k_tile_staging_stores_are_no_worse_with_the_half_swap():
    # KVStage::store of bf16 rows (E = 8): a 32-lane pass writes one row, 32
    # 8-byte pieces; a 512-byte row covers every bank twice either way.
    plain, swapped = Plane(False, 256), Plane(False, 256, half_swap=True)
    for a, rr, h in itertools.product(range(8), range(4), range(2)):
        for P in (plain, swapped):
            assert max_ways((P.off4(4 * a + rr, 8 * b + 4 * h), 8) for b in range(32)) <= 2


@pytest.mark.parametrize("es, D, C", [(4, 64, 32), (4, 64, 64), (4, 128, 32), (4, 128, 64), (2, 64, 32),
                                      (2, 64, 64), (2, 128, 32), (2, 128, 64)])
def test_out_tile_swizzle_is_a_bijection_and_spreads(es, D, C):
    T = OutTile(es, D, C)
    n = C * T.row_bytes
    # Every byte of the tile exactly once; chunk_at is at() on chunk starts.
    assert sorted(T.at(r, b) for r in range(C) for b in range(T.row_bytes)) == list(range(n))
    assert [T.chunk_at(q) for q in range(C * T.chunks)] == \
           [T.at(q // T.chunks, 16 * (q % T.chunks)) for q in range(C * T.chunks)]
    # Accumulator-layout stores (mfma_causal.hip: OT::put(Os, 16 bi + lr,
    # 16 cb + 4 g, .)): a 16-lane group writes 4 values of 16 rows.
    vb = 4 * es
    for bi, cb, g in itertools.product(range(C // 16), range(D // 16), range(4)):
        load = bank_load((T.at(16 * bi + lr, (16 * cb + 4 * g) * es), vb) for lr in range(16))
        assert max(load.values()) == 1
    # Row-contiguous transfers: 16 consecutive threads move 16 consecutive chunks.
    for q0 in range(0, C * T.chunks, 16):
        load = bank_load((T.chunk_at(q), 16) for q in range(q0, q0 + 16))
        assert len(load) == BANKS and max(load.values()) == 1


def test_row_only_swizzle_conflicts_on_short_rows():
    # Planted mistake (swz(r) = r & kMask): bf16 rows of 64 values are half a
    # span, so rows r and r + 8 of an accumulator store share banks.
    T = OutTile(2, 64, 32, per_span=False)
    load = bank_load((T.at(lr, 0), 8) for lr in range(16))
    assert max(load.values()) == 2


def test_dq_tile_single_value_stores_spread():
    # mfma_bwd.hip T32::put1(D32s, 16 bi + 4 gq + rr, 16 w + lr, .): 4 rows x
    # 16 single fp32 values per wave and (bi, rr): 64 dwords, each bank once.
    T = OutTile(4, 64, 32)
    for bi, rr, w in itertools.product(range(2), range(4), range(4)):
        load = bank_load((T.at(16 * bi + 4 * gq + rr, 4 * (16 * w + lr)), 4) for gq in range(4) for lr in range(16))
        assert len(load) == BANKS and max(load.values()) == 1


# ---------------------------------------------------------------------------
# Tile and sub-chunk ownership; buffer ranges of the unconditional flush


def tile_rows(T: int, tile: int):
    tiles = -(-T // tile) if T else 0
    return [(ti, ti * tile, min(T, ti * tile + tile)) for ti in range(tiles)]


@pytest.mark.parametrize("T, tile", [(1, 32), (31, 32), (32, 32), (33, 32), (1000, 64), (4096, 512),
                                     (65536, 512), (70001, 16384), (0, 64)])
def test_tiles_cover_every_token_once(T, tile):
    # grid (tiles, N): workgroup (ti, n) owns rows [ti tile, min(T, ti tile + tile)).
    seen = Counter()
    for _, b, e in tile_rows(T, tile):
        assert e > b
        seen.update(range(b, e))
    assert sorted(seen) == list(range(T)) and all(v == 1 for v in seen.values())


@pytest.mark.parametrize("N, tiles", [(1, 1), (3, 5), (8, 128), (128, 7), (5, 1024)])
def test_direct_kernels_map_waves_to_tiles_once(N, tiles):
    # mfma_direct.hip direct_tile(): id = 4 blockIdx.x + w -> (n, ti); grid
    # (total + 3) / 4 blocks of 4 waves; ids past the total exit.
    total = N * tiles
    seen = Counter()
    for bx in range((total + 3) // 4):
        for w in range(4):
            i = 4 * bx + w
            if i >= total:
                continue
            n, ti = divmod(i, tiles)
            assert 0 <= n < N and 0 <= ti < tiles
            seen[(n, ti)] += 1
    assert len(seen) == total and set(seen.values()) == {1}


def quad_walk(rows: int, eighths: int = 6, C: int = 32):
    """mfma_direct.hip tile_sums_quad_kernel: per wave w, the rows of every
    sub-chunk it consumes, in order, with the policy of the load that fetched
    it ('alloc' or 'nt'), and the wave's refill offsets past the last round."""
    pairs = -(-rows // (2 * C))
    pcut = -(-(pairs * eighths) // 8)
    cut = 2 * C * pcut
    waves = []
    for w in range(4):
        p = pairs - 1 - w
        first = 2 * C * p if p >= 0 else rows
        pol = "alloc" if first < cut else "nt"
        held = [(first, pol), (first + C, pol)]   # k0/v0, k1/v1
        seq, tail = [], []
        while p >= 0:
            nx = 2 * C * (p - 4)
            npol = "nt" if p - 4 >= pcut else "alloc"
            for h in range(2):
                seq.append(held[h])
                held[h] = (nx + h * C, npol)
            p -= 4
        tail = [r for r, _ in held]
        waves.append((seq, tail))
    return pairs, pcut, waves


@pytest.mark.parametrize("rows", [1, 31, 32, 63, 64, 65, 200, 256, 300, 1000, 1024, 4096])
def test_quad_sums_consume_every_sub_chunk_once_end_first(rows):
    C = 32
    pairs, pcut, waves = quad_walk(rows)
    seen = Counter()
    for seq, _ in waves:
        seen.update(r for r, _ in seq)
    # Every sub-chunk start of the tile's pairs once (the second half of the
    # last pair may lie past the tile: it reads zeros and adds nothing).
    assert sorted(seen) == list(range(0, 2 * C * pairs, C)) and set(seen.values()) == {1}
    # Round j of the four waves covers the four pairs below round j - 1's.
    for j in range(max(len(seq) for seq, _ in waves) // 2):
        got = sorted(seq[2 * j][0] // (2 * C) for seq, _ in waves if len(seq) > 2 * j)
        want = [p for p in range(pairs - 1 - 4 * j - 3, pairs - 4 * j) if p >= 0]
        assert got == want
    # The pairs below the cut arrive through allocating loads, the rest `nt`.
    for seq, _ in waves:
        for r, pol in seq:
            assert pol == ("alloc" if r // (2 * C) < pcut else "nt")


@pytest.mark.parametrize("rows", [1, 64, 300, 1024])
def test_quad_sums_refills_past_the_walk_read_zero(rows):
    # The refill after a wave's last round starts below row 0: as a 32-bit
    # buffer offset it is past the range, so the loads return zeros.
    S, es = 64, 4
    _, _, waves = quad_walk(rows)
    for seq, tail in waves:
        for r0 in tail:
            if seq:
                assert r0 < 0
            for row in range(r0, r0 + 32):
                for c in range(0, S * es, 16):
                    off = (row * S * es + c) & 0xFFFFFFFF
                    assert off >= rows * S * es


def test_quad_sums_walk_with_a_wrong_round_stride_fails():
    # Planted mistake: rounds of 2 pairs instead of 4 visit pairs twice.
    rows, C = 1024, 32
    pairs = rows // (2 * C)
    seen = Counter()
    for w in range(4):
        seen.update(range(pairs - 1 - w, -1, -2))
    assert set(seen.values()) != {1}


@pytest.mark.parametrize("tiles, groups", [(1, 1), (7, 4), (128, 8), (1000, 16), (3, 8)])
def test_scan_groups_partition_the_tiles(tiles, groups):
    # valu_kernels.hip tile_scan_kernel: group gi scans tiles
    # [gi per, min(tiles, gi per + per)), per = ceil(tiles / groups).
    per = -(-tiles // groups)
    seen = Counter()
    for gi in range(groups):
        seen.update(range(gi * per, min(tiles, gi * per + per)))
    assert sorted(seen) == list(range(tiles)) and set(seen.values()) == {1}


def buffer_store_kept(offset: int, nbytes: int, num_records: int) -> bool:
    """A raw buffer store of nbytes at a 32-bit offset: written iff it lies in
    [0, num_records).  The offset is an unsigned 32-bit value, so a negative
    int offset is 2^32 + offset, far past any range below 2^31."""
    u = offset & 0xFFFFFFFF
    if u >= num_records:
        return False
    assert u + nbytes <= num_records, "a store straddling the range end"
    return True


def flushed_rows(rows: int, C: int, es: int, D: int):
    """Rows of a tile written by the output pass: the previous sub-chunk's
    tile is flushed at the top of every sub-chunk r0 = 0, C, ... (at r0 = 0,
    rows -C..-1) and once after the loop (mfma_causal.hip sub_chunk and its
    caller; hashed_kernels.h likewise).  OutTile::write stores chunk q of the
    [C][D] tile at r0 row_bytes + 16 q; the buffer covers the tile's rows."""
    T = OutTile(es, D, C)
    rng = rows * T.row_bytes
    assert rng < 2 ** 31  # race_api.hip tile_fits_buffer
    written = Counter()

    def flush(r0):
        for q in range(C * T.chunks):  # every chunk of the tile, over the threads
            off = r0 * T.row_bytes + 16 * q
            if buffer_store_kept(off, 16, rng):
                written[off // T.row_bytes] += 1

    r0 = 0
    while r0 < rows:
        flush(r0 - C)
        r0 += C
    if r0 > 0:
        flush(r0 - C)
    return written, T.chunks


@pytest.mark.parametrize("es, D, C", [(4, 64, 32), (2, 64, 32), (4, 128, 64), (2, 128, 32)])
@pytest.mark.parametrize("rows", [1, 15, 31, 32, 33, 63, 64, 100, 512])
def test_unconditional_flush_writes_each_row_once(es, D, C, rows):
    written, chunks = flushed_rows(rows, C, es, D)
    # Every row of the tile gets all its chunks once; nothing outside it.
    assert sorted(written) == list(range(rows))
    assert set(written.values()) == {chunks}


def test_flush_offsets_before_the_tile_are_dropped_for_every_range():
    # The first flush (r0 = -C) has offsets -C row_bytes .. -16: as unsigned
    # 32-bit values they are >= 2^32 - C row_bytes, beyond any range < 2^31.
    for es, D, C in [(4, 64, 32), (4, 128, 64), (2, 128, 32)]:
        row_bytes = D * es
        worst = (-C * row_bytes) & 0xFFFFFFFF
        assert worst >= 2 ** 31
        assert not buffer_store_kept(-16, 16, 2 ** 31 - 16)


def test_dq_flush_in_the_backward_writes_each_row_once():
    # mfma_bwd.hip flush(r0): fp32 dq32 chunks (OutTile<float, 64, 32>) and,
    # for bf16 tokens, 8-byte bf16 dQ chunks at r0 * 64 * 2 + 8 qi; called
    # with r0 - kBC at the top of every sub-chunk and once after the loop.
    kBC, kBS = 32, 64
    for rows in (1, 16, 31, 32, 33, 63, 64, 65, 1000):
        w32, w16 = Counter(), Counter()
        rng32, rng16 = rows * kBS * 4, rows * kBS * 2

        def flush(r0):
            for qi in range(kBC * kBS // 4):
                if buffer_store_kept(r0 * kBS * 4 + 16 * qi, 16, rng32):
                    w32[(r0 * kBS * 4 + 16 * qi) // (kBS * 4)] += 1
                if buffer_store_kept(r0 * kBS * 2 + 8 * qi, 8, rng16):
                    w16[(r0 * kBS * 2 + 8 * qi) // (kBS * 2)] += 1

        r0 = 0
        while r0 < rows:
            flush(r0 - kBC)
            r0 += kBC
        flush(r0 - kBC)
        assert sorted(w32) == list(range(rows)) and set(w32.values()) == {kBS // 4}
        assert sorted(w16) == list(range(rows)) and set(w16.values()) == {kBS // 4}


def test_missing_final_flush_loses_the_last_sub_chunk():
    # Planted mistake: without the flush after the loop the last sub-chunk's
    # rows are never written.
    rows, C, es, D = 100, 32, 4, 64
    T = OutTile(es, D, C)
    rng = rows * T.row_bytes
    written = set()
    for r0 in range(0, rows, C):
        for q in range(C * T.chunks):
            off = (r0 - C) * T.row_bytes + 16 * q
            if buffer_store_kept(off, 16, rng):
                written.add(off // T.row_bytes)
    assert written != set(range(rows))


def test_loads_past_the_tile_read_zero():
    # KVStage::load of the sub-chunk after the last (r0 = rows rounded up):
    # every 16-byte load at or past the range reads zero, none straddles.
    for es, S in [(4, 64), (2, 64), (4, 256)]:
        for rows in (1, 31, 32, 33, 500):
            rng = rows * S * es
            C = 32
            r_next = -(-rows // C) * C
            for row in range(r_next, r_next + C):
                for c in range(0, S * es, 16):
                    off = row * S * es + c
                    assert off >= rng  # past the range: the load returns zeros


# ---------------------------------------------------------------------------
# hash_stage.h: projection ownership, plane staging layouts, corner table


def projector_loads(D: int, es: int):
    """hash_stage.h Projector::load: (lane group g, load i) -> first element
    of the 16-byte run, 4 kPerVec i + kPerVec g."""
    per = 16 // es
    return {(g, i): 4 * per * i + per * g for g in range(4) for i in range(D * es // 4 // 16)}


@pytest.mark.parametrize("D", [32, 64, 128])
def test_projection_contracts_every_row_element_once(D):
    kSeg = D // 4
    # fp32: v_mfma_f32_16x16x4_f32; load i of group g holds elements
    # 16 i + 4 g .. + 3, element j the contraction index of step 4 i + j, and
    # the planes are read at the same column (Projector::project, get4).
    ld = projector_loads(D, 4)
    fp32 = Counter(ld[(g, s4 // 4)] + j for g in range(4) for s4 in range(0, kSeg, 4) for j in range(4))
    assert sorted(fp32) == list(range(D)) and set(fp32.values()) == {1}
    assert all(ld[(g, s4 // 4)] == 16 * (s4 // 4) + 4 * g for g in range(4) for s4 in range(0, kSeg, 4))
    # bf16: v_mfma_f32_16x16x32_bf16, step kk, group g: elements 32 kk + 8 g
    # .. + 7, one 16-byte load, the planes' terms read at c = 32 kk + 8 g.
    ld = projector_loads(D, 2)
    bf16 = Counter(ld[(g, kk)] + e for g in range(4) for kk in range(kSeg // 8) for e in range(8))
    assert sorted(bf16) == list(range(D)) and set(bf16.values()) == {1}
    assert all(ld[(g, kk)] == 32 * kk + 8 * g for g in range(4) for kk in range(kSeg // 8))


@pytest.mark.parametrize("D, es", [(64, 4), (128, 4), (64, 2), (128, 2)])
def test_projection_loads_are_contiguous_per_instruction(D, es):
    # One load instruction: the four lane groups of a row read one 64-byte
    # run (16 rows, one per lr), not pieces 64 bytes apart.
    ld = projector_loads(D, es)
    for i in range(D * es // 64):
        starts = sorted(ld[(g, i)] * es for g in range(4))
        assert starts == list(range(starts[0], starts[0] + 64, 16)) and starts[0] % 64 == 0


@pytest.mark.parametrize("D", [64, 128])
def test_plane_stagings_spread_a_column_of_rows(D):
    # PlanesLds: fp32 rows of D + 4 floats; get4 of 16 rows (lr) at one column
    # touches each bank once.  PlanesB3: bf16 rows of D + 8; get8 likewise.
    for c in range(0, D, 4):
        load = bank_load((((16 + lr) * (D + 4) + c) * 4, 16) for lr in range(16))
        assert len(load) == BANKS and max(load.values()) == 1
    for c in range(0, D, 8):
        load = bank_load((((16 + lr) * (D + 8) + c) * 2, 16) for lr in range(16))
        assert len(load) == BANKS and max(load.values()) == 1
    # Planted mistake: unpadded fp32 rows put all 16 rows on the same banks.
    load = bank_load(((lr * D) * 4, 16) for lr in range(16))
    assert max(load.values()) > 1


def plane_at(D: int, swz: bool, row: int, c: int) -> int:
    """hash_stage.h plane_at<D, kSwz>: float offset of plane row `row`,
    columns c .. c + 3 (c % 4 == 0)."""
    return row * D + 4 * ((c >> 2) ^ (row & 15)) if swz else row * (D + 4) + c


@pytest.mark.parametrize("D, NPB", [(64, 1), (64, 2), (128, 1), (128, 4)])
def test_swizzled_planes_place_each_chunk_once_and_spread(D, NPB):
    # PlanesLdsT<true> (the tile sums): rows of D floats, no padding; every
    # 16-byte chunk has one place inside its row, and get4 of the 16 rows of a
    # block (lr) at one column touches each bank once.
    places = Counter(plane_at(D, True, row, c) for row in range(16 * NPB) for c in range(0, D, 4))
    assert sorted(places) == list(range(0, 16 * NPB * D, 4)) and set(places.values()) == {1}
    for row in range(16 * NPB):
        assert all(row * D <= plane_at(D, True, row, c) < (row + 1) * D for c in range(0, D, 4))
    for pb, c in itertools.product(range(NPB), range(0, D, 4)):
        load = bank_load((plane_at(D, True, 16 * pb + lr, c) * 4, 16) for lr in range(16))
        assert len(load) == BANKS and max(load.values()) == 1
    # Planted mistake: swizzling by row % 4 only leaves 4-way conflicts.
    load = bank_load(((16 + lr) * D * 4 + 16 * (lr & 3), 16) for lr in range(16))
    assert max(load.values()) > 1


def sums_u_in_k(S: int, KP: int, split: bool) -> bool:
    """hashed_kernels.h sums_u_in_k: a wave's plane values live in its own 16
    rows of the K plane tile when one decode pass covers them (16 L <= 64)
    and a token's kUP floats fit one row's pitch."""
    L = S >> KP
    npb = (L * KP + 15) // 16
    return 16 * L <= 64 and (16 * npb + 1) * 4 <= Plane(split, S).pitch


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("S, KP", [(64, 2), (64, 3), (64, 4), (64, 5), (64, 6), (128, 4), (256, 4)])
def test_sums_plane_values_stay_in_their_waves_rows(split, S, KP):
    L = S >> KP
    if L < 1 or L * KP > 64:
        pytest.skip("not a hashed shape")
    npb = (L * KP + 15) // 16
    kup = 16 * npb + 1
    P = Plane(split, S)
    if not sums_u_in_k(S, KP, split):
        assert 16 * L > 64 or 4 * kup > P.pitch
        return
    # One pass over the (token, table) items: every value is read before the
    # wave writes any feature.
    assert (16 * L + 63) // 64 == 1
    spans = []
    for w in range(4):
        base = 16 * w * (P.pitch - 4 * kup)  # the kernel's U for wave w
        lo = base + (16 * w) * kup * 4
        hi = base + (16 * w + 15) * kup * 4 + 4 * kup
        # inside rows 16 w .. 16 w + 15 of the K tile, which only wave w writes
        assert 16 * w * P.pitch <= lo and hi <= (16 * w + 16) * P.pitch
        spans.append((lo, hi))
    assert all(spans[i][1] <= spans[i + 1][0] for i in range(3))


def test_four_workgroups_fit_the_s64_lds():
    # S = d = 64, fp32 rows: the tile sums (64-token sub-chunks: K and V plane
    # tiles, the plane values inside K, swizzled planes) and the lean output
    # pass (W, K, V plane tiles, P / plane values, padded planes) each fit
    # 40 KB, a quarter of gfx950's 160 KB.
    P = Plane(True, 64)
    sums = 2 * 64 * P.pitch + 16 * 64 * 4
    assert sums <= 40 * 1024
    u = 32 * 17 * 4
    p_tile = Plane(True, 32).pitch * 32
    out = 3 * 32 * P.pitch + max(p_tile, 2 * u) + 16 * (64 + 4) * 4
    assert out <= 40 * 1024
    # With padded planes the sums would not: the planted layout.
    assert 2 * 64 * P.pitch + 16 * 68 * 4 > 40 * 1024


@pytest.mark.parametrize("C, Wd, es, NT", [(32, 64, 4, 256), (64, 64, 4, 256), (32, 64, 2, 256),
                                           (32, 128, 4, 256), (64, 128, 2, 512), (32, 64, 4, 512)])
def test_row_stage_blocks_cover_the_sub_chunk_once(C, Wd, es, NT):
    # hashed_kernels.h RowStage: blocks of kRows rows x one 16-byte vector,
    # kRows the most (4, 2, 1) that still gives every thread a block.
    E = 16 // es
    vecs = C * (Wd // E)
    rows = 4 if vecs >= 4 * NT else 2 if vecs >= 2 * NT else 1
    blocks = (C // rows) * (Wd // E)
    per = -(-blocks // NT)
    seen = Counter()
    busy = set()
    for tid, p_ in itertools.product(range(NT), range(per)):
        blk = tid + p_ * NT
        if blk >= blocks:
            continue
        busy.add(tid)
        a, b = divmod(blk, Wd // E)
        for rr in range(rows):
            seen[(rows * a + rr, b)] += 1
    assert sorted(seen) == [(r, b) for r in range(C) for b in range(Wd // E)]
    assert set(seen.values()) == {1}
    if vecs >= NT:
        assert len(busy) == NT


@pytest.mark.parametrize("S, C, NW", [(64, 32, 4), (128, 32, 4), (256, 32, 8)])
def test_lean_query_features_are_converted_in_place_by_one_thread(S, C, NW):
    # Lean output pass: the hash writes Phi_Q's quad (row t, columns l R + 4 m
    # .. + 3) into the W plane's hi / lo slots; in the mass phase thread
    # (w, g, lr) reads rows 16 bi + lr, columns 16 sb + 4 g .. + 3 (sb = w +
    # NW sbw) and writes W there.  Every quad is handled by exactly one
    # thread, so the in-place conversion races with nobody.
    P = Plane(True, S)
    owner = Counter()
    for w, g, lr, bi in itertools.product(range(NW), range(4), range(16), range(C // 16)):
        for sbw in range(S // (16 * NW)):
            sb = w + NW * sbw
            owner[P.off4(16 * bi + lr, 16 * sb + 4 * g)] += 1
    written = {P.off4(t, k0) for t in range(C) for k0 in range(0, S, 4)}
    assert set(owner) == written and set(owner.values()) == {1}
    # The hi and lo 8-byte slots of a quad lie in its row, apart from every
    # other quad's.
    slots = Counter()
    for off in written:
        slots[off] += 1
        slots[off + P.lo_off] += 1
    assert set(slots.values()) == {1}


def sigma(x):
    return 1.0 / (1.0 + math.exp(-x))


def stored_plane_value(z: float) -> float:
    """hs_write_sigmas: copysign(sigma(-|z|), z)."""
    return math.copysign(sigma(-abs(z)), z)


def sigma_pair(s: float):
    """hs_sigma_pair: (sigma(z), sigma(-z)) from the stored value."""
    b = abs(s)
    a = 1.0 - b
    return (b, a) if math.copysign(1.0, s) < 0 else (a, b)


def corner_quads(u: list[float]) -> list[float]:
    """CornerTable<KP>::decode + quad(m) for m = 0 .. 2^(KP-2) - 1."""
    KP = len(u)
    sp = [sigma_pair(x) for x in u]
    s1, s2 = sp[KP - 2], sp[KP - 1]
    low = [s1[1] * s2[1], s1[1] * s2[0], s1[0] * s2[1], s1[0] * s2[0]]
    out = []
    for m in range(1 << (KP - 2)):
        base = 1.0
        for p in range(KP - 2):
            base *= sp[p][0] if (m >> (KP - 3 - p)) & 1 else sp[p][1]
        out += [base * x for x in low]
    return out


@pytest.mark.parametrize("K", [2, 3, 4, 5, 6])
def test_corner_table_follows_the_reference_corner_order(K):
    # probs[r] = softmax_r(sum_k s_rk u_k) with s_r the r-th element of
    # itertools.product([-1, 1], repeat=K) (src/race_baseline.py:30-32,41-44);
    # the kernels store z_k = 2 u_k and multiply sigmas.
    rng = np.random.default_rng(K)
    for _ in range(20):
        u = rng.normal(size=K) * 0.7
        z = 2 * u
        got = corner_quads([stored_plane_value(x) for x in z])
        signs = np.array(list(itertools.product([-1, 1], repeat=K)), float)
        logits = signs @ u
        want = np.exp(logits - logits.max())
        want /= want.sum()
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)


def test_corner_table_with_reversed_bits_fails():
    # Planted mistake: plane 0 as the least significant bit of r.
    u = [0.3, -1.1, 0.5]
    z = [2 * x for x in u]
    got = corner_quads([stored_plane_value(x) for x in z][::-1])
    signs = np.array(list(itertools.product([-1, 1], repeat=3)), float)
    want = np.exp(signs @ np.array(u))
    want /= want.sum()
    assert not np.allclose(got, want)


def test_sigma_pair_reads_the_sign_of_zero():
    # z = -0.0 stores -sigma(0) = -0.5; the pair is then (0.5, 0.5) either way,
    # and for z != 0 the order follows the sign.
    assert sigma_pair(stored_plane_value(-0.0)) == (0.5, 0.5)
    s = stored_plane_value(1.5)
    assert sigma_pair(s) == pytest.approx((sigma(1.5), sigma(-1.5)))
    s = stored_plane_value(-1.5)
    assert sigma_pair(s) == pytest.approx((sigma(-1.5), sigma(1.5)))


@pytest.mark.parametrize("NPB", [1, 2, 4])
def test_sigma_writes_cover_each_token_plane_once(NPB):
    # hs_write_sigmas: lane (g, lr) holds D[4 g + r][lr] = plane 16 pb + 4 g + r
    # of token lr and writes U[t pitch + 16 pb + 4 g + r].
    pitch = 16 * NPB + 1
    seen = Counter()
    for g, lr, pb, r in itertools.product(range(4), range(16), range(NPB), range(4)):
        seen[lr * pitch + 16 * pb + 4 * g + r] += 1
    assert len(seen) == 16 * 16 * NPB and set(seen.values()) == {1}
    assert max(seen) < 16 * pitch


# ---------------------------------------------------------------------------
# noncausal_v4.hip: the S = d = 64 backward passes (query_grad64_kernel,
# key_grad64_kernel).  Workgroup of 256 threads, stage of 64 rows of 64 fp32.

def row_slot(i: int, j: int) -> int:
    return j ^ (i & 3)


def db_at(s: int, c: int) -> int:
    """Float index of dB[s][c] in the key side's LDS tile."""
    return s * 64 + 4 * ((c >> 2) ^ ((s >> 2) & 15)) + (c & 3)


def groups16():
    """The 16-lane groups of a workgroup (tid ranges served per LDS pass)."""
    return [range(g, g + 16) for g in range(0, 256, 16)]


def max_bank_load(addr_bytes) -> int:
    """Worst bank load of one 16-lane group's 16-byte accesses (one address
    read by several lanes is one access)."""
    return max(bank_load((a, 16) for a in set(addr_bytes)).values())


def test_stage_rows_are_staged_once_and_read_back():
    # GradStage::stash: vector e = tid + 256 m holds row e / 16, slot e % 16.
    seen = Counter()
    for tid, m in itertools.product(range(256), range(4)):
        e = tid + 256 * m
        i, v = e >> 4, e & 15
        seen[i * 64 + 4 * row_slot(i, v)] += 1
    assert sorted(seen) == list(range(0, 64 * 64, 4)) and set(seen.values()) == {1}
    # Reading slot row_slot(i, j) of row i returns columns 4 j .. 4 j + 3.
    for i, j in itertools.product(range(64), range(16)):
        v = [v for v in range(16) if row_slot(i, v) == row_slot(i, j)]
        assert v == [j]


def test_stage_stores_are_conflict_free():
    for grp in groups16():
        for m in range(4):
            addrs = []
            for tid in grp:
                e = tid + 256 * m
                i, v = e >> 4, e & 15
                addrs.append(4 * (i * 64 + 4 * row_slot(i, v)))
            assert max_bank_load(addrs) == 1


def test_map_threads_cover_every_output_once():
    # Thread (tt, cc) = (tid / 16, tid % 16): rows tt + 16 r, columns 4 cc ...
    seen = Counter()
    for tid, r, c in itertools.product(range(256), range(4), range(4)):
        tt, cc = tid >> 4, tid & 15
        seen[(tt + 16 * r, 4 * cc + c)] += 1
    assert len(seen) == 64 * 64 and set(seen.values()) == {1}


def test_reduction_tokens_follow_the_outer64_order():
    # query_grad64_kernel: thread half h takes t = 32 (i / 16) + 16 h + i % 16;
    # outer64_kernel stages 32-token blocks and half h takes tokens 16 h .. of
    # each.  Same per-thread sequence, every token once per stage.
    for h in range(2):
        ours = [32 * (i >> 4) + 16 * h + (i & 15) for i in range(32)]
        outer64 = [32 * b + 16 * h + i for b in range(2) for i in range(16)]
        assert ours == outer64
    both = sorted(32 * (i >> 4) + 16 * h + (i & 15) for h in range(2) for i in range(32))
    assert both == list(range(64))


@pytest.mark.parametrize("j", range(16))
def test_operand_reads_are_conflict_free(j):
    # Map operands: Et rows (pitch 68) and the key side's dB, both reads.
    for grp in groups16():
        for k in range(4):
            et = [4 * ((4 * j + k) * 68 + 4 * (tid & 15)) for tid in grp]
            assert max_bank_load(et) == 1
            dv_b = [4 * (db_at(4 * j + k, 0) + 4 * ((tid & 15) ^ j)) for tid in grp]
            assert max_bank_load(dv_b) == 1
        for i in range(4):
            dk_b = [4 * ((4 * (tid & 15) + i) * 64 + 4 * (j ^ (tid & 15))) for tid in grp]
            assert max_bank_load(dk_b) == 1
        # Stage rows for the maps (one row per group) and the reduction's G row.
        for r in range(4):
            assert max_bank_load([4 * (((tid >> 4) + 16 * r) * 64 + 4 * row_slot(tid >> 4, j)) for tid in grp]) == 1
        t = 5
        assert max_bank_load([4 * (t * 64 + 4 * row_slot(t, tid & 15)) for tid in grp]) == 1


def test_db_tile_places_each_element_once_and_the_reads_find_it():
    assert sorted(db_at(s, c) for s in range(64) for c in range(64)) == list(range(64 * 64))
    for s, c in itertools.product(range(64), range(64)):
        j, cc, i = c >> 2, s >> 2, s & 3
        # dK read of row 4 cc + i at slot j ^ cc; dV read of row s at slot (c >> 2) ^ (s >> 2).
        assert db_at(s, c) == (4 * cc + i) * 64 + 4 * (j ^ cc) + (c & 3)
        assert db_at(s, c) == s * 64 + 4 * ((c >> 2) ^ (s >> 2)) + (c & 3)


def test_operand_tiles_without_their_layout_conflict():
    # Planted mistakes: an unswizzled dB (the dK read of 16 rows at one slot)
    # and E transposed at pitch 64 (the prologue's column writes).
    grp = range(16)
    assert max_bank_load([4 * ((4 * tid + 0) * 64 + 4 * 3) for tid in grp]) == 16
    assert max(bank_load((4 * (c * 64 + 7), 4) for c in grp).values()) == 16
    assert max(bank_load((4 * (c * 68 + 7), 4) for c in grp).values()) == 1


# ---------------------------------------------------------------------------
# mfma_bwd.hip causal_bwd_dq_mfma_kernel<TIn, kSums, DV>: the staging slots.
# Slot e = tid + 256 s counts K's blocks (4 tokens x E features of the 64
# bucket columns), then V's and G's (of DV value columns each); a wave's 64
# slots must name one tensor, and every block of every tensor is staged once.

def bwd_stage_slots(E: int, DV: int):
    C, S = 32, 64
    blk_k, blk_v = (C // 4) * (S // E), (C // 4) * (DV // E)
    slots = -(-(blk_k + 2 * blk_v) // 256)
    out = []
    for s in range(slots):
        for tid in range(256):
            e = tid + 256 * s
            e_wave = e - (tid & 63)
            tensor = 0 if e_wave < blk_k else 1 if e_wave < blk_k + blk_v else 2 if e_wave < blk_k + 2 * blk_v else 3
            if tensor == 3:
                continue
            blk = e if tensor == 0 else e - blk_k if tensor == 1 else e - blk_k - blk_v
            width = S if tensor == 0 else DV
            a, b = divmod(blk, width // E)
            out.append((s, tid, tensor, a, b))
    return out, blk_k, blk_v


@pytest.mark.parametrize("E, DV", [(8, 64), (8, 128), (4, 64)])
def test_bwd_staging_covers_every_block_once(E, DV):
    slots, blk_k, blk_v = bwd_stage_slots(E, DV)
    seen = Counter((tensor, a, b) for _, _, tensor, a, b in slots)
    want = {(0, a, b) for a in range(8) for b in range(64 // E)}
    want |= {(t, a, b) for t in (1, 2) for a in range(8) for b in range(DV // E)}
    assert set(seen) == want and set(seen.values()) == {1}
    # a wave stages one tensor (its buffer and stride are uniform)
    per_wave = {}
    for s, tid, tensor, _, _ in slots:
        per_wave.setdefault((s, tid >> 6), set()).add(tensor)
    assert all(len(t) == 1 for t in per_wave.values())
    assert blk_k % 64 == 0 and blk_v % 64 == 0


def test_bwd_staging_with_a_misplaced_boundary_fails():
    # Planted mistake: V's blocks counted from the wrong boundary (blk_v
    # instead of blk_k) would stage K's last blocks twice and miss some of G.
    E, DV = 8, 128
    slots, blk_k, blk_v = bwd_stage_slots(E, DV)
    wrong = Counter()
    for s, tid, tensor, _, _ in slots:
        e = tid + 256 * s
        blk = e if tensor == 0 else e - blk_v if tensor == 1 else e - 2 * blk_v
        if blk < 0:
            continue
        width = 64 if tensor == 0 else DV
        wrong[(tensor, *divmod(blk, width // E))] += 1
    want = {(0, a, b) for a in range(8) for b in range(8)} | {(t, a, b) for t in (1, 2) for a in range(8) for b in range(16)}
    assert set(wrong) != want


@pytest.mark.parametrize("N, tiles", [(1, 1), (128, 32), (3, 7)])
def test_wide_walk_record_arrays_do_not_overlap(N, tiles):
    # Records of value group h start at h N tiles rec (rec = 4160 floats);
    # the reverse scan takes both arrays as 2N streams of tiles records.
    rec = 4160
    spans = []
    for h in range(2):
        for n in range(N):
            for ti in range(tiles):
                start = (h * N * tiles + n * tiles + ti) * rec
                spans.append((start, start + 64 * 64 + 64))
    spans.sort()
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    assert spans[-1][1] <= 2 * N * tiles * rec
    # the scan's stream 2N-view: stream n' = h N + n holds exactly group h, stream n
    for h in range(2):
        for n in range(N):
            assert (h * N + n) * tiles * rec == (h * N * tiles + n * tiles) * rec


# ---------------------------------------------------------------------------
# mfma_bwd.hip: the block walks over 128 buckets x 128 value columns (bf16
# tokens, eight waves, 512 threads): causal_bwd_dq_wide_kernel and
# causal_bwd_dkv_wide_kernel.

WIDE_THREADS, WIDE_S, WIDE_D, WIDE_C = 512, 128, 128, 32


def wide_stage_blocks():
    """Staging of K, V, G: thread tid takes tensor tid / kBlk (kBlk = (32 / 4)
    (128 / 8) = 128 blocks per tensor) and block (sa, sb) = ((tid % 128) /
    16, tid % 16): rows 4 sa .. 4 sa + 3, columns 8 sb .. 8 sb + 7 (one
    16-byte bf16 load per row); threads 384..511 (tensor 3) stage nothing."""
    kblk = (WIDE_C // 4) * (128 // 8)
    cover = {t: Counter() for t in range(3)}
    for tid in range(WIDE_THREADS):
        tensor = tid // kblk
        if tensor >= 3:
            continue
        sa, sb = (tid % kblk) // 16, tid % 16
        for rr in range(4):
            for e in range(8):
                cover[tensor][(4 * sa + rr, 8 * sb + e)] += 1
    return kblk, cover


def test_wide_staging_covers_each_tile_once_one_tensor_per_wave():
    kblk, cover = wide_stage_blocks()
    assert kblk % 64 == 0  # a wave's 64 threads share one tensor
    for t in range(3):
        assert set(cover[t].values()) == {1}
        assert set(cover[t]) == {(r, c) for r in range(WIDE_C) for c in range(128)}


def test_wide_row_chunks_cover_the_sub_chunk_once():
    # Q, dQ's bf16 part and remainders (bf16 rows of 128: 16 chunks) take
    # chunk tid; the dV sum and the dV tile (fp32 rows of 128: 32 chunks)
    # chunks tid and tid + 512.  Chunk c is row c / chunks, elements
    # (c % chunks) * (16 / es) ...
    for es, per in ((2, 1), (4, 2)):
        chunks = WIDE_S * es // 16
        seen = Counter()
        for tid in range(WIDE_THREADS):
            for i in range(per):
                c = tid + i * WIDE_THREADS
                row, first = c // chunks, (c % chunks) * (16 // es)
                for e in range(16 // es):
                    seen[(row, first + e)] += 1
        assert set(seen.values()) == {1}
        assert set(seen) == {(r, k) for r in range(WIDE_C) for k in range(WIDE_S)}


def test_wide_records_map_every_block_entry_once():
    # causal_bwd_dkv_wide_kernel: wave w (group g2 = w >> 2, bucket sl = 16
    # (w & 3) + lr inside the group) loads zt[cb][rr] from record (g2, cb >> 2)
    # at sl * 64 + 16 (cb & 3) + 4 gq + rr; causal_bwd_dq_wide_kernel stores
    # its suffix totals to the same places.  Every entry of the four 64 x 64
    # records once; the lane's (bucket, column) in the block is (16 w + lr,
    # 16 cb + 4 gq + rr).
    seen = Counter()
    block = Counter()
    for w in range(8):
        g2 = w >> 2
        for lane in range(64):
            gq, lr = lane >> 4, lane & 15
            sl = 16 * (w & 3) + lr
            for cb in range(8):
                for rr in range(4):
                    seen[(g2, cb >> 2, sl * 64 + 16 * (cb & 3) + 4 * gq + rr)] += 1
                    block[(16 * w + lr, 16 * cb + 4 * gq + rr)] += 1
                    # The record entry is bucket 64 g2 + sl, column 64 (cb >> 2) + ..
                    assert 64 * g2 + sl == 16 * w + lr
    assert set(seen.values()) == {1} and len(seen) == 4 * 64 * 64
    assert set(block.values()) == {1} and len(block) == WIDE_S * WIDE_D


def wide_backward_flushes(rows: int):
    """causal_bwd_dkv_wide_kernel: the walk runs r0 = last, last - 32, ..., 0
    (last = ((rows - 1) / 32) 32); each sub-chunk first flushes the dK / dV
    tile of r0 + 32 (the one before in walk order) and a final flush writes
    r0 = 0.  Tile rows of 128 values: dK bf16 chunk c at ((r0 + c / 16) ld
    + 8 (c % 16)) 2 with ld = 256 (the full S), dV fp32 chunk c at (r0 128 +
    4 c) 4; the views cover the tile's rows."""
    ld = 256
    rng_k, rng_v = rows * ld * 2, rows * WIDE_D * 4
    wk, wv = Counter(), Counter()

    def flush(r0):
        for c in range(WIDE_C * 16):
            off = ((r0 + c // 16) * ld + 8 * (c % 16)) * 2
            if buffer_store_kept(off, 16, rng_k):
                wk[(off // 2) // ld] += 1
        for c in range(WIDE_C * 32):
            off = (r0 * WIDE_D + 4 * c) * 4
            if buffer_store_kept(off, 16, rng_v):
                wv[(off // 4) // WIDE_D] += 1

    last = ((rows - 1) // WIDE_C) * WIDE_C
    r0 = last
    while r0 >= 0:
        flush(r0 + WIDE_C)
        r0 -= WIDE_C
    flush(0)
    return wk, wv


@pytest.mark.parametrize("rows", [1, 31, 32, 33, 100, 4096])
def test_wide_backward_walk_flushes_each_row_once(rows):
    wk, wv = wide_backward_flushes(rows)
    assert sorted(wk) == list(range(rows)) and set(wk.values()) == {16}
    assert sorted(wv) == list(range(rows)) and set(wv.values()) == {32}


def test_wide_backward_walk_without_the_final_flush_loses_the_first_rows():
    # Planted mistake: the flush after the loop writes the walk's last
    # sub-chunk (rows 0..31); leaving it out loses them.
    rows = 100
    ld = 256
    rng = rows * ld * 2
    written = set()
    r0 = ((rows - 1) // WIDE_C) * WIDE_C
    while r0 >= 0:
        for c in range(WIDE_C * 16):
            off = ((r0 + WIDE_C + c // 16) * ld + 8 * (c % 16)) * 2
            if buffer_store_kept(off, 16, rng):
                written.add((off // 2) // ld)
        r0 -= WIDE_C
    assert not written & set(range(WIDE_C))


# ---------------------------------------------------------------------------
# race_internal.h wide_item(): one forward-walk launch over `pairs` 128-bucket
# blocks.  Workgroup x walks item (stream n, tile ti) of block b; the
# workgroups of one item read the same V and dOut rows and must sit
# kWideXcds = 8 apart (workgroup x runs on XCD x mod 8).

XCDS = 8


def wide_item(x: int, pairs: int, items: int):
    per = XCDS * pairs
    grp, inside = divmod(x, per)
    item = grp * XCDS + inside % XCDS
    return (item if item < items else -1), inside // XCDS


def wide_grid(pairs: int, items: int) -> int:
    """launch_causal_bwd_dq_wide: ceil(items / 8) groups of 8 pairs workgroups."""
    return -(-items // XCDS) * XCDS * pairs


@pytest.mark.parametrize("pairs", [1, 2])
@pytest.mark.parametrize("items", [1, 7, 8, 9, 512, 1000])
def test_wide_forward_walks_cover_every_item_and_block_once(pairs, items):
    seen = Counter()
    xcd = {}
    pad = 0
    for x in range(wide_grid(pairs, items)):
        item, b = wide_item(x, pairs, items)
        assert 0 <= b < pairs
        if item < 0:
            pad += 1
            continue
        seen[(item, b)] += 1
        xcd.setdefault(item, set()).add(x % XCDS)
    assert set(seen.values()) == {1} and len(seen) == items * pairs
    assert pad < XCDS * pairs
    # The workgroups of one item share an XCD, and within a block the items
    # keep launch order (item i before item i + 1).
    assert all(len(v) == 1 for v in xcd.values())
    for b in range(pairs):
        order = [wide_item(x, pairs, items)[0] for x in range(wide_grid(pairs, items))
                 if wide_item(x, pairs, items)[1] == b and wide_item(x, pairs, items)[0] >= 0]
        assert order == list(range(items))
    # One block: the identity mapping of the grid before the blocks shared a launch.
    if pairs == 1:
        assert all(wide_item(x, 1, items)[0] == x for x in range(items))


def test_wide_forward_walks_interleaved_blocks_split_an_item_over_xcds():
    # Planted mistake: block = x mod pairs (the blocks of an item adjacent in
    # launch order) covers every item and block once but puts the two
    # workgroups of an item on different XCDs.
    pairs, items = 2, 64
    xcd = {}
    for x in range(items * pairs):
        item, b = divmod(x, pairs)
        xcd.setdefault(item, set()).add(x % XCDS)
    assert any(len(v) > 1 for v in xcd.values())


# ---------------------------------------------------------------------------
# mfma_bwd.hip causal_bwd_dq_wide_kernel: the LDS regions each sub-chunk
# touches between its two barriers.  A barrier ends an epoch for every wave
# at once, so two waves may touch one region in the same epoch only if
# neither writes it (the writes of one epoch by different waves are disjoint
# chunks, which the staging tests above cover).


def dq_walk_epochs(subs: int, slots: int, tiles: int = 1, end_barrier: bool = True):
    """Per epoch: {(region, 'r'|'w', wave)} of the walk over `subs`
    sub-chunks with `slots` plane slots (regions: plane slot p, Qt, M,
    D32 = the dQ tile), for each of `tiles` tiles in turn (a whole-stream
    walk): the slot index restarts at each tile, whose walk ends with a
    barrier and the last flush."""
    epochs = [set()]

    def acc(region, kind, waves=range(8)):
        for w in waves:
            epochs[-1].add((region, kind, w))

    for _ in range(tiles):
        for t in range(subs):
            plane = f"plane{t % slots}"
            acc(plane, "w", range(6))   # staging: waves 0..5 (three tensors)
            acc("Qt", "w")
            epochs.append(set())         # first barrier
            acc("D32", "r")              # flush of sub-chunk t - 1
            acc("Qt", "r")               # step 1
            acc(plane, "r")              # step 1 (K), step 2 (V, G)
            acc("M", "w", range(3))      # step 2 on waves 0..2
            epochs.append(set())         # second barrier
            acc("M", "r")                # step 3
            acc(plane, "r")              # steps 3..5 (G, V)
            acc("D32", "w")              # step 3
        if end_barrier:
            epochs.append(set())         # barrier before the tile's last flush
        acc("D32", "r")
    return epochs


def epoch_conflicts(epochs):
    bad = []
    for e, ev in enumerate(epochs):
        for region in {r for r, _, _ in ev}:
            writers = {w for r, k, w in ev if r == region and k == "w"}
            users = {w for r, k, w in ev if r == region}
            if writers and len(users) > 1 and not all(k == "w" for r, k, _ in ev if r == region):
                bad.append((e, region))
    return bad


@pytest.mark.parametrize("subs", [1, 2, 3, 128])
def test_wide_forward_walk_two_slots_need_two_barriers(subs):
    assert epoch_conflicts(dq_walk_epochs(subs, 2)) == []


@pytest.mark.parametrize("subs", [1, 3, 128])
def test_whole_stream_walk_restarts_the_slots_at_each_tile(subs):
    # With pp.whole a workgroup walks tile after tile; each tile's sub-chunks
    # start again at slot 0, which an odd number of sub-chunks left last.
    assert epoch_conflicts(dq_walk_epochs(subs, 2, tiles=3)) == []


def test_whole_stream_walk_without_the_tile_end_barrier_races():
    # Planted mistake: no barrier at the tile end; with an odd number of
    # sub-chunks the next tile's staging writes slot 0 while slower waves
    # still read it, and its Q rows overwrite Qt.
    bad = {r for _, r in epoch_conflicts(dq_walk_epochs(3, 2, tiles=2, end_barrier=False))}
    assert "plane0" in bad


def test_wide_forward_walk_one_slot_without_the_top_barrier_races():
    # Planted mistake: one plane slot and no barrier before the staging
    # stores: sub-chunk t + 1's staging writes the slot while slower waves
    # still read it in steps 3..5 of sub-chunk t.
    assert ("plane0" in {r for _, r in epoch_conflicts(dq_walk_epochs(2, 1))})


# ---------------------------------------------------------------------------
# mfma_bwd.hip block walks: Q (and dQ's two bf16 parts) go from whole 16-byte
# row chunks into Plane<false, 128> (put_row_chunk: chunk tid is row tid / 16,
# buckets 8 (tid % 16) .. + 7, stored as two put4 of four), and step 1 reads
# them with frag_tr(row0 = 0, col0 = 16 w): lane (g, lr) of wave w needs the
# bucket 16 w + lr at rows 4 g + rr + 16 bi, element 4 bi + rr.


def put_row_chunks(P: Plane, two_halves: bool = True) -> dict:
    mem = {}
    for tid in range(512):
        row, k0 = divmod(tid, 16)
        k0 *= 8
        vals = [(row, k0 + j) for j in range(8)]
        if two_halves:
            for h in range(2):
                a = P.off4(row, k0 + 4 * h)
                for j in range(4):
                    assert a + 2 * j not in mem
                    mem[a + 2 * j] = vals[4 * h + j]
        else:  # planted: the chunk stored whole at its first four's place
            a = P.off4(row, k0)
            for j in range(8):
                mem[a + 2 * j] = vals[j]
    return mem


def test_row_chunks_in_a_plane_give_each_lane_its_bucket_at_accumulator_rows():
    P = Plane(False, 128)
    mem = put_row_chunks(P)
    assert len(mem) == 32 * 128
    for w, g in itertools.product(range(8), range(4)):
        got = frag_tr(P, mem, 0, 16 * w, g)
        for lr in range(16):
            assert got[lr] == [(4 * g + e % 4 + 16 * (e // 4), 16 * w + lr) for e in range(8)]


def test_row_chunks_stored_whole_give_the_wrong_buckets():
    # Planted mistake: a 16-byte chunk written at once in natural order; the
    # plane's fpos order puts elements 4..7 of the chunk elsewhere.
    P = Plane(False, 128)
    mem = put_row_chunks(P, two_halves=False)
    got = frag_tr(P, mem, 0, 0, 0)
    assert any(got[lr] != [(e % 4 + 16 * (e // 4), lr) for e in range(8)] for lr in range(16))


# ---------------------------------------------------------------------------
# mfma_common.h mfma16 (v_mfma_f32_16x16x32_bf16) as the kernels use it: lane
# (g, lr) supplies A[lr][k] and B[k][lr] for the 8 contraction indices
# k = k_of(0, g, e) (any order of the 32 indices, the same for both
# operands), and receives C[4 g + r][lr], r < 4.  The backward walk forms dK
# and dV transposed by swapping the operands of every product: then a lane
# holds four consecutive columns of one row.


def mfma16_emul(a_frag, b_frag):
    """a_frag[lane][e], b_frag[lane][e] (lane = 16 g + lr) -> c_frag[lane][r]."""
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    for lane in range(64):
        g, lr = divmod(lane, 16)
        for e in range(8):
            k = k_of(0, g, e)
            A[lr, k] = a_frag[lane][e]
            B[k, lr] = b_frag[lane][e]
    C = A @ B
    return [[C[4 * (lane // 16) + r, lane % 16] for r in range(4)] for lane in range(64)]


def test_swapped_operands_give_the_transposed_product_four_columns_per_lane():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((64, 8))
    b = rng.standard_normal((64, 8))
    c = mfma16_emul(a, b)
    ct = mfma16_emul(b, a)
    M = np.zeros((16, 16))
    Mt = np.zeros((16, 16))
    for lane in range(64):
        g, lr = divmod(lane, 16)
        for r in range(4):
            M[4 * g + r, lr] = c[lane][r]
            Mt[4 * g + r, lr] = ct[lane][r]
    assert np.allclose(Mt, M.T)
    # Lane (g, lr) of the swapped product holds row lr, columns 4 g .. 4 g + 3.
    for lane in range(64):
        g, lr = divmod(lane, 16)
        assert np.allclose(ct[lane], [M[lr, 4 * g + r] for r in range(4)])


def test_swapping_only_one_product_of_a_sum_mixes_layouts():
    # Planted mistake: a sum of two products with only one swapped is neither
    # the product nor its transpose.
    rng = np.random.default_rng(6)
    a, b, x, y = (rng.standard_normal((64, 8)) for _ in range(4))
    mixed = np.array(mfma16_emul(b, a)) + np.array(mfma16_emul(x, y))
    right = np.array(mfma16_emul(b, a)) + np.array(mfma16_emul(y, x))
    assert not np.allclose(mixed, right)
