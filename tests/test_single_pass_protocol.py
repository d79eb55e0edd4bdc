"""CPU emulation of the one-read causal forward's work protocol (single_pass.hip).

The kernel's correctness rests on index math and on a waiting protocol
between persistent workgroups: per-XCD tickets, tile workgroups that publish
a tile's totals (flag 1) before they wait for anything, four scanner parts
per stream that each add one to a tile's flag once their share of the
exclusive prefix is stored (whole at 1 + 4), and a lagged pipeline that
stages sub-chunk s while it runs the output of sub-chunk s - L from a ring of
R = L + 1 LDS slots.  These tests restate that protocol in Python and check,
on random interleavings and with workgroups that start late (fewer resident
than launched), that every run terminates, that each tile's output step sees
the prefix of the earlier tiles' totals in tile order, and that the ring
never hands a slot to phase 1 while phase 2 still reads it.  A planted
mistake (tiles dealt out by launch index instead of by ticket) must
deadlock when few workgroups are resident, which shows the emulation can
tell the difference.
"""
from __future__ import annotations

import random

import pytest

XCDS = 8
PARTS = 4           # scanner workgroups per stream
FLAG_TOTALS, FLAG_PREFIX = 1, 1 + PARTS
RECORD_CHUNKS = (64 * 64 + 64) // 4   # 16-byte chunks of an S = d = 64 record


def sp_tile(v: int, x: int, mshift: int) -> tuple[int, int]:
    """Job v on XCD x (2**mshift streams there) -> (stream, tile)."""
    return x + XCDS * (v & ((1 << mshift) - 1)), v >> mshift


def test_jobs_cover_every_tile_of_an_xcd_once():
    for N in (8, 16):
        for tiles in (1, 3, 512):
            seen = []
            for x in range(XCDS):
                m = (N - x + XCDS - 1) // XCDS
                mshift = 1 if m > 1 else 0
                seen += [sp_tile(v, x, mshift) for v in range(m * tiles)]
            assert sorted(seen) == [(n, i) for n in range(N) for i in range(tiles)]


def test_jobs_of_a_stream_come_in_tile_order():
    # Within a stream, a smaller tile index always has a smaller ticket: the
    # property the waiting protocol rests on.
    for mshift in (0, 1):
        order = {}
        for v in range(64):
            n, i = sp_tile(v, 3, mshift)
            order.setdefault(n, []).append(i)
        for tiles_in_order in order.values():
            assert tiles_in_order == sorted(tiles_in_order)


def test_scanner_parts_own_every_record_chunk_once():
    per = RECORD_CHUNKS // PARTS
    extra = per - 256
    owned = []
    for part in range(PARTS):
        for tid in range(256):
            owned.append(per * part + tid)
            if tid < extra:
                owned.append(per * part + 256 + (tid & (extra - 1)))
    assert sorted(owned) == list(range(RECORD_CHUNKS))


@pytest.mark.parametrize("nsub, R", [(4, 7), (4, 14), (2, 3), (4, 5)])
def test_slot_ring_never_overlaps_phase_one_and_phase_two(nsub, R):
    L = R - 1
    last_read = {}
    for s in range(200):
        write = s % R
        read = (s - L) % R if s >= L else None
        assert read != write
        # The slot written now was last read by phase 2 one step earlier
        # (a barrier apart), never later.
        if write in last_read:
            assert last_read[write] <= s - 1
        if read is not None:
            last_read[read] = s
            # and phase 2 reads what phase 1 staged L steps earlier
            assert (s - L) % R == read
    # Live tiles fit the 8-entry tile ring.
    assert (L + nsub - 1) // nsub + 2 <= 8


class Emulator:
    """One XCD's persistent workgroups stepping the kernel's protocol.

    Each workgroup is a generator that yields after every action, and yields
    "wait" while a condition it polls does not hold.  A random scheduler
    advances resident workgroups; launched workgroups become resident, in
    launch order, as residents finish (when `resident` is below the count).
    The XCD's streams are n = 8 j, j < m.  With static=True (the planted
    mistake) tile workgroups take jobs by launch index instead of tickets.
    """

    def __init__(self, m, tiles, workgroups, nsub, lag, rng, resident=None, static=False):
        self.m, self.tiles, self.nsub, self.lag = m, tiles, nsub, lag
        self.mshift = 1 if m > 1 else 0
        self.rng = rng
        self.ticket = 0
        self.flags = {}
        self.records = {}   # (n, i) -> per-part totals, then (in place) prefixes
        self.totals = {}    # (n, i) -> the tile's totals (for the check)
        self.prefix_seen = {}
        self.static = static
        self.workgroups = workgroups
        self.pending = [self.workgroup(w) for w in range(workgroups)]
        self.resident = []
        self.limit = resident if resident is not None else workgroups

    def take_ticket(self):
        t = self.ticket
        self.ticket += 1
        return t

    def scanner(self, n, part):
        running = 0
        pos = 0
        while pos < self.tiles:
            ready = 0
            while pos + ready < self.tiles and ready < 16 and self.flags.get((n, pos + ready), 0) >= FLAG_TOTALS:
                ready += 1
            if ready == 0:
                yield "wait"
                continue
            for j in range(ready):
                key = (n, pos + j)
                total = self.records[key][part]
                self.records[key][part] = running
                running += total
                yield "step"
            for j in range(ready):
                self.flags[(n, pos + j)] += 1
            pos += ready

    def workgroup(self, launch):
        scanners = self.m * PARTS
        first = launch if self.static else self.take_ticket()
        yield "step"
        if first < scanners:
            yield from self.scanner(XCDS * (first // PARTS), first % PARTS)
            return
        jobs = self.m * self.tiles
        stride = self.workgroups - scanners

        def next_job(k):
            if self.static:
                return first - scanners + k * stride
            return self.take_ticket() - scanners

        ring = {0: first - scanners}
        kmax = 0 if ring[0] >= jobs else 1 << 30
        pending_flag = None
        ticket_job = None
        s = 0
        while True:
            k1, j1 = divmod(s, self.nsub)
            s2 = s - self.lag
            k2, j2 = divmod(s2, self.nsub) if s2 >= 0 else (-1, 0)
            p1 = k1 < kmax
            p2 = s2 >= 0 and k2 < kmax
            if s2 >= 0 and k2 >= kmax:
                return
            if pending_flag is not None:      # release: totals stored last step
                self.flags[pending_flag] = FLAG_TOTALS
                pending_flag = None
            if p2 and j2 == 0:                # phase 2's prefix
                key = sp_tile(ring[k2], 0, self.mshift)
                while self.flags.get(key, 0) < FLAG_PREFIX:
                    yield "wait"
                self.prefix_seen[key] = tuple(self.records[key])
            if p1 and j1 == self.nsub - 1:
                ring[k1 + 1] = ticket_job if ticket_job < jobs else -1
            if p1 and j1 == self.nsub - 2:
                ticket_job = next_job(k1 + 1)
            yield "step"
            if p1 and j1 == self.nsub - 1 and ring[k1 + 1] < 0:
                kmax = k1 + 1
            if p1 and j1 == self.nsub - 1:    # phase 1: the tile's totals
                key = sp_tile(ring[k1], 0, self.mshift)
                total = self.rng.randrange(1, 1000)
                self.totals[key] = total
                self.records[key] = [total * (p + 1) for p in range(PARTS)]
                pending_flag = key
            s += 1
            yield "step"

    def run(self, budget=200000):
        steps = 0
        while self.pending or self.resident:
            while self.pending and len(self.resident) < self.limit:
                self.resident.append(self.pending.pop(0))
            g = self.rng.choice(self.resident)
            try:
                next(g)
            except StopIteration:
                self.resident.remove(g)
            steps += 1
            if steps > budget:
                return False
        return True


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("m, tiles", [(1, 1), (1, 7), (1, 40), (2, 1), (2, 23)])
def test_protocol_terminates_with_fixed_order_prefixes(seed, m, tiles):
    rng = random.Random(seed * 1000 + m * 100 + tiles)
    workgroups = rng.choice([m * PARTS + 1, m * PARTS + 3, 32])
    resident = rng.choice([None, m * PARTS + 1, m * PARTS + 2])
    em = Emulator(m, tiles, workgroups, nsub=4, lag=6, rng=rng, resident=resident)
    assert em.run(), "the protocol did not finish"
    for j in range(m):
        running = 0
        for i in range(tiles):
            key = (XCDS * j, i)
            assert em.prefix_seen[key] == tuple(running * (p + 1) for p in range(PARTS))
            running += em.totals[key]


def test_static_tile_assignment_deadlocks_when_few_are_resident():
    # The planted mistake: tiles dealt out by launch index instead of by
    # ticket.  A resident workgroup then waits for totals owned by one that
    # is not resident yet and cannot start until a resident one finishes.
    stuck = 0
    for seed in range(10):
        rng = random.Random(seed)
        em = Emulator(1, 24, workgroups=PARTS + 6, nsub=4, lag=6, rng=rng, resident=PARTS + 2,
                      static=True)
        stuck += not em.run(budget=50000)
    assert stuck == 10
    # The same shape with tickets finishes.
    em = Emulator(1, 24, workgroups=PARTS + 6, nsub=4, lag=6, rng=random.Random(0), resident=PARTS + 2)
    assert em.run()
