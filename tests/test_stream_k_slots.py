"""The stream-K decode's partial-record protocol, checked on the CPU.

The decode kernel (csrc/paged_decode.hip, paged_decode_sk_kernel) cuts the flattened (row, tile) sequence into equal
contiguous ranges, one per workgroup ([k NT / G, (k + 1) NT / G), G = min(grid, max(min(NT, 8), ceil(NT / 4)))), and
with two waves per KV head splits each range at its midpoint.  A row's piece in a workgroup is written as the output
row when the workgroup holds the whole row, else as a partial record in one of the workgroup's two slots: slot 0 for
the piece opened at the range's first tile, slot 1 for the piece cut at the range's end.  With two halves the row
across the midpoint is merged in LDS first, and its merged piece follows the same rule.  The combine kernel
(paged_decode_sk_combine_kernel) finds a row's records from the prefix alone: workgroups kf .. kl holding its first
and last tile, slot 1 of kf when the row starts after kf's first tile (else slot 0), slot 0 of every later one.

This file models both sides of that contract over random ragged batches and grid sizes and checks that every record
the combine reads was written for that row, exactly once, that no record goes unread, and that every row held by one
workgroup is written whole exactly once.  It is a check of the protocol the two kernels implement, not of their
arithmetic (the GPU tests compare outputs with the oracle); a planted mistake in the merged piece's slot rule (the
first version's `prefix < lo` for a row starting exactly at the range's first tile) fails it.
"""
import numpy as np
import pytest


def _effective_grid(grid, nt):
    return min(grid, max(min(nt, 8), (nt + 3) // 4))


def _decode_writes(tiles, grid, halves, first_tile_rule="<="):
    """What the decode kernel writes: {(workgroup, slot): row} and {row: times written whole}."""
    B = len(tiles)
    pre = np.concatenate([[0], np.cumsum(tiles)]).astype(np.int64)
    NT = int(pre[-1])
    writes, outputs = {}, {}

    def row_of(t):  # the largest row with prefix[row] <= t (empty rows skipped)
        return min(int(np.searchsorted(pre, t, side="right") - 1), B - 1)

    def put(key, row):
        assert key not in writes, f"slot {key} written for rows {writes[key]} and {row}"
        writes[key] = row

    if NT == 0:
        return pre, NT, 0, writes, outputs
    ge = _effective_grid(grid, NT)
    for w in range(ge):
        lo_w, hi_w = w * NT // ge, (w + 1) * NT // ge
        mid = lo_w + (hi_w - lo_w) // 2 if halves == 2 else hi_w
        mid_row = -1
        if halves == 2 and lo_w < mid < hi_w:
            r = row_of(mid)
            mid_row = r if pre[r] < mid else -1
        pieces = {}
        for half in range(halves):
            lo, hi = (lo_w, mid) if half == 0 else (mid, hi_w)
            t = lo
            while t < hi:
                r = row_of(t)
                end = min(hi, int(pre[r + 1]))
                whole = t == pre[r] and end == pre[r + 1]
                if whole:
                    outputs[r] = outputs.get(r, 0) + 1
                elif mid_row >= 0 and ((half == 0 and end == mid) or (half == 1 and t == mid)):
                    pieces[half] = r
                else:
                    put((w, 0 if t == lo_w else 1), r)
                t = end
        if mid_row >= 0:
            assert pieces == {0: mid_row, 1: mid_row}, (w, pieces, mid_row)
            if pre[mid_row] >= lo_w and pre[mid_row + 1] <= hi_w:
                outputs[mid_row] = outputs.get(mid_row, 0) + 1
            else:
                from_lo = pre[mid_row] <= lo_w if first_tile_rule == "<=" else pre[mid_row] < lo_w
                put((w, 0 if from_lo else 1), mid_row)
        else:
            assert not pieces, (w, pieces)
    return pre, NT, ge, writes, outputs


def _check(tiles, grid, halves, first_tile_rule="<="):
    pre, NT, ge, writes, outputs = _decode_writes(tiles, grid, halves, first_tile_rule)
    read = set()
    for b in range(len(tiles)):
        p0, p1 = int(pre[b]), int(pre[b + 1])
        if p0 == p1:
            assert b not in outputs, f"empty row {b} written"
            continue
        kf = ((p0 + 1) * ge - 1) // NT
        kl = (p1 * ge - 1) // NT
        if kf == kl:
            assert outputs.get(b) == 1, f"row {b} held by workgroup {kf} not written whole once"
            continue
        assert b not in outputs, f"row {b} both written whole and merged"
        first_slot = 1 if kf * NT // ge < p0 else 0
        for i, k in enumerate(range(kf, kl + 1)):
            key = (k, first_slot if i == 0 else 0)
            assert writes.get(key) == b, f"row {b}: record {key} holds row {writes.get(key)}"
            read.add(key)
    assert read == set(writes), f"records nobody reads: {sorted(set(writes) - read)}"


def _batches(seed, n):
    rng = np.random.default_rng(seed)
    for trial in range(n):
        B = int(rng.integers(1, 80))
        kind = trial % 4
        if kind == 0:
            ctx = rng.integers(0, 1800, size=B)
        elif kind == 1:
            ctx = rng.integers(0, 64, size=B)
        elif kind == 2:
            ctx = np.where(rng.random(B) < 0.3, 0, rng.integers(1, 3000, size=B))
        else:
            ctx = rng.choice([0, 1, 16, 17, 32, 33, 2064], size=B)
        yield (ctx + 15) // 16


@pytest.mark.parametrize("halves", [1, 2])
def test_every_record_read_is_written_once(halves):
    for tiles in _batches(0, 600):
        for grid in (1, 2, 3, 7, 8, 16, 64, 256, 512):
            _check(tiles, grid, halves)


def test_576_row_workload_shape():
    rng = np.random.default_rng(1)
    ctx = np.exp(rng.uniform(np.log(64), np.log(1800), size=576)).astype(int)
    ctx[rng.random(576) < 0.1] = 0
    for halves, grid in ((2, 256), (1, 512)):
        _check((ctx + 15) // 16, grid, halves)


def test_planted_slot_rule_mistake_is_caught():
    """A row that starts exactly at the range's first tile and runs past its end must take slot 0; the rule
    `prefix < lo` sends it to slot 1, where the combine does not look."""
    failed = 0
    for tiles in _batches(3, 200):
        for grid in (8, 64, 256):
            try:
                _check(tiles, grid, 2, first_tile_rule="<")
            except AssertionError:
                failed += 1
    assert failed > 0


def _plan_positions(tiles, grid, halves, rec_cap, running_ob=True):
    """The per-frame plan's record placement (csrc/paged_decode.hip, paged_decode_plan_kernel): workgroup w's slot 0
    goes to the cut row holding its first tile (piece w - kf), slot 1 to the cut row holding its last tile when that
    row starts after the first tile (piece 0); piece j of the c-th cut row sits at 2c + j for j < 2, else at
    2 rec_cap + ob + j - 2 (ob: the overflow pieces of the cut rows before it).  Returns {(w, slot): position} and the
    descriptors [(row, pieces, ob)] in cut-row order."""
    B = len(tiles)
    pre = np.concatenate([[0], np.cumsum(tiles)]).astype(np.int64)
    NT = int(pre[-1])
    if NT == 0:
        return {}, []
    ge = _effective_grid(grid, NT)
    wg_of = lambda t: ((t + 1) * ge - 1) // NT
    desc, where = [], {}
    ob = 0
    for r in range(B):
        p0, p1 = int(pre[r]), int(pre[r + 1])
        if p1 > p0 and wg_of(p0) != wg_of(p1 - 1):
            n = wg_of(p1 - 1) - wg_of(p0) + 1
            where[r] = (len(desc), ob)
            desc.append((r, n, ob))
            ob += (n - 2) if running_ob else 0

    def row_of(t):
        return min(int(np.searchsorted(pre, t, side="right") - 1), B - 1)

    def pos(r, j):
        c, o = where[r]
        return 2 * c + j if j < 2 else 2 * rec_cap + o + j - 2

    out = {}
    for w in range(ge):
        lo_w, hi_w = w * NT // ge, (w + 1) * NT // ge
        r0 = row_of(lo_w)
        if r0 in where:
            out[(w, 0)] = pos(r0, w - wg_of(int(pre[r0])))
        r1 = row_of(hi_w - 1)
        if pre[r1] > lo_w and r1 in where:
            out[(w, 1)] = pos(r1, 0)
    return out, desc


@pytest.mark.parametrize("halves", [1, 2])
def test_plan_places_every_record_where_the_planned_combine_reads_it(halves):
    """Every record the decode writes has a plan position, no two records share one, every position lies inside the
    4 rec_cap slots, and the planned combine's reads (descriptor c: positions of pieces 0 .. n-1) hit exactly the
    records of that row, in the order the unplanned combine merges them."""
    for tiles in _batches(5, 400):
        for grid in (1, 2, 7, 8, 64, 256):
            _, NT, ge, writes, _ = _decode_writes(tiles, grid, halves)
            pos, desc = _plan_positions(tiles, grid, halves, rec_cap=grid)
            assert set(pos) == set(writes), (sorted(set(writes) ^ set(pos)))
            assert len(set(pos.values())) == len(pos)
            assert all(0 <= p < 4 * grid for p in pos.values())
            assert len(desc) <= max(ge - 1, 0)
            inv = {p: k for k, p in pos.items()}
            pre = np.concatenate([[0], np.cumsum(tiles)]).astype(np.int64)
            for c, (r, n, ob) in enumerate(desc):
                kf = ((int(pre[r]) + 1) * ge - 1) // NT
                first_slot = 1 if kf * NT // ge < pre[r] else 0
                for j in range(n):
                    p = 2 * c + j if j < 2 else 2 * grid + ob + j - 2
                    assert inv[p] == (kf + j, first_slot if j == 0 else 0), (r, j)
                    assert writes[inv[p]] == r


def test_planted_plan_position_mistake_is_caught():
    """Numbering every cut row's overflow pieces from 0 (no running base) makes two records share a position as soon
    as two rows are cut into three pieces or more."""
    clashes = 0
    for tiles in _batches(6, 200):
        for grid in (8, 64):
            pos, _ = _plan_positions(tiles, grid, 2, rec_cap=grid, running_ob=False)
            clashes += len(set(pos.values())) < len(pos)
    assert clashes > 0
