"""CPU: the bookkeeping of the split-K down GEMM (no GPU).

The verify gate/up launch splits the unit list (passes x strips of 16 h columns) into one
contiguous range per workgroup, ``[floor(U b / G), floor(U (b + 1) / G))``; each workgroup
writes one partial y row per pass row of every pass its range touches, at row
``rps * (b + P) + r``, and the routing writes per slot row the partial rows the combine adds
(``part_rows`` in ``w4_verify.hip``: first row ``rps * (b0 + P) + r``, count ``b1 - b0 + 1``,
b0 / b1 the workgroups of the pass's first and last units).  This model replays both sides
for many unit counts and grids and checks that every row the combine reads was written in
that launch (including by workgroups whose range is empty), that no two (workgroup, pass)
pairs share a row, that the rows read for a pass are exactly its workgroups', and that the
host's admission test keeps every range within two passes.  Planted mistakes (no zero rows
from empty ranges, a last workgroup off by one) fail it.
"""
import itertools
import random

import pytest


def ranges(U, G):
    return [(U * b // G, U * (b + 1) // G) for b in range(G)]


def written_rows(U, S, G, rows, rps, zero_empty=True):
    """Rows each workgroup writes: {row: (b, P)}; also the largest number of passes a range spans."""
    out, span = {}, 0
    for b, (ub, ue) in enumerate(ranges(U, G)):
        if ue > ub:
            p0, p1 = ub // S, (ue - 1) // S
            span = max(span, p1 - p0 + 1)
            pairs = [(b, p) for p in range(p0, p1 + 1)]
        else:
            p = ub // S
            pairs = [(b, p)] if zero_empty and ub < U and ub != p * S else []
        for bb, p in pairs:
            for r in range(rows[p]):
                row = rps * (bb + p) + r
                assert row not in out, (row, out[row], (bb, p))
                out[row] = (bb, p)
    return out, span


def read_rows(U, S, G, rows, rps, last_off=0):
    """Per (pass, row): the partial rows the combine adds (the routing's row_seg)."""
    got = {}
    for p, n in enumerate(rows):
        b0 = (G * (p * S + 1) - 1) // U
        b1 = (G * (p + 1) * S - 1) // U + last_off
        for r in range(n):
            got[(p, r)] = [rps * (b + p) + r for b in range(b0, b1 + 1)]
    return got


def check(U, S, G, rows, rps, **plant):
    written, span = written_rows(U, S, G, rows, rps, plant.get("zero_empty", True))
    reads = read_rows(U, S, G, rows, rps, plant.get("last_off", 0))
    owners = {}
    for b, (ub, ue) in enumerate(ranges(U, G)):
        for x in range(ub, ue):
            owners.setdefault(x // S, set()).add(b)
    for (p, r), rws in reads.items():
        for row in rws:
            if row not in written or written[row][1] != p:
                return False, span
        # every workgroup with units of the pass is among those read
        read_b = {written[row][0] for row in rws}
        if not owners[p] <= read_b:
            return False, span
    return True, span


def _pass_rows(rng, tokens, experts, k, shared):
    counts = [0] * experts
    for _ in range(tokens):
        for e in rng.sample(range(experts), k):
            counts[e] += 1
    rows = [min(16, c - 16 * i) for c in counts if c for i in range((c + 15) // 16)]
    if shared:
        rows += [min(16, tokens - 16 * i) for i in range((tokens + 15) // 16)]
    return rows


@pytest.mark.parametrize("tokens,experts,k,strips,grid", [
    (16, 256, 8, 32, 256), (1, 256, 8, 32, 256), (1, 8, 2, 32, 256), (5, 64, 4, 64, 256),
    (24, 16, 4, 32, 256), (16, 32, 2, 32, 256), (16, 256, 8, 32, 304), (3, 4, 1, 32, 80),
    (32, 64, 8, 32, 256), (7, 128, 4, 32, 1024),
])
def test_every_partial_row_read_was_written(tokens, experts, k, strips, grid):
    rng = random.Random(tokens * 1000 + experts + grid)
    for _ in range(20):
        rows = _pass_rows(rng, tokens, experts, k, shared=True)
        ok, _ = check(len(rows) * strips, strips, grid, rows, min(16, tokens))
        assert ok


def test_admission_keeps_ranges_within_two_passes():
    """The host admits a shape when ceil(cap S / G) <= S + 1 (cap: the most passes a routing can
    make); then no routing gives a range that spans three passes."""
    for strips, grid, cap in itertools.product((32, 64), (80, 256, 304), range(1, 400, 7)):
        if -(-cap * strips // grid) > strips + 1:
            continue
        for passes in range(1, cap + 1):
            rows = [1] * passes
            _, span = written_rows(passes * strips, strips, grid, rows, 1)
            assert span <= 2, (strips, grid, cap, passes)


def test_planted_mistakes_fail_the_model():
    rows = [1, 1, 1]                            # T=1, k=2 + shared: 96 units on 256 workgroups
    assert check(96, 32, 256, rows, 1)[0]
    assert not check(96, 32, 256, rows, 1, zero_empty=False)[0]
    rows = [16, 3, 16, 16]
    assert check(128 * 4, 128, 256, rows, 16)[0]
    assert not check(128 * 4, 128, 256, rows, 16, last_off=1)[0]
