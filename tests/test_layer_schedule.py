"""Host-side model of the one-launch expert FFN's hand-off between its gate/up and down phases.

w4_layer_kernel (csrc/w4_verify.hip) runs gate/up, then down, in one grid.  Pass P belongs to
part P % 8; the workgroups running on XCD x claim the ranges of part x from two queues (gate/up
first, then down; the first claim of each queue at start, each later claim issued while the
previous range runs), publish per-pass counts of finished gate/up units after each gate/up
range, and a down range waits (per chunk of passes) until each of its passes is fully counted.
The last workgroup to finish clears every word.  This model restates that protocol -- the
split of a part's units into `chunks` contiguous ranges (verify_gemm), publish_ready's counts,
the chunked waits, the claims -- and runs it under random interleavings, uneven workgroup
counts per XCD and limited residency, checking:

- every range of every part is processed exactly once, by a workgroup of that part's XCD;
- every pass reaches exactly its target count, and a down chunk waits only on its own part's
  passes, inside that part's block of count words (ready_stride words: counts of at most
  ceil((T*k + T) / 8) passes, then the two queues);
- no interleaving deadlocks: whenever some workgroup is blocked, another can move, as long as
  each XCD runs at least one workgroup at a time;
- the pass descriptors fit the LDS capacity the layout reserves for them.

Planted mistakes (a split that drops a unit, a workgroup that takes a down range before its
last gate/up claim came back empty) must fail the model.
"""
import numpy as np
import pytest

XCDS = 8
GRID = 256


def passes_of(ids, experts, tokens, shared):
    """Pass count of a routing: per hit expert ceil(rows / 16), the shared expert ceil(T / 16)."""
    rows = np.bincount(ids.reshape(-1), minlength=experts)
    n = int(sum((r + 15) // 16 for r in rows if r))
    return n + ((tokens + 15) // 16 if shared else 0)


def split(total, rank, ranks):
    return total * rank // ranks, total * (rank + 1) // ranks


def local_passes(total_passes, part):
    return (total_passes - part + XCDS - 1) // XCDS if total_passes > part else 0


def stride_of(max_passes):
    local = (max_passes + XCDS - 1) // XCDS
    return (local + 2 + 31) // 32 * 32


class Launch:
    """The shared state of one launch: queues, counts, and what each range did."""

    def __init__(self, total_passes, strips_gu, strips_dn, chunk, max_passes, chunks, split_fn):
        self.total, self.sg, self.sd, self.chunk, self.chunks = total_passes, strips_gu, strips_dn, chunk, chunks
        self.split = split_fn
        self.stride = stride_of(max_passes)
        self.queue = {(x, ph): 0 for x in range(XCDS) for ph in (0, 1)}
        self.counts = {}
        self.done_ranges = []

    def word(self, part, j):
        assert 0 <= j < self.stride - 2, (part, j)     # the last two words are the queues
        return part * self.stride + j

    def claim(self, part, phase):
        c = self.queue[(part, phase)]
        self.queue[(part, phase)] = c + 1
        return c

    def gate_up(self, part, c):
        ub, ue = self.split(local_passes(self.total, part) * self.sg, c, self.chunks)
        self.done_ranges.append((part, 0, c))
        if ue > ub:
            for j in range(ub // self.sg, (ue - 1) // self.sg + 1):
                n = min(ue, (j + 1) * self.sg) - max(ub, j * self.sg)
                self.counts[self.word(part, j)] = self.counts.get(self.word(part, j), 0) + n

    def down_waits(self, part, c):
        """The words each chunk of down range c waits on, chunk by chunk."""
        ub, ue = self.split(local_passes(self.total, part) * self.sd, c, self.chunks)
        if ue <= ub:
            return []
        first, last = ub // self.sd, (ue - 1) // self.sd
        return [[self.word(part, j) for j in range(pc, min(last + 1, pc + self.chunk))]
                for pc in range(first, last + 1, self.chunk)]


def workgroup(launch, part, early_down=False):
    """One workgroup of XCD `part` as a generator: yields the word it waits on when blocked."""
    next_gu, next_dn = launch.claim(part, 0), launch.claim(part, 1)
    c = next_gu
    while c < launch.chunks and not early_down:
        next_gu = launch.claim(part, 0)
        yield None
        launch.gate_up(part, c)
        c = next_gu
    pending_gu = c if early_down else launch.chunks
    c = next_dn
    while c < launch.chunks:
        next_dn = launch.claim(part, 1)
        for words in launch.down_waits(part, c):
            for w in words:
                while launch.counts.get(w, 0) < launch.sg:
                    yield w
        launch.done_ranges.append((part, 1, c))
        c = next_dn
    while pending_gu < launch.chunks:                   # the planted mistake's gate/up, after down
        nxt = launch.claim(part, 0)
        launch.gate_up(part, pending_gu)
        pending_gu = nxt


def run(launch, per_xcd, resident, rng, early_down=False):
    """Random interleaving; at most `resident` workgroups per XCD run at once. Returns steps."""
    waiting = {x: list(range(per_xcd[x])) for x in range(XCDS)}
    active = []
    steps = 0
    while True:
        for x in range(XCDS):
            while waiting[x] and sum(1 for a in active if a[0] == x) < resident:
                waiting[x].pop()
                active.append((x, workgroup(launch, x, early_down and x == 0)))
        if not active:
            return steps
        i = int(rng.integers(len(active)))
        try:
            next(active[i][1])
            steps += 1
            if steps > 200000:
                raise RuntimeError("no progress: every resident workgroup waits")
        except StopIteration:
            active.pop(i)


def check(total, strips_gu, strips_dn, chunk, max_passes, per_xcd, resident, rng, split_fn=split,
          early_down=False):
    chunks = GRID // XCDS
    launch = Launch(total, strips_gu, strips_dn, chunk, max_passes, chunks, split_fn)
    run(launch, per_xcd, resident, rng, early_down)
    expected = {(p % XCDS) * launch.stride + p // XCDS for p in range(total)}
    assert set(launch.counts) == expected
    assert all(v == strips_gu for v in launch.counts.values())
    want = sorted((x, ph, c) for x in range(XCDS) for ph in (0, 1) for c in range(chunks))
    assert sorted(launch.done_ranges) == want


def _routing(rng, tokens, experts, k, skew):
    logits = rng.standard_normal((tokens, experts))
    if skew:
        logits[:, :k] += 4.0                            # every token on the same k experts
    return np.argsort(-logits, axis=1, kind="stable")[:, :k]


@pytest.mark.parametrize("hidden,inter", [(2048, 512), (2048, 1024), (512, 512)])
@pytest.mark.parametrize("skew", [False, True])
def test_every_range_done_once_and_every_wait_met(hidden, inter, skew):
    rng = np.random.default_rng(hidden + inter + skew)
    strips_gu, strips_dn = inter // 16, hidden // 32
    for tokens in (1, 7, 16, 32):
        for experts, k, shared in ((256, 8, True), (512, 4, False), (8, 8, True)):
            ids = _routing(rng, tokens, experts, k, skew)
            total = passes_of(ids, experts, tokens, shared)
            tpasses = (tokens + 15) // 16
            assert total <= min(experts, tokens * k) * tpasses + (tpasses if shared else 0)
            for chunk, per_xcd, resident in ((8, [32] * 8, 32), (3, [33, 31, 32, 32, 30, 34, 32, 32], 32),
                                             (1, [32] * 8, 2)):
                check(total, strips_gu, strips_dn, chunk, tokens * k + tokens, per_xcd, resident, rng)


def test_one_resident_workgroup_per_xcd_still_finishes():
    """Residency of one workgroup per XCD: it claims and runs every range of its part in order."""
    rng = np.random.default_rng(5)
    check(150, 32, 64, 8, 16 * 8 + 16, [32] * 8, 1, rng)


def test_model_catches_a_dropped_unit():
    """A range split that loses the last unit of the part leaves one pass short of its target."""
    def lossy(total, rank, ranks):
        ub, ue = split(total, rank, ranks)
        return ub, ue - 1 if rank == ranks - 1 and ue > ub else ue
    with pytest.raises((AssertionError, RuntimeError)):
        check(40, 32, 64, 8, 16 * 8 + 16, [32] * 8, 32, np.random.default_rng(1), split_fn=lossy)


def test_model_catches_down_before_gate_up():
    """A workgroup that keeps a gate/up range until after its down ranges can deadlock its XCD
    when it is the only one resident there: the model must report no progress."""
    with pytest.raises(RuntimeError):
        check(150, 32, 64, 8, 16 * 8 + 16, [32] * 8, 1, np.random.default_rng(2), early_down=True)
