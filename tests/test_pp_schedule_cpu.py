"""Host model of the LDS slot schedules of the two ping-pong backward kernels
(``dkdv_pp_kernel`` and ``dq_pp_kernel`` in ``csrc/fa_bwd.hpp``).

Both run 8 waves in two groups: group 0 does M(r) (matrix products) between
barriers 2r and 2r+1 and V(r) between 2r+1 and 2r+2; group 1 runs one phase
behind (M(r) in interval 2r+1, V(r) in 2r+2).  A wave issues its share of a
tile's global -> LDS copies in a V phase, and at the end of each V phase waits
until only the copies of its last W rounds are in flight (vector loads complete
in issue order); the barrier after that V phase publishes the landed tiles.

For every run length the model checks that
* a copy lands and is published before the first phase that reads its tile,
* a slot is refilled only after every phase that reads the tile it held, and
* every tile past the prologue's is copied by both groups (both halves for
  dK/dV).
Mutated schedules (copies issued further ahead, one slot fewer, copies waited
for a round later, a tile never copied) must fail, which shows the model can
tell."""
import pytest


def _check(reads, copies, n_tiles, n_slots, wait_rounds, prologue, halves):
    for j, g, half, iv in copies:
        land = iv + 2 * wait_rounds  # waited at the end of V(r + W), published after it
        if j in reads and not land < min(reads[j]):
            return f"tile {j} (group {g}) lands in interval {land}, read from {min(reads[j])}"
        if j - n_slots >= 0 and not max(reads[j - n_slots]) < iv:
            return f"tile {j} (group {g}) overwrites tile {j - n_slots}, read until {max(reads[j - n_slots])}"
    if prologue > n_slots:
        return "prologue tiles exceed the slots"
    for j in range(prologue, n_tiles):
        got = sorted((g, h) for jj, g, h, _ in copies if jj == j)
        want = sorted((g, h) for g in (0, 1) for h in halves)
        if got != want:
            return f"tile {j} copied by {got}"
    return None


def dkdv_pp_schedule(total, n_slots=3, offset=3, wait_rounds=1, prologue=2):
    """Round r handles 32-query sub-step r of tile r >> 1 (2 rounds a tile).
    M(r): S/dP of sub-step r (Q, dO rows), dV/dK of sub-step r-1 (transposed
    rows); V(r): LSE / delta of sub-step r.  V(r) of group g copies half
    (m & 1) of tile m >> 1, m = r + offset + g."""
    reads, copies = {}, []
    for g in (0, 1):
        for r in range(0, 2 * total + 1):
            im, iv = 2 * r + g, 2 * r + 1 + g
            if r < 2 * total:
                reads.setdefault(r >> 1, []).extend([im, iv])
            if r >= 1:
                reads.setdefault((r - 1) >> 1, []).append(im)
            m = r + offset + g
            if prologue <= (m >> 1) < total:
                copies.append((m >> 1, g, m & 1, iv))
    return _check(reads, copies, total, n_slots, wait_rounds, prologue, (0, 1))


def dq_pp_schedule(n_tiles, n_slots=4, offset=2, wait_rounds=1, prologue=3):
    """Round r handles 64-key tile r.  M(r): dQ products of tile r-1 (K),
    S/dP of tile r (K, V).  V(r) of group g copies tile r + offset + g."""
    reads, copies = {}, []
    for g in (0, 1):
        for r in range(0, n_tiles + 1):
            im, iv = 2 * r + g, 2 * r + 1 + g
            if r < n_tiles:
                reads.setdefault(r, []).append(im)
            if r >= 1:
                reads.setdefault(r - 1, []).append(im)
            j = r + offset + g
            if prologue <= j < n_tiles:
                copies.append((j, g, 0, iv))
    return _check(reads, copies, n_tiles, n_slots, wait_rounds, prologue, (0,))


@pytest.mark.parametrize("n", range(0, 101))
def test_dkdv_pp_schedule(n):
    assert dkdv_pp_schedule(n) is None


@pytest.mark.parametrize("n", range(0, 101))
def test_dq_pp_schedule(n):
    assert dq_pp_schedule(n) is None


@pytest.mark.parametrize("mutation", [
    dict(offset=4),       # copies a round further ahead: overwrites a tile still read
    dict(n_slots=2),      # one slot fewer
    dict(wait_rounds=2, offset=2),  # copies a round later, waited a round later: published too late
    dict(prologue=1),     # tile 1 never copied
])
def test_dkdv_pp_schedule_mutations_fail(mutation):
    assert any(dkdv_pp_schedule(n, **mutation) is not None for n in range(0, 101))


@pytest.mark.parametrize("mutation", [
    dict(offset=3),       # copies one tile further ahead: overwrites a tile still read
    dict(n_slots=3),
    dict(wait_rounds=2),  # the copy of tile r + 2 is not published before M(r + 2)
    dict(prologue=2),
])
def test_dq_pp_schedule_mutations_fail(mutation):
    assert any(dq_pp_schedule(n, **mutation) is not None for n in range(0, 101))
