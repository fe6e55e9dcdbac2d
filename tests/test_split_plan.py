"""Split-K item size for the decode launch (host logic, no GPU).

The work list comes from the library's own planner (lf_plan_decode, host code); each item
runs as one workgroup per kv head, two workgroups per CU.  The dispatch is simulated as a
greedy list schedule (each item to the earliest free slot, in plan order), which is
independent of the closed-form cost the chooser minimises."""
import ctypes
import heapq

import numpy as np
import pytest

from logitfill_amd import _native, synth
from logitfill_amd.packed.reference import (ALONE_FACTOR, ITEM_OVERHEAD_PAGES, LATE_SLOWDOWN, age_split,
                                            choose_pages_per_split, paired_plan, paired_split,
                                            plan_work, residual_pages)

SLOTS = 512  # 256 CUs x 2 workgroups
RES = residual_pages([100])  # the c2 residual's cost (100-token tails)


def plan_items(hist_pages, pps, res=RES):
    """(b, page0, page1, flags) rows from lf_plan_decode."""
    lib = _native.load()
    B = len(hist_pages)
    cap = sum(-(-(p + res) // pps) for p in hist_pages) + B
    hp = (ctypes.c_int32 * B)(*hist_pages)
    work = (ctypes.c_int32 * (4 * cap))()
    seq = (ctypes.c_int32 * (2 * B))()
    n = lib.lf_plan_decode(hp, B, pps, res, work, cap, seq)
    assert n > 0
    return [tuple(work[4 * i:4 * i + 4]) for i in range(n)]


def makespan(hist_pages, n_kv, pps):
    """Greedy list schedule of the plan's workgroups on SLOTS slots, in page units."""
    slots = [0.0] * SLOTS
    for b, p0, p1, flags in plan_items(hist_pages, pps):
        cost = (p1 - p0) + (RES if flags else 0) + ITEM_OVERHEAD_PAGES
        for _ in range(n_kv):
            t = heapq.heappop(slots)
            heapq.heappush(slots, t + cost)
    return max(slots)


def one_round_size(hist_pages, n_kv, res=RES):
    return -(-n_kv * sum(p + res for p in hist_pages) // SLOTS)


def test_residual_cost_grows_with_the_tail():
    """3 pages for the residual pass itself plus one for a tail of 64 tokens or more, from the
    longest tail of the batch (known answers, and never below the fixed part)."""
    assert [residual_pages([t]) for t in (0, 1, 37, 63, 64, 100, 127)] == [3, 3, 3, 3, 4, 4, 4]
    assert residual_pages([]) == 3 and residual_pages([5, 100, 37]) == 4 and residual_pages([500]) == 4
    costs = [residual_pages([t]) for t in range(128)]
    assert costs == sorted(costs)


def test_uniform_batch_keeps_one_round():
    """c2: every sequence's work divides into the one-round size; the plan fills the slots
    exactly once."""
    hist_pages, n_kv, res = [256] * 16, 4, residual_pages([100])
    pps = choose_pages_per_split(hist_pages, n_kv, res)
    assert pps == 33 == one_round_size(hist_pages, n_kv, res)
    assert n_kv * len(plan_items(hist_pages, pps, res)) <= SLOTS


def test_small_batch_takes_a_cu_per_workgroup():
    """c1 (8 x 64 pages + a 37-token residual, 2 kv heads): 5-page items, 14 per sequence, 224
    workgroups -- each with a CU of its own -- instead of the one-round 3-page items (368,
    sharing CUs): (5 + overhead) x ALONE_FACTOR < 3 + overhead.  4-page items (272 workgroups)
    would share CUs again and cost more than either."""
    hist_pages, n_kv, res = [64] * 8, 2, residual_pages([37])
    assert one_round_size(hist_pages, n_kv, res) == 3
    pps = choose_pages_per_split(hist_pages, n_kv, res)
    assert pps == 5
    assert n_kv * len(plan_items(hist_pages, pps, res)) == 224 <= SLOTS // 2
    assert (5 + ITEM_OVERHEAD_PAGES) * ALONE_FACTOR < 3 + ITEM_OVERHEAD_PAGES < 4 + ITEM_OVERHEAD_PAGES


def test_ragged_batch_avoids_the_second_round():
    """c4 (32 sequences of U[4K, 64K] tokens, 8 kv heads): the one-round size leaves more
    items than slots; the chosen size's simulated makespan is at least 25 % shorter and
    within 10 % of the work bound."""
    pages, _ = synth.ragged_lengths(32, seed=4)
    n_kv = 8
    top = one_round_size(pages, n_kv)
    assert n_kv * len(plan_items(pages, top)) > SLOTS
    pps = choose_pages_per_split(pages, n_kv, RES)
    assert 1 <= pps < top
    chosen, naive = makespan(pages, n_kv, pps), makespan(pages, n_kv, top)
    assert chosen <= 0.75 * naive
    bound = sum(n_kv * (p + RES) for p in pages) / SLOTS
    assert chosen <= 1.10 * (bound + ITEM_OVERHEAD_PAGES) + pps


def test_chosen_size_is_best_of_the_scan_by_simulation():
    """Over several seeded ragged batches the chosen size is within 5 % of the best simulated
    makespan over every size up to the one-round size."""
    for seed in (1, 2, 3):
        pages, _ = synth.ragged_lengths(24, seed=seed)
        n_kv = 8
        top = one_round_size(pages, n_kv)
        best = min(makespan(pages, n_kv, s) for s in range(max(1, top // 4), top + 1))
        assert makespan(pages, n_kv, choose_pages_per_split(pages, n_kv, RES)) <= 1.05 * best


def test_edge_cases(monkeypatch):
    assert choose_pages_per_split([0], 1, RES) >= 1  # a sequence without pages is one item at any size
    assert len(plan_items([0], choose_pages_per_split([0], 1, RES))) == 1
    assert choose_pages_per_split([0, 0, 3], 2, RES) >= 1
    assert choose_pages_per_split([512], 8, RES) == one_round_size([512], 8)
    monkeypatch.setenv("LOGITFILL_AMD_PAGES_PER_SPLIT", "7")
    assert choose_pages_per_split([256] * 16, 4, RES) == 7


def test_plan_work_equals_one_planner_call_for_one_size():
    """Per-sequence sizes that are all equal give lf_plan_decode's own items for every
    sequence, the sequences in decreasing item size (ties in batch order)."""
    pages = [40, 0, 7, 33, 12]
    work, seq = plan_work(pages, [5] * 5, RES)
    items = [tuple(work[4 * i:4 * i + 4]) for i in range(len(work) // 4)]
    ref = plan_items(pages, 5)
    for b in range(5):
        mine = items[seq[2 * b]:seq[2 * b] + seq[2 * b + 1]]
        assert mine == [it for it in ref if it[0] == b]
    assert sum(seq[2 * b + 1] for b in range(5)) == len(items)
    def size(b):
        return (pages[b] + RES) / (1 if pages[b] == 0 else -(-(pages[b] + RES) // 5))
    assert [it[0] for it in items if it[3] != 0] == sorted(range(5), key=lambda b: -size(b))
    uniform = [64] * 4
    w2, _ = plan_work(uniform, [9] * 4, RES)
    assert [tuple(w2[4 * i:4 * i + 4]) for i in range(len(w2) // 4)] == plan_items(uniform, 9)


def test_plan_work_runs_of_sizes_cover_every_page():
    """Mixed sizes: each sequence's items are contiguous from its first, cover its pages once
    in order, and number ceil((pages + residual) / size)."""
    pages, sizes = [30, 30, 9, 0, 17], [4, 4, 7, 2, 3]
    work, seq = plan_work(pages, sizes, RES)
    items = [tuple(work[4 * i:4 * i + 4]) for i in range(len(work) // 4)]
    for b, (p, z) in enumerate(zip(pages, sizes)):
        first, count = seq[2 * b], seq[2 * b + 1]
        mine = items[first:first + count]
        assert all(it[0] == b for it in mine)
        assert [it[1] for it in mine][0] == 0 and mine[-1][2] == p
        assert all(mine[k][2] == mine[k + 1][1] for k in range(count - 1))
        assert count == (1 if p == 0 else -(-(p + RES) // z))


def test_age_split_gives_early_workgroups_the_larger_items():
    """c2 (16 sequences x 256 pages + a 4-page residual, 4 kv heads, 256 CUs): 8 sequences of
    7 items and 8 of 9, 128 items = one round of 512 workgroups; the estimated slowest item
    (x LATE_SLOWDOWN past the first 256 workgroups) beats the uniform 8 x 32.5 pages."""
    res = residual_pages([100])
    sizes = age_split([256] * 16, 4, res, 33, 256)
    assert sizes == [38] * 8 + [29] * 8
    work, seq = plan_work([256] * 16, sizes, res)
    n = len(work) // 4
    assert n == 128 and [seq[2 * b + 1] for b in range(16)] == [7] * 8 + [9] * 8

    def slowest(work):
        t = 0.0
        for i in range(len(work) // 4):
            b, p0, p1, kind = work[4 * i:4 * i + 4]
            size = (p1 - p0) + (res if kind else 0)
            t = max(t, size * (LATE_SLOWDOWN if (i + 1) * 4 > 256 else 1.0))
        return t

    uniform, _ = plan_work([256] * 16, [33] * 16, res)
    assert slowest(work) < 0.97 * slowest(uniform)


def test_age_split_declines_other_batches():
    """Ragged lengths, a plan short of a full round (c1: 368 of 512 workgroups), more items than
    one round, one sequence: the uniform split stays."""
    assert age_split([256, 200] * 8, 4, RES, 33, 256) is None
    assert age_split([64] * 8, 2, residual_pages([37]), 3, 256) is None
    assert age_split([256] * 16, 4, RES, 20, 256) is None
    assert age_split([256], 4, RES, 33, 256) is None


def test_paired_plan_c2():
    """c2 (16 x 256 pages + a 4-page residual, 4 kv heads, 256 CUs): 4 first items of 36 pages
    per sequence, listed (dispatched) before every sequence's 4 second items of 29, 29, 29 and
    25 pages + the residual; 512 workgroups = two per CU, each CU a first and a second item of
    65 pages together.  Every page once, each sequence's partials in its own consecutive slots,
    the residual once per sequence on its last item."""
    hist, n_kv, res, cus = [256] * 16, 4, residual_pages([100]), 256
    choice = paired_split(hist, n_kv, res, cus, choose_pages_per_split(hist, n_kv, res))
    assert choice == ("paired", 36, 0)
    k = cus // (16 * n_kv)
    work, seq = paired_plan(hist, k, choice[1], res, choice[2])
    items = [tuple(work[4 * i:4 * i + 4]) for i in range(len(work) // 4)]
    assert len(items) * n_kv == 2 * cus
    first_half = items[:len(items) // 2]
    assert all(p1 - p0 == 36 and (kind & 0xff) == 0 for _, p0, p1, kind in first_half)
    slots = [(kind >> 8) - 1 for *_, kind in items]
    assert sorted(slots) == list(range(len(items)))
    for b in range(16):
        first, count = seq[2 * b], seq[2 * b + 1]
        mine = sorted((p0, p1, kind & 0xff, (kind >> 8) - 1) for bb, p0, p1, kind in items if bb == b)
        assert count == 2 * k and sorted(s for *_, s in mine) == list(range(first, first + count))
        assert mine[0][0] == 0 and mine[-1][1] == 256
        assert all(mine[j][1] == mine[j + 1][0] for j in range(len(mine) - 1))
        assert [m[2] for m in mine].count(2) == 1 and mine[-1][2] == 2 and mine[-1][1] - mine[-1][0] == 25
        # the first and second items of a CU together: 36 + 29 = 65 = (256 + 4) / 4
        assert sorted(set(m[1] - m[0] for m in mine)) == [25, 29, 36]


def test_paired_plan_c1_small_batch():
    """c1 (8 x 64 pages + a 37-token residual, 2 kv heads, 256 CUs; the uniform plan's 224
    workgroups each have a CU of their own): 16 first items of 3 pages per sequence, listed
    before all others, then 8 items of 2 pages and a residual-only item (kind 1): 25 items per
    sequence, 400 workgroups; every page once, per-sequence consecutive slots."""
    hist, n_kv, res, cus = [64] * 8, 2, residual_pages([37]), 256
    choice = paired_split(hist, n_kv, res, cus, choose_pages_per_split(hist, n_kv, res))
    assert choice == ("paired", 3, 2)
    work, seq = paired_plan(hist, 16, 3, res, 2)
    items = [tuple(work[4 * i:4 * i + 4]) for i in range(len(work) // 4)]
    assert len(items) == 8 * 25 and len(items) * n_kv == 400
    assert all(p1 - p0 == 3 and kind & 0xff == 0 for _, p0, p1, kind in items[:8 * 16])
    assert sorted((kind >> 8) - 1 for *_, kind in items) == list(range(len(items)))
    for b in range(8):
        first, count = seq[2 * b], seq[2 * b + 1]
        mine = sorted(((kind >> 8) - 1, p0, p1, kind & 0xff) for bb, p0, p1, kind in items if bb == b)
        assert count == 25 and [m[0] for m in mine] == list(range(first, first + 25))
        pages = sorted((p0, p1) for _, p0, p1, k in mine if k != 1)
        assert pages[0][0] == 0 and pages[-1][1] == 64 and all(pages[j][1] == pages[j + 1][0] for j in range(23))
        assert [m[3] for m in mine].count(1) == 1 and mine[-1][3] == 1 and mine[-1][1] == mine[-1][2]


def test_paired_split_declines_other_batches():
    """Ragged lengths, a CU count the batch x kv heads does not divide, no pages, a pairing
    that would leave a second item without a page, a plan between the two regimes."""
    assert paired_split([256, 200] * 8, 4, RES, 256, 33) is None
    assert paired_split([256] * 12, 4, RES, 256, 33) is None
    assert paired_split([0] * 16, 4, RES, 256, 33) is None
    assert paired_split([20] * 16, 4, RES, 256, 3) is None       # 4 pages of work per second item
    assert paired_split([6] * 16, 4, RES, 256, 3) == ("paired", 1, 2)  # small regime: 384 workgroups
    assert paired_split([256] * 8, 4, RES, 256, 17) == ("paired", int(round(0.56 * 260 / 8)), 0)
    assert paired_split([256] * 16, 4, RES, 256, 45) is None     # 384 workgroups: neither regime


def test_paired_plan_valid_wherever_chosen():
    """Wherever ``paired_split`` chooses a paired plan (equal sequences of 1-600 pages, batch
    1-64, 1-8 kv heads, residual costs 3-4 pages, 64-304 CUs), ``paired_plan`` builds it: every
    page of every sequence in exactly one item, one residual carrier per sequence (the last
    second item, or a residual-only item in the small-batch form), per-sequence consecutive
    partial slots, no page-less item but the residual-only one, and at most two workgroups per
    CU."""
    rng = np.random.default_rng(7)
    chosen = 0
    for _ in range(3000):
        B = int(rng.integers(1, 65))
        n_kv = int(rng.choice([1, 2, 4, 8]))
        P = int(rng.integers(1, 601))
        res = int(rng.choice([3, 4]))
        cus = int(rng.choice([64, 80, 128, 256, 304]))
        hist = [P] * B
        choice = paired_split(hist, n_kv, res, cus, choose_pages_per_split(hist, n_kv, res) if cus == 256 else
                              max(1, -(-n_kv * B * (P + res) // (2 * cus))))
        if choice is None:
            continue
        chosen += 1
        k = cus // (B * n_kv)
        work, seq = paired_plan(hist, k, choice[1], res, choice[2])
        items = [tuple(work[4 * i:4 * i + 4]) for i in range(len(work) // 4)]
        assert len(items) * n_kv <= 2 * cus, (B, n_kv, P, res, cus, choice)
        assert sorted((kind >> 8) - 1 for *_, kind in items) == list(range(len(items)))
        assert items[:B * k] == sorted(items[:B * k], key=lambda it: (it[0], it[1]))  # first items lead
        for b in range(B):
            first, count = seq[2 * b], seq[2 * b + 1]
            mine = sorted(((kind >> 8) - 1, p0, p1, kind & 0xff) for bb, p0, p1, kind in items if bb == b)
            assert [m[0] for m in mine] == list(range(first, first + count))
            spans = sorted((p0, p1) for _, p0, p1, kd in mine if kd != 1)
            assert spans[0][0] == 0 and spans[-1][1] == P
            assert all(a[1] == c[0] for a, c in zip(spans, spans[1:])) and all(p1 > p0 for p0, p1 in spans)
            kinds = [m[3] for m in mine]
            assert kinds.count(1) + kinds.count(2) == 1
            assert (kinds.count(1) == 1) == (choice[2] > 0)
    assert chosen > 50
