"""The uniform-allocation oracle against the reference's known answers (tests/test_allocation.py),
brute force over the ranking, and the float64 largest-remainder order."""

import itertools
from fractions import Fraction

import numpy as np
import pytest

from cases import random_requests
from oracle import allocation as oa


def pins(n):
    return oa.default_pins(n)


def test_known_answers(known_answers):
    case = known_answers["uniform"]["fraction_and_own_ranking"]
    scores = [np.array(s) for s in case["scores"]]
    kept = oa.allocate_uniform(scores, [pins(len(s)) for s in scores], case["budget"])
    assert sum(int(k.sum()) for k in kept) == case["kept_total"]
    assert abs(kept[0].sum() / 5 - kept[1].sum() / 10) <= case["fraction_gap"]
    for req, block in case["must_keep"]:
        assert kept[req][block]
    case = known_answers["uniform"]["identical_requests_split_evenly"]
    scores = [np.array(case["scores"])] * case["requests"]
    counts = [int(k.sum()) for k in oa.allocate_uniform(scores, [pins(len(s)) for s in scores], case["budget"])]
    assert sum(counts) == case["kept_total"] and max(counts) - min(counts) <= case["spread"]
    case = known_answers["uniform"]["budget_below_pins"]
    with pytest.raises(ValueError):
        oa.allocate_uniform([np.ones(n) for n in case["sizes"]], [pins(n) for n in case["sizes"]], case["budget"])
    case = known_answers["uniform"]["budget_covers_everything"]
    kept = oa.allocate_uniform([np.ones(n) for n in case["sizes"]], [pins(n) for n in case["sizes"]], case["budget"])
    assert all(k.all() for k in kept)


def test_each_request_keeps_its_best_open_blocks_by_brute_force():
    # for every request the kept open blocks must be the lexicographically best set of its size under
    # (share desc, index asc): checked by enumerating every subset of that size
    rng = np.random.default_rng(11)
    for _ in range(60):
        scores, pinned = random_requests(rng, 3, 7, ties=bool(rng.random() < 0.5))
        total = sum(len(s) for s in scores)
        must = sum(int(p.sum()) for p in pinned)
        budget = int(rng.integers(must, total + 1))
        kept = oa.allocate_uniform(scores, pinned, budget)
        assert sum(int(k.sum()) for k in kept) == min(budget, total)
        for s, p, k in zip(scores, pinned, kept):
            assert k[p].all()  # pinned blocks are kept
            opened = [b for b in range(len(s)) if not p[b]]
            chosen = [b for b in opened if k[b]]
            sh = oa.shares(s)
            # the best subset of that size: lexicographically least sorted (-share, index) list
            best = min(sorted((-sh[b], b) for b in c) for c in itertools.combinations(opened, len(chosen)))
            assert sorted((-sh[b], b) for b in chosen) == best


def test_quota_split_is_largest_remainder_in_float64():
    # Every request's quota is floor(free * open_i / total) plus one for the requests first by
    # (-(remainder), index).  With exact remainders tied, float64 rounding decides: opens
    # [2337, 4125, 4999, 1259, 4880] with free 5600 leave 3 blocks over; row 4 (remainder 8/11) takes
    # one, and rows 0, 2 and 3 tie at 13/22 exactly.  The float64 remainders order them 0, 3, 2, so
    # rows 0 and 3 take the other two, where exact arithmetic with the index rule would pick 0 and 2.
    opens = [2337, 4125, 4999, 1259, 4880]
    free, total = 5600, sum(opens)
    exact = [Fraction(free * o, total) for o in opens]
    assert exact[0] - int(exact[0]) == exact[2] - int(exact[2]) == exact[3] - int(exact[3]) == Fraction(13, 22)
    scores = [np.full(o, 1.0) for o in opens]
    kept = oa.allocate_uniform(scores, [np.zeros(o, dtype=bool) for o in opens], free)
    floors = [int(e) for e in exact]
    extra = [int(k.sum()) - f for k, f in zip(kept, floors)]
    assert extra == [1, 0, 0, 1, 1]
    exact_rule = sorted(range(5), key=lambda i: (-(exact[i] - floors[i]), i))[:3]
    assert sorted(exact_rule) == [0, 2, 4]  # the two orders differ here


def test_nan_scores_rank_last_and_zero_totals_tie():
    kept = oa.allocate_uniform([np.array([1.0, np.nan, 3.0, 2.0, 5.0])], [np.array([1, 0, 0, 0, 1], bool)], 3)
    assert kept[0].tolist() == [True, True, False, False, True]  # every share is NaN: index order
    kept = oa.allocate_uniform([np.array([0.0, -1.0, 0.0, -2.0, 0.0])], [np.array([1, 0, 0, 0, 1], bool)], 4)
    assert kept[0].tolist() == [True, True, True, False, True]  # no evidence: equal shares, index order


def test_float32_scores_rank_like_their_float64_shares():
    # the device ranks max(s, 0) of float32 scores; that order equals the stable argsort of the float64 shares
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(2, 400))
        s = rng.dirichlet(np.full(n, 0.1)).astype(np.float32)
        ref = np.argsort(-oa.shares(s), kind="stable")
        key = np.lexsort((np.arange(n), -np.maximum(s, 0).astype(np.float64)))
        assert np.array_equal(ref, key)


# ---- sum and maxmin --------------------------------------------------------------------------

def plain_sum(scores, pinned, weights, budget):
    """Every unpinned block sorted by weighted share, newer blocks first on ties, then earlier requests."""
    kept = [p.copy() for p in pinned]
    cells = [(w * oa.shares(s)[b], b, i) for i, (s, p, w) in enumerate(zip(scores, pinned, weights))
             for b in np.flatnonzero(~p)]
    cells.sort(key=lambda c: (-c[0], -c[1], c[2]))
    for _gain, b, i in cells[: budget - sum(int(p.sum()) for p in pinned)]:
        kept[i][b] = True
    return kept


def plain_maxmin(scores, pinned, budget):
    """The level bisected with one search per request, then the rest spent on the lowest request."""
    sh = [oa.shares(s) for s in scores]
    order = [np.flatnonzero(~p)[np.argsort(-sh[i][~p], kind="stable")] for i, p in enumerate(pinned)]
    base = [float(sh[i][p].sum()) for i, p in enumerate(pinned)]
    prefix = [np.cumsum(sh[i][order[i]]) for i in range(len(scores))]
    free = budget - sum(int(p.sum()) for p in pinned)

    def counts_at(level):
        out = []
        for i in range(len(scores)):
            need = level - base[i]
            out.append(0 if need <= 1e-12 else min(int(np.searchsorted(prefix[i], need - 1e-12)) + 1, len(order[i])))
        return out

    low, high = 0.0, 1.0
    for _ in range(60):
        mid = (low + high) / 2
        if sum(counts_at(mid)) <= free:
            low = mid
        else:
            high = mid
    counts = counts_at(low)
    kept = [p.copy() for p in pinned]
    for i, k in enumerate(counts):
        kept[i][order[i][:k]] = True
    leftover = free - sum(counts)
    while leftover > 0:
        open_rows = [i for i in range(len(scores)) if counts[i] < len(order[i])]
        if not open_rows:
            break
        i = min(open_rows, key=lambda r: (base[r] + (float(prefix[r][counts[r] - 1]) if counts[r] else 0.0), r))
        kept[i][order[i][counts[i]]] = True
        counts[i] += 1
        leftover -= 1
    return kept


def sum_case(rng, requests):
    scores, weights, pinned = [], [], []
    for _ in range(requests):
        n = int(rng.integers(3, 40))
        scores.append(rng.integers(0, 4, size=n).astype(float))  # many equal scores, so many ties
        weights.append(float(rng.choice([1.0, 2.0, 0.5])))
        pinned.append(pins(n))
    total = sum(len(s) for s in scores)
    must = sum(int(p.sum()) for p in pinned)
    return scores, weights, pinned, int(rng.integers(must, max(total, must + 1)))


@pytest.mark.parametrize("seed", range(40))
def test_sum_equals_the_plain_sort_including_ties(seed):
    rng = np.random.default_rng(seed)
    scores, weights, pinned, budget = sum_case(rng, int(rng.integers(1, 9)))
    got, want = oa.allocate_sum(scores, pinned, weights, budget), plain_sum(scores, pinned, weights, budget)
    assert all(np.array_equal(a, b) for a, b in zip(got, want))


def test_sum_maximises_the_weighted_share_by_brute_force():
    rng = np.random.default_rng(5)
    for _ in range(40):
        scores, pinned = random_requests(rng, 3, 6, ties=bool(rng.random() < 0.5))
        weights = [float(rng.choice([1.0, 2.0, 0.5])) for _ in scores]
        total = sum(len(s) for s in scores)
        must = sum(int(p.sum()) for p in pinned)
        budget = int(rng.integers(must, total + 1))
        kept = oa.allocate_sum(scores, pinned, weights, budget)
        cells = [(w * oa.shares(s)[b]) for s, p, w in zip(scores, pinned, weights) for b in np.flatnonzero(~p)]
        free = min(budget - must, len(cells))
        best = max((sum(c) for c in itertools.combinations(cells, free)), default=0.0)
        got = sum(w * oa.shares(s)[b] for s, p, w, k in zip(scores, pinned, weights, kept) for b in np.flatnonzero(~p & k))
        assert sum(int(k.sum()) for k in kept) == min(budget, total)
        assert got >= best - 1e-12


@pytest.mark.parametrize("seed", range(40))
def test_maxmin_equals_the_plain_search(seed):
    rng = np.random.default_rng(seed)
    scores, pinned = random_requests(rng, int(rng.integers(1, 9)), 40)
    total = sum(len(s) for s in scores)
    must = sum(int(p.sum()) for p in pinned)
    budget = int(rng.integers(must, max(total, must + 1)))
    got, want = oa.allocate_maxmin(scores, pinned, budget), plain_maxmin(scores, pinned, budget)
    assert all(np.array_equal(a, b) for a, b in zip(got, want))


def test_maxmin_raises_the_lowest_share_by_brute_force():
    # the smallest retained share is the largest any split of the budget reaches
    rng = np.random.default_rng(9)
    for _ in range(30):
        scores = [rng.dirichlet(np.full(int(rng.integers(3, 6)), 0.5)) for _ in range(3)]
        pinned = [pins(len(s)) for s in scores]
        total = sum(len(s) for s in scores)
        must = sum(int(p.sum()) for p in pinned)
        budget = int(rng.integers(must, total + 1))
        kept = oa.allocate_maxmin(scores, pinned, budget)
        got = min(float(oa.shares(s)[k].sum()) for s, k in zip(scores, kept))
        best = 0.0
        opened = [np.flatnonzero(~p) for p in pinned]
        free = budget - must
        for split in itertools.product(*[range(len(o) + 1) for o in opened]):
            if sum(split) > free:
                continue
            level = min(float(oa.shares(s)[p].sum()) + np.sort(oa.shares(s)[o])[::-1][:k].sum()
                        for s, p, o, k in zip(scores, pinned, opened, split))
            best = max(best, level)
        assert got >= best - 1e-9
