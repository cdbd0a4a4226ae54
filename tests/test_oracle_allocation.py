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
