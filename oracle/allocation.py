"""CPU restatement of the budget split across requests (observe/allocation.py:39-166).

TEST INFRASTRUCTURE ONLY: what the results of ``ekv_rank_uniform``, ``ekv_rank_sum`` and
``ekv_rank_maxmin`` are compared with, never the product path.

``shares`` follows Request.shares (``:46-52``): scores clamped at 0 in float64 over their sum, or
equal shares when the sum is not positive.  ``allocate_uniform`` follows allocate (``:55-67``)
and _uniform (``:79-91``): pinned blocks count against the budget; the free budget is split as
``free * open_i / total_open`` with Python's correctly rounded int / int division, floored, and
the leftover goes one block each to the requests first by (-(exact - floor), index); each request
keeps its quota of open blocks first by (-share, block index) -- a lexicographic sort on
(block index, -share), NaN shares last as NumPy's argsort puts them.
"""

from __future__ import annotations

import heapq

import numpy as np


def default_pins(n: int) -> np.ndarray:
    """The first and the last block (observe/allocation.py:39-44)."""
    mask = np.zeros(n, dtype=bool)
    if n:
        mask[0] = mask[-1] = True
    return mask


def shares(scores) -> np.ndarray:
    clamped = np.maximum(np.asarray(scores, dtype=np.float64), 0.0)
    total = clamped.sum()
    if total <= 0.0:
        return np.full(len(clamped), 1.0 / max(len(clamped), 1))
    return clamped / total


def allocate_uniform(scores_list: list, pinned_list: list, budget: int) -> list[np.ndarray]:
    sizes = [len(s) for s in scores_list]
    pinned = [np.asarray(p, dtype=bool) for p in pinned_list]
    if any(len(p) != n for p, n in zip(pinned, sizes)):
        raise ValueError("a pinned mask must have one entry per block")
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    must = sum(int(p.sum()) for p in pinned)
    if must > budget and budget < sum(sizes):
        raise ValueError(f"the budget {budget} cannot hold the {must} pinned blocks")
    if budget >= sum(sizes):
        return [np.ones(n, dtype=bool) for n in sizes]
    free = budget - must
    opened = [np.flatnonzero(~p) for p in pinned]
    total_open = sum(len(o) for o in opened)
    exact = [free * len(o) / total_open if total_open else 0.0 for o in opened]
    quota = [int(x) for x in exact]
    leftover = free - sum(quota)
    ranked = sorted(range(len(opened)), key=lambda i: (-(exact[i] - quota[i]), i))
    for i in ranked[:leftover]:
        quota[i] += 1
    kept = [p.copy() for p in pinned]
    for i, scores in enumerate(scores_list):
        sh = shares(scores)
        blocks = opened[i]
        order = blocks[np.lexsort((blocks, -sh[blocks]))]  # NaN keys sort last
        kept[i][order[: quota[i]]] = True
    return kept


def _checked(scores_list, pinned_list, budget):
    """allocate's argument rules (observe/allocation.py:57-67): None when every block is kept."""
    sizes = [len(s) for s in scores_list]
    pinned = [np.asarray(p, dtype=bool) for p in pinned_list]
    if any(len(p) != n for p, n in zip(pinned, sizes)):
        raise ValueError("a pinned mask must have one entry per block")
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    must = sum(int(p.sum()) for p in pinned)
    if must > budget and budget < sum(sizes):
        raise ValueError(f"the budget {budget} cannot hold the {must} pinned blocks")
    if budget >= sum(sizes):
        return None, pinned, must
    return sizes, pinned, must


def allocate_sum(scores_list: list, pinned_list: list, weights: list, budget: int) -> list[np.ndarray]:
    """_greedy (observe/allocation.py:94-123): the ``free`` unpinned blocks of highest weight * share;
    a gain equal to the smallest chosen one goes to the newer block first, then to the earlier request."""
    sizes, pinned, must = _checked(scores_list, pinned_list, budget)
    if sizes is None:
        return [np.ones(len(s), dtype=bool) for s in scores_list]
    free = budget - must
    kept = [p.copy() for p in pinned]
    if free <= 0 or not scores_list:
        return kept
    opened = [np.flatnonzero(~p) for p in pinned]
    index = np.concatenate(opened)
    gain = np.concatenate([w * shares(s)[o] for s, w, o in zip(scores_list, weights, opened)])
    if free >= len(gain):
        selected = np.ones(len(gain), dtype=bool)
    else:
        worst = -gain
        threshold = np.partition(worst, free - 1)[free - 1]
        selected = worst < threshold
        ties = np.flatnonzero(worst == threshold)
        selected[ties[np.argsort(-index[ties], kind="stable")][: free - int(selected.sum())]] = True
    start = 0
    for r, blocks in enumerate(opened):
        kept[r][blocks[selected[start : start + len(blocks)]]] = True
        start += len(blocks)
    return kept


def allocate_maxmin(scores_list: list, pinned_list: list, budget: int) -> list[np.ndarray]:
    """_water_level (observe/allocation.py:126-166): raise the lowest retained share as far as the
    budget allows (a 60-step bisection of the level, every request searched at once in one array of
    its running totals shifted by 2 r), then spend what is left on the lowest request first."""
    sizes, pinned, must = _checked(scores_list, pinned_list, budget)
    if sizes is None:
        return [np.ones(len(s), dtype=bool) for s in scores_list]
    free = budget - must
    n = len(scores_list)
    sh = [shares(s) for s in scores_list]
    order = [np.flatnonzero(~p)[np.argsort(-sh[r][~p], kind="stable")] for r, p in enumerate(pinned)]
    base = [float(sh[r][p].sum()) for r, p in enumerate(pinned)]
    prefix = [np.cumsum(sh[r][order[r]]) for r in range(n)]
    stacked = np.concatenate([p + 2.0 * r for r, p in enumerate(prefix)]) if n else np.zeros(0)
    counts_open = np.array([len(o) for o in order])
    starts = np.concatenate(([0], np.cumsum(counts_open)[:-1])) if n else np.zeros(0, dtype=np.int64)
    offsets = 2.0 * np.arange(n)
    base_a = np.array(base)

    def extra(level: float) -> np.ndarray:
        need = level - base_a
        position = np.searchsorted(stacked, need - 1e-12 + offsets) - starts
        return np.where(need <= 1e-12, 0, np.minimum(position + 1, counts_open))

    low, high = 0.0, 1.0
    for _ in range(60):
        mid = (low + high) / 2
        if int(extra(mid).sum()) <= free:
            low = mid
        else:
            high = mid
    counts = [int(c) for c in extra(low)]
    kept = [p.copy() for p in pinned]
    for r, k in enumerate(counts):
        kept[r][order[r][:k]] = True
    leftover = free - sum(counts)
    retained = [base[r] + (float(prefix[r][counts[r] - 1]) if counts[r] else 0.0) for r in range(n)]
    heap = [(retained[r], r) for r in range(n) if counts[r] < len(order[r])]
    heapq.heapify(heap)
    while leftover > 0 and heap:
        level, r = heapq.heappop(heap)
        block = order[r][counts[r]]
        kept[r][block] = True
        counts[r] += 1
        leftover -= 1
        if counts[r] < len(order[r]):
            heapq.heappush(heap, (level + float(sh[r][block]), r))
    return kept
