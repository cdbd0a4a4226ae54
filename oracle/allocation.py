"""CPU restatement of the ``uniform`` allocation (observe/allocation.py:39-91).

``shares`` follows Request.shares (``:46-52``): scores clamped at 0 in float64 over their sum, or
equal shares when the sum is not positive.  ``allocate_uniform`` follows allocate (``:55-67``)
and _uniform (``:79-91``): pinned blocks count against the budget; the free budget is split as
``free * open_i / total_open`` with Python's correctly rounded int / int division, floored, and
the leftover goes one block each to the requests first by (-(exact - floor), index); each request
keeps its quota of open blocks first by (-share, block index) -- a lexicographic sort on
(block index, -share), NaN shares last as NumPy's argsort puts them.
"""

from __future__ import annotations

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
