"""CPU restatement of Controller._allocate's keep rule (observe/controller.py:398-451) for the
``uniform``, ``sum`` and ``maxmin`` objectives (``Settings.objective``, observe/controller.py:30).

A row takes part when its length exceeds ``cap_above_blocks`` and its request is present with
evidence (``:402-408``).  Its ``n = min(length, width)`` blocks score by its shares (zero-padded,
``:416-419``); block 0, the blocks from ``n - 1 - recent_blocks`` on and the blocks from its
audited length on are pinned (``:420-424``); released blocks leave the request (``:425-431``).
The budget is ``max(pinned, int(ceil(fraction * total)))`` in float64 over every block of the
taking-part rows, freed or not (``:435-437``).  Rows that do not take part keep every block, and
so does every position past a row's ``n`` (``:401, 444``).  A request holds its existing blocks only,
in order (``Request(scores=scores[exists], ...)``, ``:429-431``), so for ``sum`` a tie between requests
goes to the block that is newer within its own request's remaining blocks.
"""

from __future__ import annotations

import math

import numpy as np

from oracle.allocation import allocate_maxmin, allocate_sum, allocate_uniform


def keep_rows(
    shares: np.ndarray,
    lengths: np.ndarray,
    evidence: np.ndarray,
    fraction: float,
    recent_blocks: int = 4,
    cap_above_blocks: int = 0,
    audited_blocks: np.ndarray | None = None,
    released: np.ndarray | None = None,
    objective: str = "uniform",
    weights: np.ndarray | None = None,
) -> tuple[np.ndarray, int]:
    """The committed keep mask ``uint8[rows, width]`` and the budget.  ``weights``: each row's request
    weight (``Controller.weight``, observe/controller.py:430), 1.0 by default; only ``sum`` uses it."""
    rows, width = shares.shape
    keep = np.ones((rows, width), dtype=np.uint8)
    taking = [r for r in range(rows) if lengths[r] > cap_above_blocks and evidence[r]]
    scores_list, pinned_list, exists_list = [], [], []
    for r in taking:
        n = min(int(lengths[r]), width)
        scores = np.asarray(shares[r, :n], dtype=np.float64)
        pinned = np.zeros(n, dtype=bool)
        pinned[0] = True
        pinned[max(0, n - 1 - recent_blocks) :] = True
        if audited_blocks is not None:
            pinned[int(audited_blocks[r]) :] = True
        exists = np.ones(n, dtype=bool) if released is None else ~np.asarray(released[r, :n], dtype=bool)
        exists_list.append(exists)
        scores_list.append(scores[exists])
        pinned_list.append(pinned[exists])
    if not taking:
        return keep, 0
    total = sum(len(e) for e in exists_list)
    floor = sum(int(p.sum()) for p in pinned_list)
    budget = max(floor, int(math.ceil(fraction * total)))
    if objective == "uniform":
        kept_list = allocate_uniform(scores_list, pinned_list, budget)
    elif objective == "sum":
        w = [1.0 if weights is None else float(weights[r]) for r in taking]
        kept_list = allocate_sum(scores_list, pinned_list, w, budget)
    elif objective == "maxmin":
        kept_list = allocate_maxmin(scores_list, pinned_list, budget)
    else:
        raise ValueError(f"unknown objective {objective!r}")
    for r, exists, kept in zip(taking, exists_list, kept_list):
        full = np.zeros(len(exists), dtype=bool)
        full[exists] = kept
        keep[r, : len(exists)] = full
    return keep, budget
