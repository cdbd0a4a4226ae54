"""CPU restatement of Controller._allocate's keep rule (observe/controller.py:398-451) for the
``uniform`` objective.

A row takes part when its length exceeds ``cap_above_blocks`` and its request is present with
evidence (``:402-408``).  Its ``n = min(length, width)`` blocks score by its shares (zero-padded,
``:416-419``); block 0, the blocks from ``n - 1 - recent_blocks`` on and the blocks from its
audited length on are pinned (``:420-424``); released blocks leave the request (``:425-431``).
The budget is ``max(pinned, int(ceil(fraction * total)))`` in float64 over every block of the
taking-part rows, freed or not (``:435-437``).  Rows that do not take part keep every block, and
so does every position past a row's ``n`` (``:401, 444``).
"""

from __future__ import annotations

import math

import numpy as np

from oracle.allocation import allocate_uniform


def keep_rows(
    shares: np.ndarray,
    lengths: np.ndarray,
    evidence: np.ndarray,
    fraction: float,
    recent_blocks: int = 4,
    cap_above_blocks: int = 0,
    audited_blocks: np.ndarray | None = None,
    released: np.ndarray | None = None,
) -> tuple[np.ndarray, int]:
    """The committed keep mask ``uint8[rows, width]`` and the budget."""
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
    for r, exists, kept in zip(taking, exists_list, allocate_uniform(scores_list, pinned_list, budget)):
        full = np.zeros(len(exists), dtype=bool)
        full[exists] = kept
        keep[r, : len(exists)] = full
    return keep, budget
