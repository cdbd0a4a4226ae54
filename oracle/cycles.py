"""The per-row cycle-accumulator contract (observe/cycles.py:1-45, 116-182), as checks.

The accumulator is a device ``uint64[rows]`` that only grows (MONOTONE), whose per-window
deltas add across launches and kernels (ADDITIVE), and whose per-row shares partition unity.
"""

from __future__ import annotations

import numpy as np


def delta(start: np.ndarray, end: np.ndarray) -> dict[int, int]:
    """``{row: cycles}`` of a window; a negative delta is an error, never clamped (observe/cycles.py:116-132)."""
    out: dict[int, int] = {}
    for r, (s, e) in enumerate(zip(np.asarray(start).tolist(), np.asarray(end).tolist())):
        d = int(e) - int(s)
        if d < 0:
            raise ValueError(f"negative cycle delta ({d}) at row {r}")
        if d:
            out[r] = d
    return out


def shares(row_cycles: dict) -> dict:
    """Partition of unity over rows; empty stays empty (observe/cycles.py:177-182)."""
    total = sum(row_cycles.values())
    if total <= 0:
        return {}
    return {r: c / total for r, c in row_cycles.items()}
