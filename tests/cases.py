"""Shared builders of test inputs from the known-answer fixture and small random cases."""

from __future__ import annotations

import numpy as np


def lse_of(case: dict) -> np.ndarray:
    """The ``lse[layer, row, block, query_row]`` input of a tile-share known-answer case."""
    shape = tuple(case["shape"])
    lse = np.full(shape, case["fill"], dtype=np.float32)
    for layer, row, q, values in case.get("set", []):
        lse[layer, row, :, q] = np.array(values, dtype=np.float32)
    if "tile_masses" in case:  # what the kernel stores per block: the tile's log mass split over 2 blocks
        masses = np.array(case["tile_masses"])
        lse[...] = np.repeat(np.log(masses / case["tile_blocks"]), case["tile_blocks"]).astype(np.float32).reshape(shape)
    if "block_masses_by_query" in case:
        masses = np.array(case["block_masses_by_query"])  # [query, block]
        lse[...] = np.log(masses).T.astype(np.float32).reshape(shape)
    return lse


def block_lse(scores: np.ndarray, sizes: list[int]) -> np.ndarray:
    """The log-sum-exp of the scores of each block."""
    out, start = [], 0
    for n in sizes:
        out.append(np.log(np.exp(scores[start : start + n]).sum()))
        start += n
    return np.array(out)


def softmax_mass(scores: np.ndarray, sizes: list[int]) -> np.ndarray:
    """The softmax weight of each block, computed directly from the scores."""
    w = np.exp(scores - scores.max())
    w /= w.sum()
    starts = np.cumsum([0, *sizes[:-1]])
    return np.array([w[s : s + n].sum() for s, n in zip(starts, sizes)])


def loop_view(table: list[int], length: int, keep: list[bool], block_size: int) -> tuple[list[int], int]:
    """The kept blocks and view length of one request, built one block at a time
    (the construction of tests/test_block_view.py:45-52)."""
    n = -(-length // block_size)
    if n <= 0:
        return [], 0
    chosen = [b for b in range(n) if keep[b] or b in (0, n - 1)]
    return [table[b] for b in chosen], (len(chosen) - 1) * block_size + length - (n - 1) * block_size


def random_requests(rng: np.random.Generator, count: int, max_blocks: int, ties: bool = False):
    """(scores, pinned) lists; with ``ties`` the scores take few distinct values."""
    scores, pinned = [], []
    for _ in range(count):
        n = int(rng.integers(2, max_blocks + 1))
        if ties:
            s = rng.integers(0, 4, size=n).astype(np.float32)
        else:
            s = (rng.random(n) ** float(rng.uniform(1, 6))).astype(np.float32)
        p = np.zeros(n, dtype=bool)
        p[0] = p[-1] = True
        if rng.random() < 0.3:
            p[rng.integers(0, n, size=max(1, n // 5))] = True
        scores.append(s)
        pinned.append(p)
    return scores, pinned


def audit_on(plane, caches=()) -> None:
    """Switch a recording plane on the way the engine does (runtime/block_view.py:283-288 with
    runtime/audit.py:86-113): the layer table first, then the flag."""
    plane.attach([int(c.data_ptr()) for c in caches] or [0])
    plane.set(True)
