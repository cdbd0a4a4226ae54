"""CPU restatement of the share normalisation (observe/tile_shares.py:58-173).

``log_weights`` follows read_tile_rows (``:129-173``): ``u = m + log(l) - float32(log(T))`` in
float32.  ``normalize`` follows normalize_tile_lse (``:58-103``), restated record by record in
float64: for each (layer, row, query row) the blocks ``b < row_blocks[row]`` carry
``u + log(T / valid_in_tail)`` when they sit in a partial last tile (``:84-87``); the finite ones
form a softmax (``:90-95``); the row's result is the mean of those softmaxes over the records
that had one (``:96, 101-102``) or the renormalised per-block max (``:97-100``); cells past the
row are 0 and a row with no record is all NaN (``:103``).
"""

from __future__ import annotations

import numpy as np


def log_weights(m: np.ndarray, l: np.ndarray, tile_blocks: int) -> np.ndarray:
    """``u`` from the two planes, float32 like the reference's reader."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return (np.asarray(m, np.float32) + np.log(np.asarray(l, np.float32))) - np.float32(np.log(tile_blocks))


def normalize(lse: np.ndarray, row_blocks: np.ndarray, tile_blocks: int, aggregate: str = "mean") -> np.ndarray:
    """Shares ``float64[rows, width]`` from ``lse[layer, row, block, query_row]``."""
    if aggregate not in ("mean", "max"):
        raise ValueError(f"unknown aggregate {aggregate!r}")
    lse = np.asarray(lse)
    if lse.ndim != 4:
        raise ValueError("lse must be [layers, rows, blocks, query_rows]")
    layers, rows, width, cells = lse.shape
    row_blocks = np.asarray(row_blocks)
    if row_blocks.shape != (rows,) or tile_blocks < 1:
        raise ValueError("row_blocks must give one length per row, and tile_blocks must be positive")
    out = np.zeros((rows, width))
    for r in range(rows):
        n = int(row_blocks[r])
        live = max(0, min(n, width))
        regain = np.zeros(live)
        if n % tile_blocks != 0:
            tail_start = (n // tile_blocks) * tile_blocks
            regain[tail_start:live] = np.log(tile_blocks / max(n - tail_start, 1))
        vectors = []
        for layer in range(layers):
            for c in range(cells):
                u = lse[layer, r, :live, c].astype(np.float64) + regain
                ok = np.isfinite(u)
                if not ok.any():
                    continue
                w = np.where(ok, np.exp(np.where(ok, u, 0.0) - u[ok].max()), 0.0)
                vectors.append(w / w.sum())
        if not vectors:
            out[r] = np.nan
            continue
        stack = np.array(vectors)
        if aggregate == "mean":
            out[r, :live] = stack.sum(axis=0) / len(vectors)
        else:
            peak = stack.max(axis=0)
            total = peak.sum()
            out[r, :live] = peak / total if total > 0 else 0.0
    return out


def read_rows(planes: np.ndarray, layers: int, row_ids: np.ndarray, tile_blocks: int) -> np.ndarray:
    """``u[layers, len(row_ids), width, cells]`` of the chosen rows of a host copy of the block
    ``planes[2, table_layers, rows, width, cells]`` (what read_tile_rows returns)."""
    row_ids = np.asarray(row_ids)
    if row_ids.size > 1 and np.any(np.diff(row_ids) <= 0):
        raise ValueError("row_ids must be ascending and distinct")
    return log_weights(planes[0, :layers][:, row_ids], planes[1, :layers][:, row_ids], tile_blocks)
