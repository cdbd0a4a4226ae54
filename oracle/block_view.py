"""CPU restatement of the block-table view (runtime/block_view.py:36-56, 272-281, 297-329).

``compact`` follows compact_block_table: ``n = ceil(L / bs)`` (floor division), blocks 0 and
``n - 1`` are forced into the keep and blocks ``>= n`` out (``:49-51``); the row becomes its kept
entries in order followed by the others in order -- the stable argsort of ``~keep`` (``:52, 56``)
-- written here as the concatenation of the kept and the dropped entries of each row; the length is ``(kept - 1) * bs + last`` for
``n > 0`` (``:53-55``).  ``compose`` follows DecodeView.build's keep (``:272-281``) and ``count``
its read counters (``:297-329``).
"""

from __future__ import annotations

import numpy as np


def compact(table: np.ndarray, seq_lens: np.ndarray, keep: np.ndarray, block_size: int):
    table = np.asarray(table)
    rows, width = table.shape
    view = np.zeros_like(table)
    lens = np.zeros(rows, dtype=np.int64)
    positions = np.arange(width)
    for r in range(rows):
        length = int(seq_lens[r])
        n = (length + block_size - 1) // block_size  # Python floor division, as torch's
        k = (np.asarray(keep[r], dtype=bool) | (positions == 0) | (positions == n - 1)) & (positions < n)
        kept = table[r][k]
        view[r] = np.concatenate([kept, table[r][~k]])
        lens[r] = (len(kept) - 1) * block_size + (length - (n - 1) * block_size) if n > 0 else 0
    return view, lens


def compose(
    committed: np.ndarray,
    live: bool,
    audited: np.ndarray | None,
    decoding: np.ndarray | None,
    released: np.ndarray | None,
) -> np.ndarray:
    """The keep mask handed to the compaction (runtime/block_view.py:272-281)."""
    keep = np.asarray(committed, dtype=bool).copy()
    if not live:
        keep[:] = True
    elif audited is not None:
        keep |= np.asarray(audited, dtype=bool)[:, None]
    if decoding is not None:
        keep |= ~np.asarray(decoding, dtype=bool)[:, None]
    if released is not None:
        keep &= ~np.asarray(released, dtype=bool)
    return keep


def count(
    read_lens: np.ndarray,
    full_lens: np.ndarray,
    decoding: np.ndarray | None,
    audited: np.ndarray | None,
    expired: bool,
    block_size: int,
) -> np.ndarray:
    """The increments of DecodeView's five counters: read, full, audit, untrimmed, expired."""
    read = (np.asarray(read_lens, np.int64) + block_size - 1) // block_size
    full = (np.asarray(full_lens, np.int64) + block_size - 1) // block_size
    whole = np.asarray(read_lens) == np.asarray(full_lens)
    if decoding is not None:
        read, full = read * decoding, full * decoding
    in_audit = np.zeros(len(read), dtype=bool) if audited is None else np.asarray(audited, dtype=bool)
    live_whole = whole & ~in_audit & (not expired)
    return np.array(
        [read.sum(), full.sum(), (read * in_audit).sum(), (read * live_whole).sum(), read.sum() if expired else 0],
        dtype=np.int64,
    )
