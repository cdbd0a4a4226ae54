"""The SGLang index-list compaction restated on the CPU (runtime/sglang_compact.py:22-106).

TEST INFRASTRUCTURE ONLY: what the results of ``ekv_compact_slots`` are compared with, never the product
path.
"""

from __future__ import annotations

import numpy as np


def compact(indptr, slots, keep, audit, active: bool, n_real: int, n_rows: int, block_tokens: int) -> dict:
    """The plan and the gather of one call: ``new_indptr``, ``lens``, the kept blocks of each row
    (``table``), the new list ``out`` and the increments of the five read counters."""
    indptr = np.asarray(indptr, dtype=np.int64)
    slots = np.asarray(slots)
    keep = np.asarray(keep, dtype=bool)
    bt = block_tokens
    new_indptr = [0]
    lens, table = [], []
    read = full = audit_read = untrimmed = 0
    for row in range(n_rows):  # plan_kernel, runtime/sglang_compact.py:41-72
        length = int(indptr[row + 1] - indptr[row])
        blocks = -(-length // bt) if length > 0 else 0
        real = row < n_real
        audited = audit is not None and real and bool(audit[row])
        whole = (not active) or audited or (row >= n_real)
        chosen = [b for b in range(blocks) if whole or b == 0 or b == blocks - 1 or (real and keep[row, b])]
        kept = len(chosen)
        new_length = (kept - 1) * bt + length - (blocks - 1) * bt if blocks > 0 else 0
        table.append(chosen)
        lens.append(new_length)
        new_indptr.append(new_indptr[-1] + new_length)
        if real:
            read += kept
            full += blocks
            audit_read += kept if audited else 0
            untrimmed += kept if (new_length == length and not audited and active) else 0
    counts = [read, full, audit_read, untrimmed, read if not active else 0]
    # gather_kernel, runtime/sglang_compact.py:83-106: position p belongs to the last row whose new
    # offset is <= p, which is the row whose [start, start + length) holds it, and comes from that
    # row's kept block offset // bt at offset % bt
    out = np.zeros(new_indptr[-1], dtype=slots.dtype)
    for row in range(n_rows):
        offset = np.arange(lens[row])
        if len(offset) == 0:
            continue
        block = np.asarray(table[row], dtype=np.int64)[offset // bt]
        out[new_indptr[row] : new_indptr[row + 1]] = slots[indptr[row] + block * bt + offset % bt]
    return {"new_indptr": new_indptr, "lens": lens, "table": table, "out": out, "counts": counts}
