"""The compaction of SGLang's key-value index list on the GPU, with no host synchronisation
(runtime/sglang_compact.py:1-12 of the reference).

SGLang's decode kernel reads request ``r`` from ``slots[indptr[r]:indptr[r+1]]``, one token slot per
entry.  The view groups ``block_tokens`` consecutive entries of a request into a block and keeps
some blocks.  ``ekv_compact_slots`` plans every row (the blocks it reads, their order, the new
length, the read counters), gathers the new list in parallel and writes it back into the engine's
buffers, all on the stream.

A row keeps its first block and its last block, which holds its newest token and may be partial,
always.  A row reads all its blocks when the policy is not live (``active`` false), when it is
audited in this step, and when it is a row that a CUDA graph adds to fill its batch (rows from
``n_real`` on).
"""

from __future__ import annotations

import torch

import ekv_hip

COUNTS = 5  # blocks read, blocks a full read would read, read in audits, read untrimmed, read without a live policy


class SlotCompactor:
    """The buffers of the compaction, kept from step to step (runtime/sglang_compact.py:109-167).
    They grow when a batch needs more and never shrink."""

    def __init__(self, width: int, block_tokens: int, device: torch.device) -> None:
        self.width, self.block_tokens, self.device = width, block_tokens, device
        self.counts = torch.zeros(COUNTS, dtype=torch.int64, device=device)
        self.no_audit = torch.zeros(1, dtype=torch.uint8, device=device)
        self._rows = 0
        self.new_indptr = self.lens = self.table = torch.empty(0, dtype=torch.int32, device=device)
        self._out: torch.Tensor = torch.empty(0, dtype=torch.int64, device=device)

    def _reserve(self, rows: int, entries: int, dtype: torch.dtype) -> None:
        if rows > self._rows:
            self._rows = rows
            self.new_indptr = torch.empty(rows + 1, dtype=torch.int32, device=self.device)
            self.lens = torch.empty(rows, dtype=torch.int32, device=self.device)
            self.table = torch.empty(rows, self.width, dtype=torch.int32, device=self.device)
        entries = max(entries, 1)  # the device buffer is never empty
        if entries > self._out.shape[0] or dtype != self._out.dtype:
            self._out = torch.empty(max(entries, self._out.shape[0]), dtype=dtype, device=self.device)

    def compact(
        self,
        indptr: torch.Tensor,
        slots: torch.Tensor,
        keep: torch.Tensor,
        audit: torch.Tensor | None,
        active: bool,
        n_real: int,
        n_rows: int,
        entries: int,
    ) -> torch.Tensor:
        """Rewrite ``indptr[:n_rows + 1]`` and ``slots[:entries]`` in place to the view, and return the new lengths.

        ``keep`` is the bool ``[rows, width]`` policy of the view, ``audit`` the uint8 rows audited in this step
        (or ``None``), and ``entries`` the length of the engine's list, ``indptr[n_rows]``, which the host knows.
        Entries of ``slots`` past the new list keep their old values."""
        if indptr.dtype != torch.int32 or indptr.stride(0) != 1:
            raise ValueError("indptr must be contiguous int32")
        if slots.dtype not in (torch.int32, torch.int64) or slots.stride(0) != 1:
            raise ValueError("slots must be contiguous int32 or int64")
        if keep.dtype not in (torch.bool, torch.uint8) or keep.dim() != 2 or keep.stride(1) != 1:
            raise ValueError("keep must be a bool [rows, width] mask with contiguous rows")
        if keep.shape[1] < self.width and n_rows > 0:
            raise ValueError(f"keep has {keep.shape[1]} columns, the view is {self.width} blocks wide")
        if audit is not None and (audit.dtype not in (torch.bool, torch.uint8) or audit.stride(0) != 1):
            raise ValueError("audit must be a contiguous uint8 / bool vector")
        self._reserve(max(n_rows, 1), entries, slots.dtype)
        ekv_hip.call(
            "ekv_compact_slots",
            indptr.data_ptr(), slots.data_ptr(), slots.element_size(), keep.data_ptr(), keep.stride(0),
            ekv_hip.ptr(audit), int(bool(active)), int(n_real), int(n_rows), self.width, self.block_tokens,
            int(entries), self.new_indptr.data_ptr(), self.lens.data_ptr(), self.table.data_ptr(),
            self.table.stride(0), self._out.data_ptr(), self.counts.data_ptr(), 1, ekv_hip.stream_handle(),
        )
        return self.lens[:n_rows]
