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


def _capacity(need: int) -> int:
    """The next power of two at or above ``need`` (at least 1): buffers grow by doubling."""
    return 1 << max(0, int(need) - 1).bit_length()


class SlotCompactor:
    """Device scratch of the compaction and the read counters, for one view (the contract of
    runtime/sglang_compact.py:99-167).

    The scratch -- the new offsets, lengths and block tables of the rows, and the gathered list --
    lives across steps so that a step allocates nothing once the batches have been seen; it grows to
    the next power of two when a batch needs more rows, entries or a wider slot type."""

    def __init__(self, width: int, block_tokens: int, device: torch.device) -> None:
        if width <= 0 or block_tokens <= 0:
            raise ValueError(f"a view of {width} blocks of {block_tokens} tokens is empty")
        self.width, self.block_tokens, self.device = width, block_tokens, device
        self.counts = torch.zeros(COUNTS, dtype=torch.int64, device=device)  # accumulated by the kernels
        self._row_room = 0
        # the plan of the last call, per row: new offsets, new token counts, kept block ids
        self.new_indptr = self.lens = self.table = torch.empty(0, dtype=torch.int32, device=device)
        self._gathered = torch.empty(0, dtype=torch.int64, device=device)

    def _room_for(self, rows: int, entries: int, slot_dtype: torch.dtype) -> None:
        if rows > self._row_room:
            self._row_room = _capacity(rows)
            n, dev = self._row_room, self.device
            self.new_indptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
            self.lens = torch.empty(n, dtype=torch.int32, device=dev)
            self.table = torch.empty(n, self.width, dtype=torch.int32, device=dev)
        if entries > self._gathered.numel() or slot_dtype != self._gathered.dtype:
            self._gathered = torch.empty(_capacity(max(entries, self._gathered.numel())), dtype=slot_dtype,
                                         device=self.device)

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
        """The view of one decode batch, written over the engine's list: ``indptr[:n_rows + 1]`` and
        ``slots[:entries]`` are rewritten in place on the stream, and the rows' new token counts are
        returned (a device view of this object's scratch, valid until the next call).

        ``keep`` bool / uint8 ``[rows, width]``: the committed blocks of each row; ``audit`` (uint8 /
        bool per row, or None): the rows read whole for this step's audit; ``active``: the lease holds;
        rows from ``n_real`` on are a graph's padding and read whole; ``entries`` = ``indptr[n_rows]``,
        which the host knows.  Entries of ``slots`` past the new list keep what they held."""
        if indptr.dtype != torch.int32 or indptr.stride(0) != 1:
            raise ValueError("indptr must be a contiguous int32 vector")
        if slots.dtype not in (torch.int32, torch.int64) or slots.stride(0) != 1:
            raise ValueError("slots must be a contiguous int32 or int64 vector")
        if keep.dtype not in (torch.bool, torch.uint8) or keep.dim() != 2 or keep.stride(1) != 1:
            raise ValueError("keep must be a [rows, width] bool / uint8 mask with contiguous rows")
        if n_rows > 0 and keep.shape[1] < self.width:
            raise ValueError(f"keep has {keep.shape[1]} blocks per row, the view {self.width}")
        if audit is not None and (audit.dtype not in (torch.bool, torch.uint8) or audit.stride(0) != 1):
            raise ValueError("audit must be a contiguous bool / uint8 vector")
        for name, t in (("indptr", indptr), ("slots", slots), ("keep", keep), ("audit", audit)):
            if t is not None and not t.is_cuda:
                raise ValueError(f"{name} must be a device tensor")
        self._room_for(max(n_rows, 1), max(entries, 1), slots.dtype)
        ekv_hip.call(
            "ekv_compact_slots",
            indptr.data_ptr(), slots.data_ptr(), slots.element_size(), keep.data_ptr(), keep.stride(0),
            ekv_hip.ptr(audit), int(bool(active)), int(n_real), int(n_rows), self.width, self.block_tokens,
            int(entries), self.new_indptr.data_ptr(), self.lens.data_ptr(), self.table.data_ptr(),
            self.table.stride(0), self._gathered.data_ptr(), self.counts.data_ptr(), 1, ekv_hip.stream_handle(),
        )
        return self.lens[:n_rows]
