"""The controller's keep rule on the device: which rows are measured, which blocks are pinned, how
large the budget is, and the ``uniform`` split of it (observe/controller.py:398-451).

``Controller._allocate`` walks the live rows on the host: a row is measured when it is longer than
``cap_above_blocks`` and its request has evidence; its first block, its ``recent_blocks`` newest
blocks and every block added since its audit are pinned; freed blocks leave the request; the
budget is ``max(pinned, ceil(fraction * total))`` over the measured rows' blocks, and
``allocate(..., objective)`` splits it.  ``uniform_keep_rows`` applies the same rule to device
arrays in one launch of ``ekv_rank_uniform``.  The controller's host loop, mailbox, leases and
step-time target stay host code and are not part of this module.
"""

from __future__ import annotations

import torch

from observe.allocation import uniform_keep


def uniform_keep_rows(
    shares: torch.Tensor,
    lengths: torch.Tensor,
    evidence: torch.Tensor,
    fraction: float,
    *,
    recent_blocks: int = 4,
    cap_above_blocks: int = 0,
    audited_blocks: torch.Tensor | None = None,
    released: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The keep mask ``uint8[rows, width]`` the controller commits under the ``uniform`` objective.

    ``shares`` float32 [rows, width]: each request's shares (zero past its evidence);
    ``lengths`` int32 [rows]: blocks per row; ``evidence`` bool [rows]: the row holds a request
    with shares; ``audited_blocks`` int32 [rows]: its length at its audit (blocks past it are
    pinned, observe/controller.py:423-424); ``released`` uint8 [rows, width]: freed blocks."""
    if not 0.0 < fraction <= 1.0:
        raise ValueError("the budget fraction must be in (0, 1]")
    if recent_blocks < 0 or cap_above_blocks < 0:
        raise ValueError("invalid controller settings")
    measured = (evidence.to(torch.bool) & (lengths > cap_above_blocks)).to(torch.uint8)  # controller.py:402-408
    blocks = torch.clamp(lengths, max=shares.shape[1]).to(torch.int32)
    return uniform_keep(
        shares,
        blocks,
        measured=measured,
        pin_from=audited_blocks,
        recent_blocks=recent_blocks,
        released=released,
        fraction=fraction,
        out=out,
        stream=stream,
    )
