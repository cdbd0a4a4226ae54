"""The controller's keep rule on the device: which rows are measured, which blocks are pinned, how
large the budget is, and its split under each objective (observe/controller.py:398-451).

``Controller._allocate`` walks the live rows on the host: a row is measured when it is longer than
``cap_above_blocks`` and its request has evidence; its first block, its ``recent_blocks`` newest
blocks and every block added since its audit are pinned; freed blocks leave the request; the
budget is ``max(pinned, ceil(fraction * total))`` over the measured rows' blocks, and
``allocate(..., objective)`` splits it.  ``keep_rows`` applies the same rule to device arrays for
each objective: ``uniform`` in one launch of ``ekv_rank_uniform`` (``uniform_keep_rows``), ``sum``
(``Settings.objective``'s default, observe/controller.py:30) and ``maxmin`` through
``ekv_controller_keep``, which gives each measured row's remaining blocks to the objective as one
request, the requests numbered in row order.  The controller's host loop, mailbox, leases and
step-time target stay host code and are not part of this module.
"""

from __future__ import annotations

import torch

import ekv_hip
from observe.allocation import _MASK_DTYPES, Objective, _workspace, check_tensors, uniform_keep

_OBJECTIVE_CODES = {"sum": ekv_hip.OBJ_SUM, "maxmin": ekv_hip.OBJ_MAXMIN}


def keep_rows(
    shares: torch.Tensor,
    lengths: torch.Tensor,
    evidence: torch.Tensor,
    fraction: float,
    *,
    objective: Objective = "sum",
    recent_blocks: int = 4,
    cap_above_blocks: int = 0,
    audited_blocks: torch.Tensor | None = None,
    released: torch.Tensor | None = None,
    weights: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The keep mask ``uint8[rows, width]`` the controller commits (observe/controller.py:398-451)
    and the int64 summary (budget, blocks, pinned, status, requests, free).

    Arguments as ``uniform_keep_rows``; ``shares`` float32 or float64; ``weights`` float64 [rows]:
    each row's request weight (``Controller.weight``, observe/controller.py:430), ``sum`` only.
    ``workspace``: a uint8 device tensor of at least ``keep_rows_workspace_bytes(objective, rows,
    width)`` bytes (allocated here when None; ``uniform`` needs none without ``released``)."""
    if objective == "uniform":
        if weights is not None:
            raise ValueError("the uniform objective does not use request weights")
        return uniform_keep_rows(shares, lengths, evidence, fraction, recent_blocks=recent_blocks,
                                 cap_above_blocks=cap_above_blocks, audited_blocks=audited_blocks,
                                 released=released, out=out, stream=stream)
    if objective not in _OBJECTIVE_CODES:
        raise ValueError(f"unknown objective {objective!r}")
    if objective == "maxmin" and weights is not None:
        raise ValueError("the maxmin objective does not use request weights")
    if not 0.0 < fraction <= 1.0:
        raise ValueError("the budget fraction must be in (0, 1]")
    if recent_blocks < 0 or cap_above_blocks < 0:
        raise ValueError("invalid controller settings")
    if not isinstance(shares, torch.Tensor) or shares.ndim != 2:
        raise ValueError("shares must be a [rows, width] tensor")
    rows, width = int(shares.shape[0]), int(shares.shape[1])
    dev = check_tensors(("shares", shares, (torch.float32, torch.float64), (rows, width)),
                        ("lengths", lengths, torch.int32, (rows,)), ("evidence", evidence, _MASK_DTYPES, (rows,)),
                        ("audited_blocks", audited_blocks, torch.int32, (rows,)),
                        ("released", released, _MASK_DTYPES, (rows, width)),
                        ("weights", weights, torch.float64, (rows,)))
    if out is None:
        out = torch.empty(rows, width, dtype=torch.uint8, device=dev)
    elif check_tensors(("out", out, torch.uint8, (rows, width))) != dev:
        raise ValueError(f"out must be on {dev}")
    summary = torch.zeros(6, dtype=torch.int64, device=dev)
    code = _OBJECTIVE_CODES[objective]
    ws = _workspace("workspace", workspace, keep_rows_workspace_bytes(objective, rows, width), dev)
    ekv_hip.call(
        "ekv_controller_keep", code, shares.data_ptr(),
        ekv_hip.F64 if shares.dtype == torch.float64 else ekv_hip.F32, shares.stride(0),
        lengths.data_ptr(), evidence.data_ptr(), ekv_hip.ptr(audited_blocks), ekv_hip.ptr(released),
        released.stride(0) if released is not None else 0, ekv_hip.ptr(weights), rows, width, int(recent_blocks),
        int(cap_above_blocks), float(fraction), out.data_ptr(), out.stride(0), summary.data_ptr(), ws.data_ptr(),
        ws.numel(), ekv_hip.stream_handle(stream),
    )
    return out, summary


def keep_rows_workspace_bytes(objective: Objective, rows: int, width: int) -> int:
    """Device bytes ``keep_rows`` needs as its workspace under ``sum`` or ``maxmin``."""
    if objective not in _OBJECTIVE_CODES:
        raise ValueError(f"no workspace for objective {objective!r}")
    return int(ekv_hip.load().ekv_controller_keep_workspace(_OBJECTIVE_CODES[objective], int(rows), int(width)))


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
