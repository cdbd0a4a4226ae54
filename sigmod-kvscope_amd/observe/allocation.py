"""Allocate a read budget across requests by the attention each block carries (observe/allocation.py:1-19).

Each request scores each of its blocks by the share of its attention on the block.  ``uniform``
gives every request the same fraction of its unpinned blocks, each ranked by its own shares:
the free budget is split by largest remainder in IEEE double and each request keeps its quota of
open blocks by (share descending, block index ascending) (``ekv_rank_uniform``).  ``sum`` keeps the
free budget's unpinned blocks of highest weight * share over all requests, a tie going to the newer
block, then the earlier request (``ekv_rank_sum``, float64 shares with NumPy's totals).  ``maxmin``
raises the lowest retained share by the reference's bisection of the level and gives the leftover
to the lowest request first (``ekv_rank_maxmin``).  Pinned
blocks (by default the first and the last) always count against the budget, and a budget below
them is an error.

The device ranks float32 shares.  For float32 scores that order is exactly the reference's stable
argsort of the float64 ``shares()``; float64 scores are rounded to float32 first.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal

import numpy as np
import torch

import ekv_hip

Objective = Literal["sum", "maxmin", "uniform"]


@dataclass(frozen=True)
class Request:
    """One request: the score of each block, how much its retained share counts, its pinned blocks
    (observe/allocation.py:31-52)."""

    scores: np.ndarray
    weight: float = 1.0
    pinned: np.ndarray | None = None

    def pinned_mask(self) -> np.ndarray:
        if self.pinned is not None:
            return np.asarray(self.pinned, dtype=bool)
        mask = np.zeros(len(self.scores), dtype=bool)
        if len(self.scores):
            mask[0] = mask[-1] = True
        return mask

    def shares(self) -> np.ndarray:
        """Scores clamped at 0 and normalised to sum to 1; equal shares without evidence."""
        clamped = np.maximum(np.asarray(self.scores, dtype=np.float64), 0.0)
        total = clamped.sum()
        if total <= 0.0:
            return np.full(len(clamped), 1.0 / max(len(clamped), 1))
        return clamped / total


def allocate(requests: Sequence[Request], budget: int, objective: Objective = "sum") -> list[np.ndarray]:
    """A bool keep mask per request; at most ``budget`` blocks are kept (observe/allocation.py:55-76)."""
    sizes = [len(r.scores) for r in requests]
    pinned = [r.pinned_mask() for r in requests]
    if any(len(p) != n for p, n in zip(pinned, sizes)):
        raise ValueError("a pinned mask must have one entry per block")
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    must = sum(int(p.sum()) for p in pinned)
    if must > budget and budget < sum(sizes):
        raise ValueError(f"the budget {budget} cannot hold the {must} pinned blocks")
    if budget >= sum(sizes):
        return [np.ones(n, dtype=bool) for n in sizes]
    if objective in ("maxmin", "uniform") and any(r.weight != 1.0 for r in requests):
        raise ValueError(f"the {objective} objective does not use request weights")
    if objective == "uniform":
        return _uniform_on_device(requests, pinned, budget)
    if objective == "sum":
        return _sum_on_device(requests, pinned, budget)
    if objective == "maxmin":
        return _maxmin_on_device(requests, pinned, budget)
    raise ValueError(f"unknown objective {objective!r}")


def _padded(requests: Sequence[Request], pinned: list[np.ndarray]):
    """Scores (float64), pins and block counts of the requests as [rows, width] device tensors."""
    rows = len(requests)
    sizes = [len(r.scores) for r in requests]
    width = max(max(sizes, default=1), 1)
    scores = np.zeros((rows, width), dtype=np.float64)
    pins = np.zeros((rows, width), dtype=np.uint8)
    for i, (req, pin) in enumerate(zip(requests, pinned)):
        scores[i, : sizes[i]] = np.asarray(req.scores, dtype=np.float64)
        pins[i, : sizes[i]] = pin
    return (torch.from_numpy(scores).cuda(), torch.from_numpy(pins).cuda(),
            torch.tensor(sizes, dtype=torch.int32).cuda(), sizes)


def _sum_on_device(requests: Sequence[Request], pinned: list[np.ndarray], budget: int) -> list[np.ndarray]:
    scores, pins, blocks, sizes = _padded(requests, pinned)
    weights = torch.tensor([float(r.weight) for r in requests], dtype=torch.float64).cuda()
    keep = sum_keep(scores, blocks, weights=weights, pinned=pins, budget=budget)[0].cpu().numpy()
    return [keep[i, : sizes[i]].astype(bool) for i in range(len(requests))]


def _maxmin_on_device(requests: Sequence[Request], pinned: list[np.ndarray], budget: int) -> list[np.ndarray]:
    scores, pins, blocks, sizes = _padded(requests, pinned)
    keep = maxmin_keep(scores, blocks, pinned=pins, budget=budget)[0].cpu().numpy()
    return [keep[i, : sizes[i]].astype(bool) for i in range(len(requests))]


def maxmin_keep(
    scores: torch.Tensor,
    blocks: torch.Tensor,
    *,
    budget: int,
    pinned: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The ``maxmin`` keep mask ``uint8[rows, width]`` on the device (observe/allocation.py:126-166)
    and the int64 summary (budget, blocks, pinned, status, requests, free); arguments as sum_keep."""
    if scores.dtype == torch.float32:
        scores = scores.double()
    if scores.dtype != torch.float64 or scores.stride(1) != 1:
        raise ValueError("scores must be float64 (or float32) with contiguous rows")
    rows, width = int(scores.shape[0]), int(scores.shape[1])
    if blocks.dtype != torch.int32 or blocks.shape != (rows,):
        raise ValueError("blocks must be int32 [rows]")
    if pinned is not None and (pinned.dtype not in (torch.uint8, torch.bool) or pinned.stride(-1) != 1):
        raise ValueError("pinned must be a uint8 / bool mask with contiguous rows")
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    if out is None:
        out = torch.empty(rows, width, dtype=torch.uint8, device=scores.device)
    summary = torch.zeros(6, dtype=torch.int64, device=scores.device)
    need = int(ekv_hip.load().ekv_rank_maxmin_workspace(rows, width))
    workspace = torch.empty(need, dtype=torch.uint8, device=scores.device)
    ekv_hip.call(
        "ekv_rank_maxmin", scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(pinned),
        pinned.stride(0) if pinned is not None else 0, rows, width, int(budget), out.data_ptr(), out.stride(0),
        summary.data_ptr(), workspace.data_ptr(), need, ekv_hip.stream_handle(stream),
    )
    return out, summary


def sum_keep(
    scores: torch.Tensor,
    blocks: torch.Tensor,
    *,
    budget: int,
    weights: torch.Tensor | None = None,
    pinned: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The ``sum`` keep mask ``uint8[rows, width]`` on the device (observe/allocation.py:94-123) and
    the int64 summary (budget, blocks, pinned, status, requests, free).

    ``scores`` float64 [rows, width] (float32 is widened, exactly); ``blocks`` int32 [rows];
    ``weights`` float64 [rows] (default 1.0); ``pinned`` a uint8 / bool mask (default: the first
    and the last block of each row)."""
    if scores.dtype == torch.float32:
        scores = scores.double()
    if scores.dtype != torch.float64 or scores.stride(1) != 1:
        raise ValueError("scores must be float64 (or float32) with contiguous rows")
    rows, width = int(scores.shape[0]), int(scores.shape[1])
    if blocks.dtype != torch.int32 or blocks.shape != (rows,):
        raise ValueError("blocks must be int32 [rows]")
    if weights is not None and (weights.dtype != torch.float64 or weights.shape != (rows,)):
        raise ValueError("weights must be float64 [rows]")
    if pinned is not None and (pinned.dtype not in (torch.uint8, torch.bool) or pinned.stride(-1) != 1):
        raise ValueError("pinned must be a uint8 / bool mask with contiguous rows")
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    if out is None:
        out = torch.empty(rows, width, dtype=torch.uint8, device=scores.device)
    summary = torch.zeros(6, dtype=torch.int64, device=scores.device)
    need = int(ekv_hip.load().ekv_rank_sum_workspace(rows))
    workspace = torch.empty(need, dtype=torch.uint8, device=scores.device)
    ekv_hip.call(
        "ekv_rank_sum", scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(weights),
        ekv_hip.ptr(pinned), pinned.stride(0) if pinned is not None else 0, rows, width, int(budget),
        out.data_ptr(), out.stride(0), summary.data_ptr(), workspace.data_ptr(), need,
        ekv_hip.stream_handle(stream),
    )
    return out, summary


def _uniform_on_device(requests: Sequence[Request], pinned: list[np.ndarray], budget: int) -> list[np.ndarray]:
    rows = len(requests)
    sizes = [len(r.scores) for r in requests]
    width = max(max(sizes, default=1), 1)
    scores = np.zeros((rows, width), dtype=np.float32)
    pins = np.zeros((rows, width), dtype=np.uint8)
    for i, (req, pin) in enumerate(zip(requests, pinned)):
        scores[i, : sizes[i]] = np.asarray(req.scores, dtype=np.float32)
        pins[i, : sizes[i]] = pin
    keep = uniform_keep(
        torch.from_numpy(scores).cuda(),
        torch.tensor(sizes, dtype=torch.int32).cuda(),
        pinned=torch.from_numpy(pins).cuda(),
        budget=budget,
    )[0].cpu().numpy()
    return [keep[i, : sizes[i]].astype(bool) for i in range(rows)]


def uniform_keep(
    scores: torch.Tensor,
    blocks: torch.Tensor,
    *,
    measured: torch.Tensor | None = None,
    pinned: torch.Tensor | None = None,
    pin_from: torch.Tensor | None = None,
    recent_blocks: int = 0,
    released: torch.Tensor | None = None,
    fraction: float = 1.0,
    budget: int = -1,
    out: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The ``uniform`` keep mask ``uint8[rows, width]`` of every row, on the device, and the int64
    summary (budget, total, pinned floor, status, requests, free).

    ``scores`` float32 [rows, width]; ``blocks`` int32 [rows] blocks per row.  Pins are ``pinned``
    when given (Request.pinned), else block 0, the ``recent_blocks`` newest after the last, and
    blocks >= ``pin_from`` (observe/controller.py:420-424).  ``budget < 0`` takes the controller's
    ``max(floor, ceil(fraction * total))`` (observe/controller.py:435-437)."""
    rows, width = int(scores.shape[0]), int(scores.shape[1])
    if scores.dtype != torch.float32 or scores.stride(1) != 1:
        raise ValueError("scores must be float32 with contiguous rows")
    if blocks.dtype != torch.int32 or blocks.shape != (rows,):
        raise ValueError("blocks must be int32 [rows]")
    for name, t in (("measured", measured), ("pinned", pinned), ("released", released)):
        if t is not None and (t.dtype not in (torch.uint8, torch.bool) or t.stride(-1) != 1):
            raise ValueError(f"{name} must be a uint8 / bool mask with contiguous rows")
    if measured is not None and measured.shape != (rows,):
        raise ValueError("measured must be [rows]")
    for name, t in (("pinned", pinned), ("released", released)):
        if t is not None and t.shape != (rows, width):
            raise ValueError(f"{name} must be [rows, width] like scores")
    if pin_from is not None and (pin_from.dtype != torch.int32 or pin_from.shape != (rows,)):
        raise ValueError("pin_from must be int32 [rows]")
    if out is None:
        out = torch.empty(rows, width, dtype=torch.uint8, device=scores.device)
    summary = torch.zeros(6, dtype=torch.int64, device=scores.device)
    workspace = None
    if pinned is not None or released is not None:
        workspace = torch.empty(2 * max(rows, 1), dtype=torch.int32, device=scores.device)
    ekv_hip.call(
        "ekv_rank_uniform_ws",
        scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(measured),
        ekv_hip.ptr(pinned), pinned.stride(0) if pinned is not None else 0,
        ekv_hip.ptr(pin_from), int(recent_blocks),
        ekv_hip.ptr(released), released.stride(0) if released is not None else 0,
        rows, width, float(fraction), int(budget), out.data_ptr(), out.stride(0), summary.data_ptr(),
        ekv_hip.ptr(workspace), ekv_hip.stream_handle(stream),
    )
    return out, summary
