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

``uniform`` ranks float32 scores by value -- for float32 scores that order is exactly the
reference's stable argsort of the float64 ``shares()`` -- and float64 scores by their float64 shares
``max(s, 0) / total`` themselves (``ekv_rank_uniform64``, the total being NumPy's pairwise sum), so
that two scores that divide to one share tie as they do in the reference.  ``allocate`` always takes
the float64 path.

Every device wrapper checks its tensors on the host (device, dtype, shape, contiguous rows) and
raises ``ValueError`` before any launch.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal

import numpy as np
import torch

import ekv_hip

Objective = Literal["sum", "maxmin", "uniform"]
_MASK_DTYPES = (torch.uint8, torch.bool)


def check_tensors(*specs) -> torch.device | None:
    """Refuse, with ValueError, tensors a kernel would misread.  ``specs`` are ``(name, tensor, dtypes,
    shape)``, ``tensor`` None for an absent optional one.  Every tensor's shape, dtype and row
    contiguity are checked first, then that all are on one GPU; returns that device."""
    present = [(name, t, dtypes, shape) for name, t, dtypes, shape in specs if t is not None]
    for name, t, dtypes, shape in present:
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"{name} must be a torch tensor")
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
        if t.dtype not in (dtypes if isinstance(dtypes, tuple) else (dtypes,)):
            raise ValueError(f"{name} must be {dtypes}, got {t.dtype}")
        if t.ndim and t.stride(-1) != 1:
            raise ValueError(f"{name} must have contiguous rows")
    device = None
    for name, t, _, _ in present:
        if not t.is_cuda:
            raise ValueError(f"{name} must be a device tensor")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{name} is on {t.device}, the others on {device}")
    return device


def _out(out: torch.Tensor | None, rows: int, width: int, device) -> torch.Tensor:
    if out is None:
        return torch.empty(rows, width, dtype=torch.uint8, device=device)
    if check_tensors(("out", out, torch.uint8, (rows, width))) != device:
        raise ValueError(f"out must be on {device}")
    return out


def _workspace(name: str, workspace: torch.Tensor | None, need: int, device) -> torch.Tensor:
    if workspace is None:
        return torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    if not (workspace.is_cuda and workspace.dtype == torch.uint8 and workspace.is_contiguous()):
        raise ValueError(f"{name} must be a contiguous uint8 device tensor")
    if workspace.device != device or workspace.numel() < need:
        raise ValueError(f"{name} must hold at least {need} bytes on {device}")
    return workspace


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


def _rows_width(scores) -> tuple[int, int]:
    if not isinstance(scores, torch.Tensor) or scores.ndim != 2:
        raise ValueError("scores must be a [rows, width] tensor")
    return int(scores.shape[0]), int(scores.shape[1])


def maxmin_keep(
    scores: torch.Tensor,
    blocks: torch.Tensor,
    *,
    budget: int,
    pinned: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The ``maxmin`` keep mask ``uint8[rows, width]`` on the device (observe/allocation.py:126-166)
    and the int64 summary (budget, blocks, pinned, status, requests, free); arguments as sum_keep.
    ``workspace``: a uint8 device tensor of at least ``maxmin_workspace_bytes(rows, width)`` bytes
    (allocated here when None)."""
    rows, width = _rows_width(scores)
    dev = check_tensors(("scores", scores, (torch.float32, torch.float64), (rows, width)),
                        ("blocks", blocks, torch.int32, (rows,)), ("pinned", pinned, _MASK_DTYPES, (rows, width)))
    scores = scores.double() if scores.dtype == torch.float32 else scores
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    out = _out(out, rows, width, dev)
    summary = torch.zeros(6, dtype=torch.int64, device=dev)
    need = maxmin_workspace_bytes(rows, width)
    workspace = _workspace("workspace", workspace, need, dev)
    ekv_hip.call(
        "ekv_rank_maxmin", scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(pinned),
        pinned.stride(0) if pinned is not None else 0, rows, width, int(budget), out.data_ptr(), out.stride(0),
        summary.data_ptr(), workspace.data_ptr(), workspace.numel(), ekv_hip.stream_handle(stream),
    )
    return out, summary


def maxmin_workspace_bytes(rows: int, width: int) -> int:
    """Device bytes ``maxmin_keep`` needs as its workspace."""
    return int(ekv_hip.load().ekv_rank_maxmin_workspace(int(rows), int(width)))


def sum_workspace_bytes(rows: int) -> int:
    """Device bytes ``sum_keep`` needs as its workspace."""
    return int(ekv_hip.load().ekv_rank_sum_workspace(int(rows)))


def sum_keep(
    scores: torch.Tensor,
    blocks: torch.Tensor,
    *,
    budget: int,
    weights: torch.Tensor | None = None,
    pinned: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The ``sum`` keep mask ``uint8[rows, width]`` on the device (observe/allocation.py:94-123) and
    the int64 summary (budget, blocks, pinned, status, requests, free).

    ``scores`` float64 [rows, width] (float32 is widened, exactly); ``blocks`` int32 [rows];
    ``weights`` float64 [rows] (default 1.0); ``pinned`` a uint8 / bool [rows, width] mask (default:
    the first and the last block of each row); ``workspace`` a uint8 device tensor of at least
    ``sum_workspace_bytes(rows)`` bytes (allocated here when None)."""
    rows, width = _rows_width(scores)
    dev = check_tensors(("scores", scores, (torch.float32, torch.float64), (rows, width)),
                        ("blocks", blocks, torch.int32, (rows,)), ("weights", weights, torch.float64, (rows,)),
                        ("pinned", pinned, _MASK_DTYPES, (rows, width)))
    scores = scores.double() if scores.dtype == torch.float32 else scores
    if budget < 0:
        raise ValueError("the budget cannot be negative")
    out = _out(out, rows, width, dev)
    summary = torch.zeros(6, dtype=torch.int64, device=dev)
    need = sum_workspace_bytes(rows)
    workspace = _workspace("workspace", workspace, need, dev)
    ekv_hip.call(
        "ekv_rank_sum", scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(weights),
        ekv_hip.ptr(pinned), pinned.stride(0) if pinned is not None else 0, rows, width, int(budget),
        out.data_ptr(), out.stride(0), summary.data_ptr(), workspace.data_ptr(), workspace.numel(),
        ekv_hip.stream_handle(stream),
    )
    return out, summary


def _uniform_on_device(requests: Sequence[Request], pinned: list[np.ndarray], budget: int) -> list[np.ndarray]:
    scores, pins, blocks, sizes = _padded(requests, pinned)
    keep = uniform_keep(scores, blocks, pinned=pins, budget=budget)[0].cpu().numpy()
    return [keep[i, : sizes[i]].astype(bool) for i in range(len(requests))]


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
    workspace: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The ``uniform`` keep mask ``uint8[rows, width]`` of every row, on the device, and the int64
    summary (budget, total, pinned floor, status, requests, free).

    ``scores`` float32 or float64 [rows, width] (float64 ranks the float64 shares); ``blocks`` int32
    [rows] blocks per row.  Pins are ``pinned`` when given (Request.pinned), else block 0, the
    ``recent_blocks`` newest after the last, and blocks >= ``pin_from`` (observe/controller.py:420-424).
    ``budget < 0`` takes the controller's ``max(floor, ceil(fraction * total))``
    (observe/controller.py:435-437).  ``workspace``: a uint8 device tensor of at least
    ``uniform_workspace_bytes(rows, scores.dtype)`` bytes (allocated here when None and needed)."""
    rows, width = _rows_width(scores)
    dev = check_tensors(("scores", scores, (torch.float32, torch.float64), (rows, width)),
                        ("blocks", blocks, torch.int32, (rows,)), ("measured", measured, _MASK_DTYPES, (rows,)),
                        ("pinned", pinned, _MASK_DTYPES, (rows, width)),
                        ("released", released, _MASK_DTYPES, (rows, width)),
                        ("pin_from", pin_from, torch.int32, (rows,)))
    out = _out(out, rows, width, dev)
    summary = torch.zeros(6, dtype=torch.int64, device=dev)
    wide = scores.dtype == torch.float64
    need = uniform_workspace_bytes(rows, scores.dtype) if (wide or pinned is not None or released is not None) else 0
    ws = _workspace("workspace", workspace, need, dev) if need else None
    common = (
        scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(measured),
        ekv_hip.ptr(pinned), pinned.stride(0) if pinned is not None else 0,
        ekv_hip.ptr(pin_from), int(recent_blocks),
        ekv_hip.ptr(released), released.stride(0) if released is not None else 0,
        rows, width, float(fraction), int(budget), out.data_ptr(), out.stride(0), summary.data_ptr(),
    )
    if wide:
        ekv_hip.call("ekv_rank_uniform64", *common, ws.data_ptr(), ws.numel(), ekv_hip.stream_handle(stream))
    else:
        ekv_hip.call("ekv_rank_uniform_ws", *common, ekv_hip.ptr(ws), ekv_hip.stream_handle(stream))
    return out, summary


def uniform_workspace_bytes(rows: int, dtype=torch.float32) -> int:
    """Device bytes ``uniform_keep`` needs as its workspace: the per-row totals of float64 scores
    and the mask counts (float32 scores need it only with pinned or released masks)."""
    if dtype == torch.float64:
        return int(ekv_hip.load().ekv_rank_uniform64_workspace(int(rows)))
    return 8 * max(int(rows), 1)
