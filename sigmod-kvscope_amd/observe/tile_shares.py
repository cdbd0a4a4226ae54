"""Attention share of each block, from the tile records the audit kernel writes.

On an audit step the recorder stores, per layer, request row, block and query row, the largest
score ``m`` of the block's tile and the sum ``l`` of ``exp(score - m)`` over the tile's keys,
in two planes ``[2][layer][row][block][query_row]`` (observe/tile_shares.py:1-17).  The log
weight of a block is ``u = m + log(l) - log(tile_blocks)``; an unwritten cell is NaN and a tile
with no keys has ``l = 0``, so ``u = -inf``.  Normalising ``u`` over the blocks of one
(layer, row, query row) gives the share of that query's attention on each block, and the shares
of a request's layers and query rows average to the request's share per block.

The normalisation runs on the GPU (``ekv_normalize_tile_lse`` / ``ekv_tile_shares``) in float32.
``read_tile_lse`` / ``read_tile_rows`` keep the reference's host-reader contract: they copy the
chosen rows through a ``cuda``-like object's ``d2h_many`` and return ``u`` on the host.
``tile_shares`` and ``DeviceTileShareSource`` compute the shares where the planes are, without
copying them.
"""

from __future__ import annotations

from typing import Literal

import numpy as np
import torch

import ekv_hip
from observe.zero_touch import pub_path, read_json_lines

Aggregate = Literal["mean", "max"]
_AGGREGATES = {"mean": ekv_hip.AGG_MEAN, "max": ekv_hip.AGG_MAX}


def share_descriptor(pid: int) -> dict[str, int | str]:
    """The statistic block of process ``pid`` with the tile size of the kernel recording into it
    (observe/tile_shares.py:26-52).  Of several recording kernels the narrowest tile wins (the decode
    kernel's).  Raises ``RuntimeError`` until one has published."""
    descriptors = pub_path(pid)
    coverage_path = descriptors.replace("ekv_pass_", "ekv_coverage_")
    tile_of = {int(rec.get("host_va", 0) or 0): rec for rec in read_json_lines(coverage_path)}
    found = []
    for rec in read_json_lines(descriptors):
        if not int(rec.get("tile_lse_dev", 0)):
            continue
        tile = int(tile_of.get(int(rec["host_va"]), {}).get("attn_share_tile_blocks", 0))
        if tile:
            found.append(dict(rec, attn_share_tile_blocks=tile))
    if not found:
        raise RuntimeError(f"process {pid} has not compiled a kernel that records the attention statistic")
    return min(found, key=lambda rec: int(rec["attn_share_tile_blocks"]))


def _aggregate_code(aggregate: str) -> int:
    if aggregate not in _AGGREGATES:
        raise ValueError(f"unknown aggregate {aggregate!r}")
    return _AGGREGATES[aggregate]


def normalize_tile_lse(
    lse, row_blocks, tile_blocks: int, aggregate: Aggregate = "mean"
):
    """The attention share per (row, block) from ``lse[layer, row, block, query_row]``
    (observe/tile_shares.py:58-103), computed on the GPU.

    A partial last tile gives its weight back to the blocks that exist, cells past the row are
    dropped, each (layer, query row) with a finite value is one share vector, and the result is
    their mean (or the renormalised per-block max).  A row with no finite value is all NaN.
    A NumPy input gives a float64 NumPy result; a device tensor gives a float32 device tensor.
    """
    code = _aggregate_code(aggregate)
    on_device = isinstance(lse, torch.Tensor) and lse.is_cuda
    if lse.ndim != 4:
        raise ValueError("lse must be [layers, rows, blocks, query_rows]")
    layers, rows, width, cells = (int(x) for x in lse.shape)
    blocks_host = row_blocks.cpu().numpy() if isinstance(row_blocks, torch.Tensor) else np.asarray(row_blocks)
    if blocks_host.shape != (rows,) or tile_blocks < 1:
        raise ValueError("row_blocks must give one length per row, and tile_blocks must be positive")
    if on_device:
        u = lse.to(torch.float32).contiguous()
    else:
        u = torch.from_numpy(np.ascontiguousarray(lse, dtype=np.float32)).cuda()
    lengths = torch.from_numpy(blocks_host.astype(np.int32)).to(u.device)
    out = torch.empty(rows, width, dtype=torch.float32, device=u.device)
    if rows and width and layers:
        ekv_hip.call(
            "ekv_normalize_tile_lse",
            u.data_ptr(), rows * width * cells, width * cells, layers, cells, width,
            lengths.data_ptr(), rows, int(tile_blocks), code, out.data_ptr(), width,
            ekv_hip.stream_handle(),
        )
    elif rows:
        out.fill_(float("nan"))
    if on_device:
        return out
    return out.cpu().numpy().astype(np.float64)


def read_tile_lse(
    cuda: object,
    base: int,
    table_layers: int,
    layers: int,
    rows: int,
    width: int,
    group_rows: int,
    live_rows: int,
    tile_blocks: int,
) -> np.ndarray:
    """``u[layers, live_rows, width, group_rows]`` of the first ``live_rows`` rows (observe/tile_shares.py:106-126)."""
    return read_tile_rows(cuda, base, table_layers, layers, rows, width, group_rows, np.arange(live_rows), tile_blocks)


def read_tile_rows(
    cuda: object,
    base: int,
    table_layers: int,
    layers: int,
    rows: int,
    width: int,
    group_rows: int,
    row_ids: np.ndarray,
    tile_blocks: int,
) -> np.ndarray:
    """``u[layers, len(row_ids), width, group_rows]`` of the ascending rows ``row_ids``
    (observe/tile_shares.py:129-173): one ``d2h_many`` request per run of adjacent rows in each
    layer of each plane, so the copy follows the rows asked for."""
    row_ids = np.asarray(row_ids)
    if row_ids.size > 1 and np.any(row_ids[1:] <= row_ids[:-1]):
        raise ValueError("row_ids must be ascending and distinct")
    row_bytes = width * group_rows * 4
    layer_bytes = rows * row_bytes
    plane_bytes = table_layers * layer_bytes
    runs: list[tuple[int, int]] = []
    for r in row_ids.tolist():
        if runs and runs[-1][0] + runs[-1][1] == r:
            runs[-1] = (runs[-1][0], runs[-1][1] + 1)
        else:
            runs.append((r, 1))
    requests = [
        (base + plane * plane_bytes + layer * layer_bytes + first * row_bytes, count * row_bytes)
        for plane in (0, 1)
        for layer in range(layers)
        for first, count in runs
    ]
    blobs = cuda.d2h_many(requests)  # type: ignore[attr-defined]
    per_layer = len(runs)
    planes = []
    for plane in (0, 1):
        per = []
        for layer in range(layers):
            start = (plane * layers + layer) * per_layer
            joined = b"".join(blobs[start : start + per_layer])
            per.append(np.frombuffer(joined, dtype=np.float32).reshape(len(row_ids), width, group_rows))
        planes.append(np.stack(per) if per else np.zeros((0, len(row_ids), width, group_rows), np.float32))
    m, total = planes
    with np.errstate(divide="ignore", invalid="ignore"):  # l = 0 has weight exp(-inf) = 0
        return m + np.log(total) - np.float32(np.log(tile_blocks))


def tile_shares(
    base: int,
    table_layers: int,
    layers: int,
    rows: int,
    width: int,
    group_rows: int,
    row_ids: torch.Tensor | None,
    row_blocks: torch.Tensor | None,
    tile_blocks: int,
    aggregate: Aggregate = "mean",
    out: torch.Tensor | None = None,
    stream=None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Shares ``float32[len(row_ids), width]`` of the chosen rows straight from the device planes at
    ``base`` (read_tile_rows + normalize_tile_lse fused on the GPU; nothing is copied to the host).

    ``row_ids`` / ``row_blocks`` are int32 device tensors (None: every row / full width).  The rows'
    layers are split over several workgroups through a device workspace (``workspace``, a uint8
    device tensor of at least ``shares_workspace_bytes`` bytes, zero-filled before its first use and
    not written by anything else between calls; or one allocated here)."""
    code = _aggregate_code(aggregate)
    n = rows if row_ids is None else int(row_ids.shape[0])
    if out is None:
        out = torch.empty(n, width, dtype=torch.float32, device="cuda")
    if out.shape != (n, width) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be float32 [rows, width] with contiguous rows")
    for t in (row_ids, row_blocks):
        if t is not None and (t.dtype != torch.int32 or not t.is_cuda or t.stride(0) != 1):
            raise ValueError("row_ids and row_blocks must be contiguous int32 device tensors")
    layer_stride = rows * width * group_rows
    need = shares_workspace_bytes(n, width, layers)
    if workspace is None:
        workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=out.device)
    if workspace.dtype != torch.uint8 or not workspace.is_cuda or workspace.numel() < need:
        raise ValueError(f"workspace must be a uint8 device tensor of at least {need} bytes")
    ekv_hip.call(
        "ekv_tile_shares_ws",
        int(base), table_layers * layer_stride, layer_stride, width * group_rows, layers, group_rows, width,
        ekv_hip.ptr(row_ids), ekv_hip.ptr(row_blocks), n, int(tile_blocks), code, out.data_ptr(), out.stride(0),
        workspace.data_ptr(), workspace.numel(), ekv_hip.stream_handle(stream),
    )
    return out


def shares_workspace_bytes(rows: int, width: int, layers: int) -> int:
    """Device bytes ``tile_shares`` needs as its workspace for ``rows`` output rows."""
    return int(ekv_hip.load().ekv_tile_shares_workspace(int(rows), int(width), int(layers)))


def check_workspace(workspace: torch.Tensor | None) -> None:
    """Raise ``RuntimeError`` when a call on ``workspace`` (None: this device's scratch of the
    allocation-free form) lost a partial: its rows came out as NaN and the slot may have been
    written after the call.  The workspace is reset first, so the next call runs on a sound one.
    Waits for the device."""
    import ctypes

    status = ctypes.c_int32(0)
    address = 0 if workspace is None else workspace.data_ptr()
    ekv_hip.call("ekv_tile_shares_status", address, ctypes.byref(status))
    if status.value == 0:
        return
    ekv_hip.call("ekv_tile_shares_reset", address, 0 if workspace is None else workspace.numel(), 0)
    ekv_hip.synchronize()
    raise RuntimeError("a share partial never reached the workgroup that adds a row's partials: those rows are "
                       "NaN; the workspace has been reset")


class DeviceTileShareSource:
    """Reads the live rows' shares with the normalisation on the device.

    It answers ``read(live_rows, row_blocks)`` as the controller's ``TileShareSource.read``
    (observe/controller.py:92-136) does -- NaN rows without evidence, rows of 0 blocks not read --
    but copies only the ``[rows, width]`` float32 shares to the host, not both planes of every layer."""

    def __init__(self, cuda: object, entry: dict[str, int | str], pid: int, aggregate: Aggregate = "mean") -> None:
        import os

        self.aggregate = aggregate
        self.cuda = cuda
        self.rows = int(entry["max_rows"])
        self.width = int(entry["ncap"])
        self.group_rows = int(entry["tile_lse_group_rows"])
        self.max_layers = int(entry["tile_lse_layers"])
        self.tile_blocks = int(entry["attn_share_tile_blocks"])
        local = pid == os.getpid()
        self.base = int(entry["tile_lse_dev"]) if local else cuda.ipc_open(str(entry["tile_lse_ipc"]))  # type: ignore[attr-defined]
        self.table = int(entry["layer_table_dev"]) if local else cuda.ipc_open(str(entry["layer_table_ipc"]))  # type: ignore[attr-defined]
        # buffers for the most rows a read can ask for, allocated once: every read reuses them
        self._ids = torch.empty(self.rows, dtype=torch.int32, device="cuda")
        self._lengths = torch.empty(self.rows, dtype=torch.int32, device="cuda")
        self._out = torch.empty(self.rows, self.width, dtype=torch.float32, device="cuda")
        self._staging = torch.empty(2, self.rows, dtype=torch.int32, pin_memory=True)
        need = shares_workspace_bytes(self.rows, self.width, self.max_layers)
        self._workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")

    def read(self, live_rows: int, row_blocks: np.ndarray) -> np.ndarray:
        raw = self.cuda.d2h(self.table, self.max_layers * 8)  # type: ignore[attr-defined]
        layers = int(np.count_nonzero(np.frombuffer(raw, dtype=np.uint64)))
        if layers == 0:
            raise RuntimeError("the layer table is empty: the serving process has not filled it")
        if not 0 <= live_rows <= self.rows:
            raise ValueError(f"{live_rows} live rows, the plane holds {self.rows}")
        shares = np.full((live_rows, self.width), np.nan)
        wanted = np.flatnonzero(np.asarray(row_blocks[:live_rows]) > 0)
        if wanted.size == 0:
            return shares
        k = int(wanted.size)
        staged = self._staging.numpy()
        staged[0, :k] = wanted
        staged[1, :k] = np.asarray(row_blocks)[wanted]
        ids, lengths, out = self._ids[:k], self._lengths[:k], self._out[:k]
        ids.copy_(self._staging[0, :k], non_blocking=True)
        lengths.copy_(self._staging[1, :k], non_blocking=True)
        tile_shares(
            self.base, self.max_layers, layers, self.rows, self.width, self.group_rows, ids, lengths,
            self.tile_blocks, self.aggregate, out=out, workspace=self._workspace,
        )
        shares[wanted] = out.cpu().numpy()  # waits for the copies and the kernels
        check_workspace(self._workspace)
        return shares
