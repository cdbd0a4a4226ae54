"""The attention-share statistic recorded by an audit kernel of its own, for any attention backend.

After each attention layer of an audit step, the HIP kernel ``ekv_audit_tile_lse`` records

  m[layer][row][block][query row] = the largest score over the keys of the block's tile
  l[layer][row][block][query row] = the sum of exp(score - m) over those keys

for the query rows of one KV group per layer (layer L records group L mod groups), only for the
rows selected for the step, as runtime/audit_kernel.py:1-17 describes.  The layout, units and
descriptor files are the reference's, so ``observe.tile_shares`` reads either.  Constructed with
``kv_heads``, the plane records every KV head of every layer instead (``cells`` =
kv_heads * group_rows query rows per block), which the same readers average over.

With a timer (``timer=True`` or ``EKV_TIMER`` set) every audit launch also adds, per row, the
cycles its work took (``s_memtime``) into a cumulative device ``uint64[rows]`` published as
``timer_dev`` / ``timer_ipc``: the per-row cycle accumulator the pass's timer keeps
(mlir_pass/lib/eKVTimer.cpp:1348-1387, read as observe/cycles.py:1-45 describes).
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

import ekv_hip
from observe.zero_touch import pub_path
from runtime.audit import AuditPlane

TILE_BLOCKS = 2  # blocks per tile: one value is recorded per tile (runtime/audit_kernel.py:31)


def _enabled(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0", "false")


class RecordingPlane(AuditPlane):
    """An audit plane whose statistic block is allocated here and recorded by ``ekv_audit_tile_lse``
    (runtime/audit_kernel.py:123-265)."""

    def __init__(
        self,
        layers: int,
        rows: int,
        width: int,
        group_rows: int,
        block_size: int,
        *,
        kv_heads: int | None = None,
        timer: bool | None = None,
    ) -> None:
        super().__init__()
        if group_rows > 16:
            raise ValueError(f"{group_rows} query heads per KV head: the kernel handles at most 16")
        tile_tokens = block_size * TILE_BLOCKS
        if tile_tokens & (tile_tokens - 1):
            raise ValueError("a tile of the audit kernel must hold a power of two of tokens")
        if min(layers, rows, width, group_rows, block_size) <= 0 or (kv_heads is not None and kv_heads <= 0):
            raise ValueError("plane dimensions must be positive")
        self._layers = layers
        self.rows, self.width, self.group_rows, self.block_size = rows, width, group_rows, block_size
        self.kv_heads = kv_heads
        self.cells = group_rows * (kv_heads or 1)  # query rows recorded per block
        self._layer_of: dict[str, int] = {}  # layer name -> number, in the order the layers first run
        self.lse_bytes = 2 * layers * rows * width * self.cells * 4  # plane 0 the tile max, plane 1 the sum
        self._lse = self._allocate(self.lse_bytes)
        ekv_hip.memset(self._lse, 0xFF, self.lse_bytes)  # NaN: unwritten
        self._flag_dev = self._allocate(4)
        self._table_dev = self._allocate(layers * 8)
        ekv_hip.memset(self._flag_dev, 0, 4)
        ekv_hip.memset(self._table_dev, 0, layers * 8)
        self._select = torch.zeros(rows, dtype=torch.uint8, device="cuda")
        self._token = torch.zeros(rows, dtype=torch.int32, device="cuda")
        # the step plan: the work list of the step's launches, built at its first layer
        self._plan_bytes = int(ekv_hip.load().ekv_audit_plan_bytes(rows, width))
        self._plan = self._allocate(self._plan_bytes) if self._plan_bytes else 0
        if self._plan:
            ekv_hip.memset(self._plan, 0, self._plan_bytes)  # an empty plan until the first is built
        self.timer = _enabled("EKV_TIMER") if timer is None else bool(timer)
        self._cycles_dev = 0
        if self.timer:
            self._cycles_dev = self._allocate(rows * 8)
            ekv_hip.memset(self._cycles_dev, 0, rows * 8)  # zeroed once; cumulative afterwards
        self._publish()

    # -- device memory and descriptors --------------------------------------------------------

    def _allocate(self, size: int) -> int:
        """Device memory the plane holds for the life of the process (stable addresses for graphs)."""
        try:
            return ekv_hip.malloc(size)
        except (RuntimeError, ValueError) as err:
            raise RuntimeError(f"hipMalloc of {size} bytes failed: {err}") from err

    def _ipc(self, address: int) -> str:
        return ekv_hip.ipc_handle(address).hex()

    def _publish(self) -> None:
        """Append the descriptor records the controller reads (runtime/audit_kernel.py:160-180)."""
        entry = {
            "host_va": self._lse,
            "ncap": self.width,
            "max_rows": self.rows,
            "tile_lse_dev": self._lse,
            "tile_lse_ipc": self._ipc(self._lse),
            "tile_lse_layers": self._layers,
            "tile_lse_group_rows": self.cells,
            "stat_flag_dev": self._flag_dev,
            "layer_table_dev": self._table_dev,
            "layer_table_ipc": self._ipc(self._table_dev),
        }
        if self._cycles_dev:
            entry["timer_dev"] = self._cycles_dev
            entry["timer_ipc"] = self._ipc(self._cycles_dev)
            entry["kernel"] = "ekv_audit_tile_lse"
        path = pub_path(self.pid)
        with open(path, "a") as f:
            f.write(json.dumps(entry) + "\n")
        os.chmod(path, 0o600)
        coverage = {"host_va": self._lse, "attn_share_tile_blocks": TILE_BLOCKS}
        with open(path.replace("ekv_pass_", "ekv_coverage_"), "a") as f:
            f.write(json.dumps(coverage) + "\n")

    def _discover(self) -> bool:
        return True  # the block exists from construction

    @property
    def strides(self) -> tuple[int, int, int]:
        """Element strides of the statistic block: (plane, layer, row)."""
        row = self.width * self.cells
        layer = self.rows * row
        return self._layers * layer, layer, row

    @property
    def lse_address(self) -> int:
        return self._lse

    @property
    def cycles_address(self) -> int:
        return self._cycles_dev

    def read_planes(self) -> np.ndarray:
        """A host copy of both planes, ``float32[2, layers, rows, width, cells]``."""
        raw = ekv_hip.d2h(self._lse, self.lse_bytes)
        return np.frombuffer(raw, dtype=np.float32).reshape(2, self._layers, self.rows, self.width, self.cells)

    def read_cycles(self) -> np.ndarray:
        """A host copy of the per-row cycle accumulator (zeros when there is no timer)."""
        if not self._cycles_dev:
            return np.zeros(self.rows, dtype=np.uint64)
        return np.frombuffer(ekv_hip.d2h(self._cycles_dev, self.rows * 8), dtype=np.uint64).copy()

    def clear(self, layer: int | None = None) -> None:
        """Mark every cell (or those of one layer) unwritten again (NaN)."""
        plane, layer_stride, _row = self.strides
        if layer is None:
            ekv_hip.memset(self._lse, 0xFF, self.lse_bytes)
            return
        for p in (0, 1):
            ekv_hip.memset(self._lse + 4 * (p * plane + layer * layer_stride), 0xFF, 4 * layer_stride)

    # -- the engine-facing protocol ---------------------------------------------------------

    @property
    def layer_names(self) -> list[str]:
        """The attention layers in the order they first ran, which is their layer number."""
        return sorted(self._layer_of, key=self._layer_of.__getitem__)

    def select(self, audited: np.ndarray, token_start: np.ndarray) -> None:
        """Choose the rows to record next step and the token index of each row's query
        (runtime/audit_kernel.py:190-194)."""
        n = len(audited)
        if n > self.rows:
            raise ValueError(f"{n} rows exceed the plane's {self.rows}")
        self._select[:n].copy_(torch.from_numpy(np.asarray(audited).astype(np.uint8)))
        self._token[:n].copy_(torch.from_numpy(np.asarray(token_start).astype(np.int32)))

    def record(
        self,
        layer_name: str,
        table: torch.Tensor,
        lens: torch.Tensor,
        query: torch.Tensor,
        kv_cache: torch.Tensor,
        scale: float,
    ) -> None:
        """Record one attention layer after it attended (runtime/audit_kernel.py:196-222).

        Layers are numbered by name in the order they first run; the launch is the same on every
        step because the kernel reads the audit flag on the device, so a graph can capture it.
        """
        if kv_cache.ndim != 5 or kv_cache.shape[1] != 2:
            raise ValueError(f"expected a KV cache [blocks, 2, block, heads, dim], got {tuple(kv_cache.shape)}")
        if kv_cache.shape[2] != self.block_size:
            raise ValueError("the KV cache's block size differs from the view's")
        layer = self._layer_of.setdefault(layer_name, len(self._layer_of))
        planned = bool(self._plan)
        if planned and layer == 0:  # the step's first layer: every layer of the step reads these buffers
            self.plan(table, lens)
        self.launch(layer, table, lens, query, kv_cache[:, 0], scale, planned=planned)

    def _batch_shape(self, table: torch.Tensor, lens: torch.Tensor) -> tuple[int, int]:
        for name, t in (("table", table), ("lens", lens)):
            if not t.is_cuda:
                raise ValueError(f"{name} must be a device tensor")
        if table.dtype != torch.int32 or lens.dtype != torch.int32:
            raise ValueError("the block table and lengths must be int32")
        if table.ndim != 2 or table.stride(1) != 1 or lens.ndim != 1 or lens.stride(0) != 1:
            raise ValueError("the block table rows and the lengths must be contiguous")
        return min(self.rows, table.shape[0], lens.shape[0]), min(self.width, table.shape[1])

    def plan(self, table: torch.Tensor, lens: torch.Tensor, *, stream=None) -> None:
        """Build the step plan from the view buffers and the selected rows: each audit workgroup's
        tiles with their rows, block ids and query tokens, the work list every launch of the step
        shares (``launch(..., planned=True)``).  Launched on the stream like the audits, so a graph
        that captures a step captures it."""
        if not self._plan:
            raise RuntimeError("this plane is too large for a step plan")
        rows, width = self._batch_shape(table, lens)
        ekv_hip.call(
            "ekv_audit_plan",
            table.data_ptr(), table.stride(0), lens.data_ptr(), self._token.data_ptr(), self._select.data_ptr(),
            self._flag_dev, rows, width, self.block_size, TILE_BLOCKS,
            self._plan, self._plan_bytes, self.rows, self.width, ekv_hip.stream_handle(stream),
        )

    def launch(
        self,
        layer: int,
        table: torch.Tensor,
        lens: torch.Tensor,
        query: torch.Tensor,
        keys: torch.Tensor,
        scale: float,
        *,
        k_scale: float = 1.0,
        chunk_tiles: int = 0,
        planned: bool = False,
        stream=None,
    ) -> None:
        """Launch the audit kernel for ``layer``; ``keys`` is the key cache [blocks, block, heads, dim]
        (runtime/audit_kernel.py:224-265).  ``k_scale`` dequantises an fp8 key cache.  ``planned``
        reads the work list ``plan`` built from the same table, lengths and selection; otherwise the
        launch builds it itself."""
        if layer >= self._layers:
            raise RuntimeError(f"more attention layers ran than the {self._layers} the plane was sized for")
        kv_heads, dim = keys.shape[2], keys.shape[3]
        if kv_heads * self.group_rows != query.shape[1] or dim != query.shape[2]:
            raise ValueError("the query and KV cache shapes do not match the plane's group size")
        if self.kv_heads is not None and kv_heads != self.kv_heads:
            raise ValueError(f"the plane records {self.kv_heads} KV heads, the cache has {kv_heads}")
        if keys.shape[1] != self.block_size:
            raise ValueError("the key cache's block size differs from the plane's")
        for name, t in (("query", query), ("keys", keys)):
            if not t.is_cuda:
                raise ValueError(f"{name} must be a device tensor")
        rows, width = self._batch_shape(table, lens)
        if query.stride(2) != 1 or keys.stride(3) != 1:
            raise ValueError("query and key rows must be contiguous in the head dimension")
        if planned and not self._plan:
            raise RuntimeError("this plane is too large for a step plan")
        plane, layer_stride, row_stride = self.strides
        if self.kv_heads is None:
            group_first, groups = layer % kv_heads, 1  # runtime/audit_kernel.py:250
        else:
            group_first, groups = 0, kv_heads
        common = (
            query.data_ptr(), ekv_hip.dtype_code(query.dtype), query.stride(0), query.stride(1),
            keys.data_ptr(), ekv_hip.dtype_code(keys.dtype), keys.stride(0), keys.stride(1), keys.stride(2),
            float(k_scale),
            table.data_ptr(), table.stride(0), lens.data_ptr(), self._token.data_ptr(), self._select.data_ptr(),
            self._flag_dev,
            self._lse, plane, layer_stride, row_stride, self.cells,
            self._cycles_dev, self.rows if self._cycles_dev else 0,
            float(scale), layer, group_first, groups, self.group_rows,
            rows, width, self.block_size, TILE_BLOCKS, dim,
        )
        if planned:
            ekv_hip.call("ekv_audit_tile_lse_planned", *common, self._plan, self._plan_bytes, self.rows, self.width,
                         ekv_hip.stream_handle(stream))
        else:
            ekv_hip.call("ekv_audit_tile_lse", *common, int(chunk_tiles), ekv_hip.stream_handle(stream))
