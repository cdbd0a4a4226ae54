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
(mlir_pass/lib/eKVTimer.cpp:1348-1387, read as observe/cycles.py:1-45 describes).  The timer is
published on a descriptor line of its own with the pass's keys (``pid``, ``kernel``, ``max_rows``,
``timer_dev``, ``timer_ipc``, ``timer_bytes``; mlir_pass/lib/eKVTimer.cpp:588-590), so the
reference's readers (``find_published`` / ``read_pass_cycles``, ``Capture.cycle_deltas``) find it.

Batched layers.  A decode step's audit launches differ only in the layer, so by default
(``batch_layers``, or ``EKV_AUDIT_BATCH=0`` to turn it off) ``record`` launches the audit of the
step's layers once, when the last layer that has ever recorded records
(``ekv_audit_tile_lse_layers``): the records are those of the per-layer launches, bit for bit, and
the launch's fixed costs are paid once per step.  Under graph capture the launch reads every layer's
query in place (the capture keeps that memory for it); outside one each layer's query rows are first
staged into a plane-owned buffer.  Pending layers also launch on ``flush()``, at the next ``select``
and before the planes are read.
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
IPC_LIMIT_BYTES = 2 << 30  # a statistic block exported by IPC handle stays below 2 GiB


def _enabled(name: str, default: bool = False) -> bool:
    value = os.environ.get(name, "")
    if value == "":
        return default
    return value not in ("0", "false")


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
        batch_layers: bool | None = None,
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
        if self.lse_bytes >= IPC_LIMIT_BYTES:
            raise ValueError(
                f"a statistic block of {self.lse_bytes} bytes ({layers} layers x {rows} rows x {width} blocks x "
                f"{self.cells} cells x 2 planes x 4 B) reaches the {IPC_LIMIT_BYTES} bytes its IPC export allows")
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
        self._plan_inputs: tuple | None = None  # (table, row stride, lens, rows, width) the plan was built from
        self._plan_stale = True  # a selection has changed since the plan was built
        # batched layers: the step's recorded layers waiting for one launch, and their staged queries
        self.batch_layers = _enabled("EKV_AUDIT_BATCH", True) if batch_layers is None else bool(batch_layers)
        self._pending: list[ekv_hip.AuditLayer] = []
        self._held: list[torch.Tensor] = []  # queries a pending launch reads in place
        self._pending_shape: tuple | None = None  # what the pending layers share
        self._staged = 0
        self._staged_shape: tuple | None = None  # (dtype, heads per row, head_dim) of the staging buffer
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
        lines = [entry]
        if self._cycles_dev:
            # the timer as the pass publishes it (mlir_pass/lib/eKVTimer.cpp:588-590): the readers of
            # observe/zero_touch.py:66-93, :190-225 and observe/capture.py:77-99 need pid and timer_bytes.
            # A line of its own, so that a reader of capture buffers (host_va) never takes the planes for one.
            lines.append({
                "pid": self.pid,
                "kernel": "ekv_audit_tile_lse",
                "max_rows": self.rows,
                "ncap": self.width,
                "timer_dev": self._cycles_dev,
                "timer_ipc": self._ipc(self._cycles_dev),
                "timer_bytes": self.rows * 8,
            })
        path = pub_path(self.pid)
        with open(path, "a") as f:
            for line in lines:
                f.write(json.dumps(line) + "\n")
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
        """A host copy of both planes, ``float32[2, layers, rows, width, cells]`` (pending layers launch first)."""
        self.flush()
        raw = ekv_hip.d2h(self._lse, self.lse_bytes)
        return np.frombuffer(raw, dtype=np.float32).reshape(2, self._layers, self.rows, self.width, self.cells)

    def read_cycles(self) -> np.ndarray:
        """A host copy of the per-row cycle accumulator (zeros when there is no timer)."""
        if not self._cycles_dev:
            return np.zeros(self.rows, dtype=np.uint64)
        self.flush()
        return np.frombuffer(ekv_hip.d2h(self._cycles_dev, self.rows * 8), dtype=np.uint64).copy()

    def clear(self, layer: int | None = None) -> None:
        """Mark every cell (or those of one layer) unwritten again (NaN)."""
        self.flush()
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
        (runtime/audit_kernel.py:190-194).  Rows past the batch are cleared: the reference writes only
        the batch's rows, which leaves a shrinking batch's old rows selected with old lengths and query
        tokens for the step plan and the launches to read."""
        n = len(audited)
        if n > self.rows:
            raise ValueError(f"{n} rows exceed the plane's {self.rows}")
        if len(token_start) < n:
            raise ValueError(f"{n} rows need as many query tokens, got {len(token_start)}")
        self.flush()  # the previous step's layers read the selection they were staged with
        chosen = np.zeros(self.rows, dtype=np.uint8)
        chosen[:n] = np.asarray(audited).astype(np.uint8)
        tokens = np.zeros(self.rows, dtype=np.int32)
        tokens[:n] = np.asarray(token_start[:n]).astype(np.int32)
        self._select.copy_(torch.from_numpy(chosen))
        self._token.copy_(torch.from_numpy(tokens))
        self._plan_stale = True

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
        if layer >= self._layers:
            raise RuntimeError(f"more attention layers ran than the {self._layers} the plane was sized for")
        planned = bool(self._plan)
        if planned and (layer == 0 or self._plan_stale or self._inputs(table, lens) != self._plan_inputs):
            # the step's first layer (or new view buffers): every layer of the step reads this plan
            self.flush()
            self.plan(table, lens)
        keys = kv_cache[:, 0]
        if not (planned and self.batch_layers and self._batchable(query, keys)):
            self.launch(layer, table, lens, query, keys, scale, planned=planned)
            return
        self._check_layer(query, keys)
        # Under graph capture the launch reads each layer's query where it is: the references held
        # until the launch keep the capture from giving that memory to anything before it, so every
        # replay has the queries in place.  Outside a capture the query may be memory that a graph
        # replayed between the layers reuses (a piecewise-captured model), so it is staged.
        direct = torch.cuda.is_current_stream_capturing()
        heads, dim = self.cells, keys.shape[3]
        q_layout = (0, query.stride(0), query.stride(1)) if direct else (1, heads * dim, dim)
        shape = (ekv_hip.dtype_code(query.dtype), ekv_hip.dtype_code(keys.dtype), tuple(keys.stride()[:3]),
                 keys.shape[2], dim, ekv_hip.stream_handle(), q_layout)
        if self._pending and (shape != self._pending_shape or any(e.layer == layer for e in self._pending)):
            self.flush()
        self._pending_shape = shape
        if direct:
            self._held.append(query)
            self._pending.append(self.direct(layer, query, keys, scale))
        else:
            self._pending.append(self.stage(layer, query, keys, scale))
        if layer == len(self._layer_of) - 1:  # the last layer that has run: the step's layers are in
            self.flush()

    def _inputs(self, table: torch.Tensor, lens: torch.Tensor) -> tuple:
        rows, width = self._batch_shape(table, lens)
        return table.data_ptr(), table.stride(0), lens.data_ptr(), rows, width

    def _batchable(self, query: torch.Tensor, keys: torch.Tensor) -> bool:
        try:
            q_code, k_code = ekv_hip.dtype_code(query.dtype), ekv_hip.dtype_code(keys.dtype)
        except ValueError:
            return False
        return bool(ekv_hip.load().ekv_audit_shape(q_code, k_code, keys.shape[3], self.block_size) & ekv_hip.AUDIT_PLANNED)

    def stage(self, layer: int, query: torch.Tensor, keys: torch.Tensor, scale: float, *, k_scale: float = 1.0,
              stream=None) -> "ekv_hip.AuditLayer":
        """Copy the layer's selected query rows into its slot of the staging buffer (on the stream, after
        the selection); returns the layer's entry for ``launch_layers``.  ``keys`` is the key cache
        [blocks, block, heads, dim]; ``k_scale`` dequantises an fp8 one."""
        kv_heads, dim = keys.shape[2], keys.shape[3]
        heads = self.cells  # the audited query heads: one group, or every KV head's
        head_first = 0 if self.kv_heads is not None else (layer % kv_heads) * self.group_rows
        shape = (query.dtype, heads, dim)
        if self._staged_shape is None:
            self._staged = self._allocate(self._layers * self.rows * heads * dim * query.element_size())
            self._staged_shape = shape
        elif shape != self._staged_shape:
            raise ValueError(f"the queries changed from {self._staged_shape} to {shape}: a plane records one model")
        slot = self._staged + layer * self.rows * heads * dim * query.element_size()
        ekv_hip.call(
            "ekv_audit_stage_queries", query.data_ptr(), ekv_hip.dtype_code(query.dtype), query.stride(0),
            query.stride(1), head_first, heads, dim, self._token.data_ptr(), self._select.data_ptr(), self._flag_dev,
            self.rows, slot, heads * dim, ekv_hip.stream_handle(stream),
        )
        group_first = 0 if self.kv_heads is not None else layer % kv_heads
        return ekv_hip.AuditLayer(slot, keys.data_ptr(), layer, group_first, head_first, float(scale), float(k_scale), 0)

    def direct(self, layer: int, query: torch.Tensor, keys: torch.Tensor, scale: float, *,
               k_scale: float = 1.0) -> "ekv_hip.AuditLayer":
        """The layer's entry for ``launch_layers`` reading ``query`` [tokens, heads, dim] in place: the
        caller keeps it unchanged until the launch."""
        group_first = 0 if self.kv_heads is not None else layer % keys.shape[2]
        return ekv_hip.AuditLayer(query.data_ptr(), keys.data_ptr(), layer, group_first, 0, float(scale),
                                  float(k_scale), 0)

    def flush(self) -> None:
        """Launch the audit of the layers recorded since the last launch (nothing if none are pending)."""
        if not self._pending:
            return
        entries, (q_code, k_code, k_strides, kv_heads, dim, stream, q_layout) = self._pending, self._pending_shape
        self._pending = []
        self._launch_layers(entries, q_code, k_code, k_strides, kv_heads, dim, stream, q_layout)
        self._held = []  # the launch is enqueued after every query it reads

    def launch_layers(self, entries: list, keys: torch.Tensor, query: torch.Tensor, *, staged: bool,
                      stream=None) -> None:
        """One audit launch (per 32 layers) over ``entries``, from ``stage`` (``staged``) or ``direct``,
        and the step plan; ``keys`` is any of their key caches [blocks, block, heads, dim] and ``query``
        any of their queries (the strides and shape they share)."""
        dim = keys.shape[3]
        q_layout = (1, self.cells * dim, dim) if staged else (0, query.stride(0), query.stride(1))
        self._launch_layers(list(entries), ekv_hip.dtype_code(query.dtype), ekv_hip.dtype_code(keys.dtype),
                            tuple(keys.stride()[:3]), keys.shape[2], dim, ekv_hip.stream_handle(stream), q_layout)

    def _launch_layers(self, entries, q_code, k_code, k_strides, kv_heads, dim, stream, q_layout) -> None:
        if self._plan_inputs is None:
            raise RuntimeError("no step plan has been built: plan() the view buffers first")
        table, stride, lens, rows, width = self._plan_inputs
        kb, kp, kh = k_strides
        by_row, q_token, q_head = q_layout
        groups = 1 if self.kv_heads is None else kv_heads
        plane, layer_stride, row_stride = self.strides
        array = (ekv_hip.AuditLayer * len(entries))(*entries)
        ekv_hip.call(
            "ekv_audit_tile_lse_layers", array, len(entries), by_row, q_code, q_token, q_head, k_code, kb, kp, kh,
            table, stride, lens, self._token.data_ptr(), self._select.data_ptr(), self._flag_dev,
            self._lse, plane, layer_stride, row_stride, self.cells,
            self._cycles_dev, self.rows if self._cycles_dev else 0,
            groups, self.group_rows, rows, width, self.block_size, TILE_BLOCKS, dim,
            self._plan, self._plan_bytes, self.rows, self.width, stream,
        )

    def _check_layer(self, query: torch.Tensor, keys: torch.Tensor) -> None:
        """The shape checks of ``launch`` (runtime/audit_kernel.py:234-238)."""
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
        if query.stride(2) != 1 or keys.stride(3) != 1:
            raise ValueError("query and key rows must be contiguous in the head dimension")

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
        self.flush()  # pending layers read the plan being replaced
        self._plan_inputs = self._inputs(table, lens)
        self._plan_stale = False
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
        self._check_layer(query, keys)
        kv_heads, dim = keys.shape[2], keys.shape[3]
        rows, width = self._batch_shape(table, lens)
        if not planned and self._plan:
            forms = ekv_hip.load().ekv_audit_shape(ekv_hip.dtype_code(query.dtype), ekv_hip.dtype_code(keys.dtype),
                                                   dim, self.block_size)
            if not forms & ekv_hip.AUDIT_SELF_CONTAINED and forms & ekv_hip.AUDIT_PLANNED:
                self.plan(table, lens, stream=stream)  # only the planned launch has this shape
                planned = True
        if planned and not self._plan:
            raise RuntimeError("this plane is too large for a step plan")
        if planned and self._inputs(table, lens) != self._plan_inputs:
            raise RuntimeError("the step plan was built from other view buffers: plan() them first")
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
