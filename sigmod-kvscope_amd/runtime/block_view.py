"""The decode view of a paged block table: a per-request read budget the attention kernel enforces.

A paged attention kernel finds a request's keys through its block-table row and stops at its length.
Give it a row that lists only some blocks and a length that ends at the last of them, and it reads
only those blocks -- unchanged, and exactly, for full causal attention, whose keys carry their
positions in the cache (the contract of runtime/block_view.py:1-15).

``DecodeView`` holds what the controller committed for each row (the blocks to read, the blocks the
engine released, the audits it asked for, the lease), and turns every batch into its view: rows that
decode read their committed blocks; rows that prefill, rows being audited, and every row once the
lease has lapsed read their whole table; released blocks are never read.  One ``ekv_build_view``
launch per step composes those rules on the device, compacts every row, writes the lengths and adds
the read counters, into buffers whose addresses never change so that captured graphs keep reading
them.  The engine-facing functions at the end install the view and the audit kernel into vLLM's
attention backends.
"""

from __future__ import annotations

import os
import time
from collections.abc import Callable
from dataclasses import dataclass
from typing import Protocol

import numpy as np
import torch

import ekv_hip
from observe.allocation import check_tensors
from runtime.audit import AuditPlane


class StatisticSwitch(Protocol):
    """The part of an audit plane the view drives (runtime/block_view.py:28-33): the rows a step
    records, and recording on or off."""

    def set(self, on: bool) -> None: ...

    def select(self, audited: np.ndarray, token_start: np.ndarray) -> None: ...


_MASKS = (torch.bool, torch.uint8)


def _table_shape(table: torch.Tensor, seq_lens: torch.Tensor) -> tuple[int, int]:
    if not isinstance(table, torch.Tensor) or table.ndim != 2:
        raise ValueError("the block table must be a [rows, width] tensor")
    rows, width = int(table.shape[0]), int(table.shape[1])
    if not isinstance(seq_lens, torch.Tensor) or seq_lens.ndim != 1 or seq_lens.shape[0] < rows:
        raise ValueError(f"{rows} table rows need as many int32 lengths")
    check_tensors(("table", table, torch.int32, (rows, width)),
                  ("seq_lens", seq_lens, torch.int32, tuple(seq_lens.shape)))
    return rows, width


def compact_block_table(
    table: torch.Tensor, seq_lens: torch.Tensor, keep: torch.Tensor, block_size: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """Each row's view of the blocks ``keep`` marks (runtime/block_view.py:36-56): the row's first and
    last block are read whatever ``keep`` says, the read blocks come first in their order and the rest
    follow in theirs, and the length counts the read blocks in full except the last, which keeps its
    own fill (0 for a row without tokens).  Returns new device tensors (view table, view lengths)."""
    rows, width = _table_shape(table, seq_lens)
    check_tensors(("table", table, torch.int32, (rows, width)), ("keep", keep, _MASKS, (rows, width)))
    view = torch.empty(rows, width, dtype=torch.int32, device=table.device)
    lens = torch.empty(rows, dtype=torch.int32, device=table.device)
    ekv_hip.call(
        "ekv_compact_view",
        table.data_ptr(), table.stride(0), seq_lens.data_ptr(), keep.data_ptr(), keep.stride(0),
        rows, width, int(block_size), view.data_ptr(), view.stride(0), lens.data_ptr(), ekv_hip.stream_handle(),
    )
    return view, lens


def uniform_view(
    scores: torch.Tensor,
    blocks: torch.Tensor,
    table: torch.Tensor,
    seq_lens: torch.Tensor,
    block_size: int,
    *,
    fraction: float = 1.0,
    budget: int = -1,
    recent_blocks: int = 0,
    measured: torch.Tensor | None = None,
    pin_from: torch.Tensor | None = None,
    counts: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The ``uniform`` ranking and the view built from it in one kernel: what
    ``observe.allocation.uniform_keep`` followed by ``compact_block_table`` on its keep returns
    (observe/allocation.py:39-91 with observe/controller.py:398-451, then runtime/block_view.py:36-56),
    as ``(keep, summary, view, view_lens)``.  Each row's workgroup compacts its table row from the keep
    it has just decided.  Explicit pinned / released masks go through the two calls instead.
    ``counts`` (int64 [rows, 5]) accumulates DecodeView's read counters as ``DecodeView.build`` does for
    live decoding rows outside the audit (runtime/block_view.py:313-329)."""
    rows, width = _table_shape(table, seq_lens)
    check_tensors(("scores", scores, torch.float32, (rows, width)), ("blocks", blocks, torch.int32, (rows,)),
                  ("table", table, torch.int32, (rows, width)), ("measured", measured, _MASKS, (rows,)),
                  ("pin_from", pin_from, torch.int32, (rows,)), ("counts", counts, torch.int64, (rows, 5)))
    if counts is not None and not counts.is_contiguous():
        raise ValueError("counts must be a contiguous int64 [rows, 5] tensor")
    keep = torch.empty(rows, width, dtype=torch.uint8, device=scores.device)
    summary = torch.zeros(6, dtype=torch.int64, device=scores.device)
    view = torch.empty(rows, width, dtype=torch.int32, device=table.device)
    lens = torch.empty(rows, dtype=torch.int32, device=table.device)
    ekv_hip.call(
        "ekv_rank_uniform_view",
        scores.data_ptr(), scores.stride(0), blocks.data_ptr(), ekv_hip.ptr(measured), ekv_hip.ptr(pin_from),
        int(recent_blocks), rows, width, float(fraction), int(budget), keep.data_ptr(), keep.stride(0),
        summary.data_ptr(), table.data_ptr(), table.stride(0), seq_lens.data_ptr(), int(block_size),
        view.data_ptr(), view.stride(0), lens.data_ptr(), ekv_hip.ptr(counts), ekv_hip.stream_handle(),
    )
    return keep, summary, view, lens


@dataclass
class _Mirror:
    """A device copy of a host mask, refreshed when its version moves."""

    tensor: torch.Tensor | None = None
    version: int = -1

    def of(self, host: np.ndarray, version: int, device: torch.device) -> torch.Tensor:
        if self.tensor is None or self.version != version or self.tensor.device != device:
            self.tensor = torch.from_numpy(host.astype(np.uint8)).to(device)
            self.version = version
        return self.tensor


@dataclass
class _Step:
    """What one build decides on the host before the device work."""

    rows: int  # the batch's rows
    live: bool  # the lease holds
    decode: np.ndarray  # rows computing one token
    audited: np.ndarray  # [view rows] rows this step audits


class _RowState:
    """Per row, what the controller committed and what the row's audits covered; ``moved`` carries
    it with the requests when the scheduler reorders them."""

    def __init__(self, rows: int, width: int) -> None:
        self.keep = np.ones((rows, width), dtype=bool)  # read this block
        self.released = np.zeros((rows, width), dtype=bool)  # the engine took the block back
        self.audited = np.zeros(rows, dtype=bool)  # the row's request has had a completed audit
        self.audited_blocks = np.zeros(rows, dtype=np.int64)  # its length in blocks at that audit
        self.wants_audit = np.zeros(rows, dtype=bool)  # its next decode step is an audit

    def moved(self, source: np.ndarray, fresh: np.ndarray, audit_fresh: np.ndarray) -> None:
        """Row r takes the state of row source[r]; rows in ``fresh`` start over (full reads, no
        release, no audit yet), asking for an audit where ``audit_fresh`` says so."""
        self.keep = self.keep[source]
        self.released = self.released[source]
        self.audited = self.audited[source]
        self.audited_blocks = self.audited_blocks[source]
        self.wants_audit = self.wants_audit[source]
        self.keep[fresh] = True
        self.released[fresh] = False
        self.audited[fresh] = False
        self.audited_blocks[fresh] = 0
        self.wants_audit[fresh] = audit_fresh[fresh]


class DecodeView:
    """One serving process's committed read policy and the view it gives each batch
    (runtime/block_view.py:59-401).

    The controller's generations arrive through the ``write_*`` methods, already mapped to the
    current scheduler rows.  ``deadline_ns`` is a ``time.monotonic_ns`` instant: past it, or before
    any commit, every row reads in full, so a stopped controller costs nothing to undo.  A row whose
    audit was asked for reads in full at its next decode step, which the audit plane records; the
    request is consumed by that step."""

    COUNTERS = ("read", "full", "audit", "untrimmed", "expired")

    def __init__(
        self,
        rows: int,
        width: int,
        block_size: int,
        audit: StatisticSwitch | None = None,
        prefill_audit: bool = False,
    ) -> None:
        if rows <= 0 or width <= 0 or block_size <= 0:
            raise ValueError(f"a view of {rows} rows x {width} blocks of {block_size} tokens is empty")
        if prefill_audit and audit is None:
            raise ValueError("auditing in the last prefill step needs an audit plane to record with")
        self.rows, self.width, self.block_size = rows, width, block_size
        self.audit = audit
        # audit a new request in the step that computes the end of its prompt, which reads every
        # block anyway; it needs kernels in which only the newest tokens' program records
        self.prefill_audit = prefill_audit
        self.final_prefill = np.zeros(rows, dtype=bool)  # rows computing the end of their prompt next
        self.on_prefill_audit: Callable[[], None] | None = None  # the plane's check, before such a step
        self._state = _RowState(rows, width)
        self.released_version = 0
        self.version = 0
        self.deadline_ns = 0
        self.last_audit_rows = np.zeros(rows, dtype=bool)  # the rows of the last completed audit
        self.audit_step = False
        self.audits_started = 0
        self.audits_completed = 0
        self.on_audit_start: Callable[[], None] | None = None  # the publisher announces an audit
        self.audit_gate: Callable[[], bool] | None = None  # False holds the audit requests back
        self.before_build: Callable[[], None] | None = None  # the publisher's last chance to apply
        self._pending: np.ndarray | None = None  # rows of an audit step the device may still run
        self._pending_blocks = np.zeros(rows, dtype=np.int64)
        self._device: torch.device | None = None
        self._keep_dev, self._released_dev = _Mirror(), _Mirror()
        self._table: torch.Tensor | None = None
        self._lens: torch.Tensor | None = None
        self._counts: torch.Tensor | None = None  # int64 [rows, 5], one slot per row, summed when read
        self._audited_dev: torch.Tensor | None = None
        self._decoding_dev: torch.Tensor | None = None

    # -- the per-row state, under the reference's attribute names --------------------------------

    @property
    def keep(self) -> np.ndarray:
        return self._state.keep

    @keep.setter
    def keep(self, value: np.ndarray) -> None:
        self._state.keep = np.asarray(value, dtype=bool)

    @property
    def released(self) -> np.ndarray:
        return self._state.released

    @property
    def row_audited(self) -> np.ndarray:
        return self._state.audited

    @property
    def audited_blocks(self) -> np.ndarray:
        return self._state.audited_blocks

    @property
    def audit_rows(self) -> np.ndarray:
        return self._state.wants_audit

    # -- what the controller writes (runtime/block_view.py:133-218) -------------------------------

    def write_row_controls(self, mask: np.ndarray, log_weight: np.ndarray | None = None) -> int:
        """Commit a generation: nonzero ``mask[row, block]`` reads the block."""
        if log_weight is not None:
            raise ValueError("the view keeps or drops whole blocks; it has no use for log weights")
        mask = np.asarray(mask)
        if mask.shape != (self.rows, self.width):
            raise ValueError(f"a {mask.shape} mask for a view of {(self.rows, self.width)}")
        self.keep = mask != 0
        self.version += 1
        return 1

    def write_lease_deadline(self, deadline_ns: int) -> int:
        self.deadline_ns = int(deadline_ns)
        return 1

    def write_audit_rows(self, requested: np.ndarray) -> int:
        """Ask for an audit of the marked rows, each served by one decode step."""
        requested = np.asarray(requested, dtype=bool)
        if requested.shape != (self.rows,):
            raise ValueError(f"{requested.shape} audit requests for a view of {self.rows} rows")
        if self.audit is None and requested.any():
            raise ValueError("an audit needs an audit plane to switch the statistic on, and this view has none")
        self._state.wants_audit |= requested
        return 1

    def write_final_prefill(self, rows: np.ndarray) -> None:
        """The rows that compute the end of their prompt in the next step (only the next one)."""
        rows = np.asarray(rows, dtype=bool)
        if rows.shape[0] > self.rows:
            raise ValueError(f"{rows.shape[0]} prefill marks for a view of {self.rows} rows")
        self.final_prefill = np.zeros(self.rows, dtype=bool)
        self.final_prefill[: rows.shape[0]] = rows

    def write_release(self, mask: np.ndarray) -> list[tuple[int, int]]:
        """Release the marked blocks; returns the ``(row, block)`` pairs newly released.

        Only blocks that an audit of the row's present request covered may go: a mark for a row
        without one, or beyond the length that audit saw, is ignored, and so are the first block
        and the audit's last block, which every view reads."""
        mask = np.asarray(mask) != 0
        if mask.shape != (self.rows, self.width):
            raise ValueError(f"a {mask.shape} release for a view of {(self.rows, self.width)}")
        st = self._state
        block = np.arange(self.width)[None, :]
        covered = st.audited[:, None] & (block >= 1) & (block < (st.audited_blocks - 1)[:, None])
        fresh = mask & covered & ~st.released
        if fresh.any():
            st.released = st.released | fresh
            self.released_version += 1
        rows, blocks = np.nonzero(fresh)
        return [(int(r), int(b)) for r, b in zip(rows, blocks)]

    def reassign_rows(self, moved: dict[int, int], new: list[int], empty: list[int]) -> None:
        """The scheduler reordered its requests: ``moved[row]`` is the row a request held in the previous
        batch, and it takes its state along; ``new`` rows hold requests not seen before (full reads, and
        an audit at their first decode step when there is a plane); ``empty`` rows hold none."""
        source = np.arange(self.rows)
        for row, old in moved.items():
            source[row] = old
        fresh = np.zeros(self.rows, dtype=bool)
        fresh[list(new) + list(empty)] = True
        audit_fresh = np.zeros(self.rows, dtype=bool)
        if self.audit is not None:
            audit_fresh[list(new)] = True
        audit_fresh[list(empty)] = False  # a row listed as both holds no request
        before = self._state.released
        self._state.moved(source, fresh, audit_fresh)
        if not np.array_equal(before, self._state.released):
            self.released_version += 1
        self.version += 1

    # -- the engine's side ----------------------------------------------------------------------

    def active(self) -> bool:
        return self.deadline_ns > time.monotonic_ns()

    def may_audit(self) -> bool:
        return self.audit_gate is None or bool(self.audit_gate())

    def start_audit(self) -> None:
        """An audit step starts: counted, and announced before the device runs it, because its
        statistic replaces the previous audit's."""
        self.audits_started += 1
        if self.on_audit_start is not None:
            self.on_audit_start()

    def finish_audit(self) -> None:
        """Close the previous step's audit once the device has written it (runtime/block_view.py:373-389).
        Only audit steps wait for the device.  It must run before requests move between rows, since the
        audited rows are the rows of that step's batch."""
        if self._pending is None:
            return
        flush = getattr(self.audit, "flush", None)
        if flush is not None:
            flush()  # layers an audit kernel still holds for one launch
        if self._device is not None and self._device.type == "cuda":
            torch.cuda.synchronize(self._device)
        rows, st = self._pending, self._state
        self.last_audit_rows = rows
        st.audited |= rows
        st.audited_blocks[rows] = self._pending_blocks[rows]
        self.audits_completed += 1
        self._pending = None

    def _decide(self, seq_lens: torch.Tensor, query_lens: torch.Tensor) -> _Step:
        """The host's part of a build: which rows decode, which are audited, and the plane's switch."""
        live = self.active()  # read once, before anything that may wait for the device
        self.finish_audit()
        n = len(query_lens)
        q = np.asarray(query_lens.numpy() if isinstance(query_lens, torch.Tensor) else query_lens)
        decode = q == 1
        servable = decode | (self.final_prefill[:n] & self.prefill_audit)
        self.final_prefill = np.zeros(self.rows, dtype=bool)
        audited = np.zeros(self.rows, dtype=bool)
        audited[:n] = self._state.wants_audit[:n] & servable
        if audited.any() and not self.may_audit():
            audited[:] = False  # the controller has not read the last audit yet
        if (audited[:n] & ~decode).any() and self.on_prefill_audit is not None:
            self.on_prefill_audit()
        self._state.wants_audit[audited] = False
        self.audit_step = bool(audited.any())
        if self.audit_step:
            self._pending = audited
            self.start_audit()
            bs = self.block_size
            self._pending_blocks[:n] = ((seq_lens[:n] + bs - 1) // bs).cpu().numpy()
        if self.audit is not None:
            token_start = np.concatenate(([0], np.cumsum(q)[:-1])) if n else np.zeros(0, dtype=np.int64)
            self.audit.select(audited[:n], token_start)
            self.audit.set(self.audit_step)
        return _Step(n, live, decode, audited)

    def _buffers_on(self, device: torch.device) -> None:
        if self._table is not None:
            return
        self._device = device
        self._table = torch.zeros(self.rows, self.width, dtype=torch.int32, device=device)
        self._lens = torch.zeros(self.rows, dtype=torch.int32, device=device)
        self._counts = torch.zeros(self.rows, len(self.COUNTERS), dtype=torch.int64, device=device)
        self._audited_dev = torch.zeros(self.rows, dtype=torch.uint8, device=device)
        self._decoding_dev = torch.ones(self.rows, dtype=torch.uint8, device=device)

    def _row_flags(self, flags: np.ndarray, n: int, target: torch.Tensor) -> torch.Tensor:
        target[:n].copy_(torch.from_numpy(flags[:n].astype(np.uint8)))
        return target

    def build(
        self, table: torch.Tensor, seq_lens: torch.Tensor, query_lens: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """The view (table, lengths) of a batch of ``len(query_lens)`` rows, in the persistent buffers
        (runtime/block_view.py:225-295).  ``query_lens`` (host) counts the tokens each row computes:
        one decodes and gets its view, more prefills and reads its whole row."""
        if self.before_build is not None:
            self.before_build()
        n = len(query_lens)
        rows, width = _table_shape(table, seq_lens)
        if width != self.width or n > self.rows or rows < n:
            raise ValueError(f"a batch of {n} rows x {width} blocks does not fit a view of "
                             f"{self.rows} x {self.width}")
        step = self._decide(seq_lens, query_lens)
        self._buffers_on(table.device)
        if n == 0:
            return self._table[:0], self._lens[:0]
        dev = table.device
        keep = self._keep_dev.of(self._state.keep, self.version, dev)
        released = self._released_dev.of(self._state.released, self.released_version, dev) \
            if self._state.released.any() else None
        audited = self._row_flags(step.audited, n, self._audited_dev) if self.audit_step else None
        decoding = None if step.decode.all() else self._row_flags(step.decode, n, self._decoding_dev)
        ekv_hip.call(
            "ekv_build_view",
            table.data_ptr(), table.stride(0), seq_lens.data_ptr(), keep.data_ptr(), keep.stride(0),
            ekv_hip.ptr(released), released.stride(0) if released is not None else 0,
            ekv_hip.ptr(audited), ekv_hip.ptr(decoding), int(step.live),
            n, width, self.block_size,
            self._table.data_ptr(), self._table.stride(0), self._lens.data_ptr(), self._counts.data_ptr(),
            ekv_hip.stream_handle(),
        )
        return self._table[:n], self._lens[:n]

    def skip(self, seq_lens: torch.Tensor, query_lens: torch.Tensor) -> None:
        """A batch that reads the engine's own table (a shared-prefix cascade) records nothing; its
        decode rows are counted as full reads (runtime/block_view.py:352-361)."""
        self.finish_audit()
        self.audit_step = False
        if self.audit is not None:
            self.audit.set(False)
        n = len(query_lens)
        if n == 0:
            return
        if n > self.rows:
            raise ValueError(f"a batch of {n} rows does not fit a view of {self.rows} rows")
        if not isinstance(seq_lens, torch.Tensor) or seq_lens.ndim != 1 or seq_lens.shape[0] < n:
            raise ValueError(f"{n} rows need as many lengths")
        lens = seq_lens[:n].to(torch.int32).contiguous()
        check_tensors(("seq_lens", lens, torch.int32, (n,)))
        self._buffers_on(lens.device)
        decode = np.asarray(query_lens.numpy() if isinstance(query_lens, torch.Tensor) else query_lens) == 1
        decoding = self._row_flags(decode, n, self._decoding_dev)
        ekv_hip.call(  # no table: the rows read in full and only the counters move
            "ekv_build_view",
            0, 0, lens.data_ptr(), 0, 0, 0, 0, 0, decoding.data_ptr(), 1,
            n, 1, self.block_size, 0, 0, 0, self._counts.data_ptr(), ekv_hip.stream_handle(),
        )

    @property
    def buffers(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The view's table and lengths: what the engine's kernels read and graphs capture."""
        if self._table is None or self._lens is None:
            raise RuntimeError("no batch has been built into this view yet")
        return self._table, self._lens

    def _totals(self) -> list[int]:
        if self._counts is None:
            return [0] * len(self.COUNTERS)
        return [int(x) for x in self._counts.sum(dim=0).tolist()]

    def reads(self) -> tuple[int, int]:
        """Blocks read, and blocks full reads would have read, over all decode steps."""
        totals = self._totals()
        return totals[0], totals[1]

    def read_breakdown(self) -> dict[str, int]:
        """Blocks read, split into audit steps, rows read in full without evidence, and lapsed leases."""
        return dict(zip(self.COUNTERS, self._totals()))


# -- installation into vLLM (runtime/block_view.py:404-626) ------------------------------------------

_view: DecodeView | None = None
_plane: AuditPlane | None = None
_layers: tuple[str, ...] = ()  # the attention layers of the one cache group the view serves


def _enabled(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0", "false")


def _audit_plane(builder, cam) -> AuditPlane | None:
    """The plane recording the statistic: the audit kernel's with ``EKV_AUDIT_KERNEL``, the compiler
    pass's with ``EKV_ATTN_SHARE``, none without either.  Both at once would record it twice."""
    kernel, compiled = _enabled("EKV_AUDIT_KERNEL"), _enabled("EKV_ATTN_SHARE")
    if kernel and compiled:
        raise RuntimeError("set one of EKV_ATTN_SHARE and EKV_AUDIT_KERNEL: each records the statistic")
    if compiled:
        return AuditPlane()
    if not kernel:
        return None
    from runtime.audit_kernel import RecordingPlane

    config = builder.vllm_config
    model, parallel = config.model_config, config.parallel_config
    query_heads = model.get_num_attention_heads(parallel)
    return RecordingPlane(
        layers=model.get_num_layers_by_block_type(parallel, "attention"),
        rows=config.scheduler_config.max_num_seqs,
        width=cam.block_table_tensor.shape[1],
        group_rows=query_heads // model.get_num_kv_heads(parallel),
        block_size=builder.kv_cache_spec.block_size,
    )


def require_supported_attention(builder) -> None:
    """Refuse a cache group the view cannot trim exactly (runtime/block_view.py:436-469).

    Dropping blocks from a decode row is exact only for plain full causal self-attention over one
    cache group: the kept keys are then read in their order with their positions.  Any other cache
    group kind (sliding window, chunked local, state space, ...), a window or chunk inside a full
    attention spec, and layers with a sliding window, an ALiBi position bias or other than decoder
    self-attention are refused with a RuntimeError naming the cause."""
    from vllm.v1.attention.backend import AttentionType
    from vllm.v1.kv_cache_interface import FullAttentionSpec

    spec = builder.kv_cache_spec
    kind = type(spec).__name__
    if type(spec) is not FullAttentionSpec:
        raise RuntimeError(f"cache group of {kind}: the view trims full causal attention only")
    if spec.sliding_window is not None or spec.attention_chunk_size is not None:
        raise RuntimeError(f"{kind} with a sliding window or chunked attention: the view cannot trim it")
    layers = builder.vllm_config.compilation_config.static_forward_context
    for name in builder.layer_names:
        layer = layers[name]
        if layer.sliding_window is not None:
            raise RuntimeError(f"layer {name} has a sliding window of {layer.sliding_window}: its blocks cannot "
                               "be dropped exactly")
        if getattr(layer.impl, "alibi_slopes", None) is not None:
            raise RuntimeError(f"layer {name} adds a position bias (ALiBi): its blocks cannot be dropped exactly")
        if layer.attn_type != AttentionType.DECODER:
            raise RuntimeError(f"layer {name} runs {layer.attn_type.value} attention: the view trims decoder "
                               "self-attention only")


def _view_for(builder, cam) -> DecodeView:
    """The process's view, made at the first batch from the engine's row count, table width and block
    size; one cache group only."""
    global _view, _plane, _layers
    names = tuple(builder.layer_names)
    if _view is not None:
        if names != _layers:
            raise RuntimeError("the model has several KV-cache groups; a block-table view serves one")
        return _view
    require_supported_attention(builder)
    plane = _audit_plane(builder, cam)
    prefill_audit = _enabled("EKV_PREFILL_AUDIT")
    if prefill_audit and not _enabled("EKV_ATTN_SHARE"):
        # only the compiler pass reports which kernels record from the newest tokens' program alone
        raise RuntimeError("EKV_PREFILL_AUDIT works with the compiler pass's statistic (EKV_ATTN_SHARE) only")
    view = DecodeView(
        rows=builder.vllm_config.scheduler_config.max_num_seqs,
        width=cam.block_table_tensor.shape[1],
        block_size=builder.kv_cache_spec.block_size,
        audit=plane,
        prefill_audit=prefill_audit,
    )
    if prefill_audit and plane is not None:
        view.on_prefill_audit = plane.require_newest_rows
    _view, _plane, _layers = view, plane, names
    return view


def _query_lens(cam) -> torch.Tensor:
    """Tokens each request computes in the batch, from the host copy of the query offsets."""
    offsets = cam.query_start_loc_cpu[: cam.num_reqs + 1]
    return offsets[1:] - offsets[:-1]


def _patch_once(owner, attribute: str, marker: str, make) -> bool:
    """Replace ``owner.attribute`` by ``make(original)`` unless a wrapper marked ``marker`` is there."""
    original = getattr(owner, attribute)
    if getattr(original, marker, False):
        return False
    wrapper = make(original)
    setattr(wrapper, marker, True)
    setattr(owner, attribute, wrapper)
    return True


def install_decode_view() -> int:
    """Give every attention batch of vLLM's Triton and FlashInfer backends its view; returns how many
    builders were patched (runtime/block_view.py:504-560).

    Call it before the engine exists: vLLM captures its graphs while building its first attention
    metadata, and the first batch makes the view with the engine's own shape, so the graphs capture
    the view's buffers.  The Triton builder's metadata gets the view's table and lengths in place of
    the engine's; FlashInfer plans its launch on the host from the lengths, so it builds from the
    view's batch."""
    from vllm.v1.attention.backends.flashinfer import FlashInferMetadataBuilder
    from vllm.v1.attention.backends.triton_attn import TritonAttentionMetadataBuilder

    def triton(original):
        def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
            metadata = original(self, common_prefix_len, common_attn_metadata, fast_build)
            cam = common_attn_metadata
            view = _view_for(self, cam)
            if common_prefix_len > 0:  # a cascade reads the engine's own table
                view.skip(cam.seq_lens, _query_lens(cam))
            else:
                metadata.block_table, metadata.seq_lens = view.build(cam.block_table_tensor, cam.seq_lens,
                                                                     _query_lens(cam))
            return metadata

        return build

    def flashinfer(original):
        def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
            cam = common_attn_metadata
            view = _view_for(self, cam)
            if common_prefix_len > 0:
                view.skip(cam.seq_lens, _query_lens(cam))
                return original(self, common_prefix_len, cam, fast_build)
            table, lens = view.build(cam.block_table_tensor, cam.seq_lens, _query_lens(cam))
            # the planner reads the lengths on the host: it gets the view's, copied on first use
            batch = cam.replace(block_table_tensor=table, seq_lens=lens, max_seq_len=int(lens.max()),
                                _seq_lens_cpu=None)
            return original(self, common_prefix_len, batch, fast_build)

        return build

    patched = _patch_once(TritonAttentionMetadataBuilder, "build", "_ekv_decode_view", triton)
    patched += _patch_once(FlashInferMetadataBuilder, "build", "_ekv_decode_view", flashinfer)
    return int(patched)


def install_audit_kernel() -> int:
    """Record the statistic after every attention layer of vLLM's Triton and FlashInfer backends, with
    ``EKV_AUDIT_KERNEL`` set; returns how many implementations were patched
    (runtime/block_view.py:563-596).  Call it before the engine exists.  Each launch is the same every
    step (the kernel reads the flag on the device), so graphs can capture it."""
    from vllm.v1.attention.backends.flashinfer import FlashInferImpl
    from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl

    from runtime.audit_kernel import RecordingPlane

    def recording(original):
        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
            output = original(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs)
            if attn_metadata is None:  # the engine's memory profiling runs without a batch
                return output
            view = current_view()
            if not isinstance(view.audit, RecordingPlane):
                raise RuntimeError("the audit kernel is installed, but the view records with no recording plane")
            table, lens = view.buffers
            view.audit.record(layer.layer_name, table, lens, query, kv_cache, self.scale)
            return output

        return forward

    patched = sum(_patch_once(impl, "forward", "_ekv_audit_kernel", recording)
                  for impl in (TritonAttentionImpl, FlashInferImpl))
    return int(patched)


def current_view() -> DecodeView:
    """The process's view; the engine makes it with its first attention batch."""
    if _view is None:
        raise RuntimeError("the engine has built no attention batch yet: install the decode view before "
                           "creating the engine")
    return _view


def attach_audit_plane(runner) -> DecodeView:
    """The view, after handing the audit plane the engine's KV-cache addresses
    (runtime/block_view.py:599-626).  The caches exist only once the engine has allocated them, so this
    runs at the first scheduling step.  The audit kernel numbers layers by name, so its table lists
    each named layer's cache; the compiler pass finds a layer by its cache address, in the order of
    ``runner.kv_caches``."""
    from runtime.audit_kernel import RecordingPlane

    view = current_view()
    if isinstance(_plane, RecordingPlane):
        context = runner.compilation_config.static_forward_context
        _plane.attach([context[name].kv_cache.data_ptr() for name in _plane.layer_names])
    elif _plane is not None:
        _plane.attach([cache.data_ptr() for cache in runner.kv_caches if cache is not None])
    return view
