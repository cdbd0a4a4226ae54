"""A per-request view of the block table for decode attention (runtime/block_view.py:1-15).

A paged attention kernel reads a request's KV cache through its block-table row and its length,
so a shorter row with a shorter length is a read budget the kernel enforces unchanged.  The view
is exact for full causal attention.  ``DecodeView`` holds the committed policy and gives every
batch its view: identity before a commit, after the lease expires, for audited rows and for
prefilling rows; released blocks are never read.  The device work of a step -- composing the
keep mask, the stable compaction of every row, the view lengths and the five read counters -- is
one launch of ``ekv_build_view`` writing into persistent buffers that captured graphs read.
"""

from __future__ import annotations

import os
import time
from collections.abc import Callable
from typing import Protocol

import numpy as np
import torch

import ekv_hip
from runtime.audit import AuditPlane


class StatisticSwitch(Protocol):
    """What the view needs to turn the statistic on for a step and off after it (runtime/block_view.py:28-33)."""

    def set(self, on: bool) -> None: ...

    def select(self, audited: np.ndarray, token_start: np.ndarray) -> None: ...


def _check_table(table: torch.Tensor, seq_lens: torch.Tensor) -> None:
    if not (table.is_cuda and seq_lens.is_cuda):
        raise ValueError("the block table and lengths must be device tensors")
    if table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("the block table and lengths must be int32")
    if table.ndim != 2 or table.stride(1) != 1 or seq_lens.ndim != 1 or seq_lens.stride(0) != 1:
        raise ValueError("the block table rows and the lengths must be contiguous")
    if seq_lens.shape[0] < table.shape[0]:
        raise ValueError("one length per table row is needed")


def compact_block_table(
    table: torch.Tensor, seq_lens: torch.Tensor, keep: torch.Tensor, block_size: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """The view of each row that keeps the blocks marked in ``keep`` (runtime/block_view.py:36-56).

    The first and last block of every request are always kept; kept blocks stay in their order at
    the front of the row and the dropped ones follow in their order; the length is the kept blocks
    times ``block_size`` less the unfilled part of the last block, 0 for a row without tokens."""
    _check_table(table, seq_lens)
    rows, width = int(table.shape[0]), int(table.shape[1])
    if keep.shape != (rows, width) or keep.dtype not in (torch.bool, torch.uint8) or keep.stride(1) != 1:
        raise ValueError("keep must be a bool [rows, width] mask with contiguous rows")
    if not keep.is_cuda:
        raise ValueError("keep must be a device tensor")
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
    _check_table(table, seq_lens)
    rows, width = int(scores.shape[0]), int(scores.shape[1])
    if scores.dtype != torch.float32 or scores.stride(1) != 1 or not scores.is_cuda:
        raise ValueError("scores must be a float32 device tensor with contiguous rows")
    if table.shape != (rows, width):
        raise ValueError("the block table must be [rows, width] like scores")
    if blocks.dtype != torch.int32 or blocks.shape != (rows,):
        raise ValueError("blocks must be int32 [rows]")
    if measured is not None and (measured.dtype not in (torch.uint8, torch.bool) or measured.shape != (rows,)):
        raise ValueError("measured must be a uint8 / bool [rows] mask")
    if pin_from is not None and (pin_from.dtype != torch.int32 or pin_from.shape != (rows,)):
        raise ValueError("pin_from must be int32 [rows]")
    if counts is not None and (counts.dtype != torch.int64 or counts.shape != (rows, 5) or not counts.is_contiguous()):
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


class DecodeView:
    """The committed read policy of one serving process and the view it gives each decode batch
    (runtime/block_view.py:59-401)."""

    COUNTERS = ("read", "full", "audit", "untrimmed", "expired")

    def __init__(
        self,
        rows: int,
        width: int,
        block_size: int,
        audit: StatisticSwitch | None = None,
        prefill_audit: bool = False,
    ) -> None:
        if min(rows, width, block_size) <= 0:
            raise ValueError("view dimensions must be positive")
        if prefill_audit and audit is None:
            raise ValueError("an audit in the last prefill step needs an audit plane")
        self.rows, self.width, self.block_size = rows, width, block_size
        self.audit = audit
        self.prefill_audit = prefill_audit
        self.final_prefill = np.zeros(rows, dtype=bool)  # rows computing the last tokens of their prompt next
        self.on_prefill_audit: Callable[[], None] | None = None
        self.keep = np.ones((rows, width), dtype=bool)
        # blocks the engine took back: never read again, under any policy
        self.released = np.zeros((rows, width), dtype=bool)
        self.released_version = 0
        self.row_audited = np.zeros(rows, dtype=bool)
        self.audited_blocks = np.zeros(rows, dtype=np.int64)
        self._pending_blocks = np.zeros(rows, dtype=np.int64)
        self.audit_rows = np.zeros(rows, dtype=bool)
        self.last_audit_rows = np.zeros(rows, dtype=bool)
        self.deadline_ns = 0
        self.version = 0
        self.audit_step = False
        self.audits_completed = 0
        self.audits_started = 0
        self.on_audit_start: Callable[[], None] | None = None
        self.audit_gate: Callable[[], bool] | None = None
        self.before_build: Callable[[], None] | None = None
        self._audit_pending = False
        self._pending_rows = np.zeros(rows, dtype=bool)
        self._device: torch.device | None = None
        self._counts: torch.Tensor | None = None
        self._device_keep: torch.Tensor | None = None
        self._device_version = -1
        self._device_released: torch.Tensor | None = None
        self._released_device_version = -1
        self._audited_dev: torch.Tensor | None = None
        self._decoding_dev: torch.Tensor | None = None
        self._table: torch.Tensor | None = None
        self._lens: torch.Tensor | None = None

    # -- the controller-facing writes (runtime/block_view.py:133-218) -----------------------------

    def write_row_controls(self, mask: np.ndarray, log_weight: np.ndarray | None = None) -> int:
        """Commit one generation: ``mask[row, block]`` nonzero reads the block."""
        if log_weight is not None:
            raise ValueError("a block-table view enforces hard keep decisions only")
        mask = np.asarray(mask)
        if mask.shape != self.keep.shape:
            raise ValueError(f"mask shape {mask.shape} != view shape {self.keep.shape}")
        self.keep = mask != 0
        self.version += 1
        return 1

    def write_lease_deadline(self, deadline_ns: int) -> int:
        self.deadline_ns = int(deadline_ns)
        return 1

    def write_audit_rows(self, requested: np.ndarray) -> int:
        """Ask for an audit of the marked rows; each request is consumed by one decode step."""
        requested = np.asarray(requested, dtype=bool)
        if requested.shape != self.audit_rows.shape:
            raise ValueError(f"audit shape {requested.shape} != {self.audit_rows.shape}")
        if requested.any() and self.audit is None:
            raise ValueError("an audit was requested but the view has no audit plane to switch the statistic on")
        self.audit_rows |= requested
        return 1

    def write_final_prefill(self, rows: np.ndarray) -> None:
        rows = np.asarray(rows, dtype=bool)
        if rows.shape[0] > self.rows:
            raise ValueError(f"{rows.shape[0]} rows exceed the view's {self.rows}")
        self.final_prefill[:] = False
        self.final_prefill[: rows.shape[0]] = rows

    def write_release(self, mask: np.ndarray) -> list[tuple[int, int]]:
        """Mark blocks released; returns the new ``(row, block)`` pairs.  Only blocks an audit of the
        row's current request covered, never block 0 nor the last block at that audit."""
        mask = np.asarray(mask) != 0
        if mask.shape != self.released.shape:
            raise ValueError(f"release shape {mask.shape} != view shape {self.released.shape}")
        eligible = np.zeros_like(mask)
        for row in np.flatnonzero(self.row_audited):
            eligible[row, : max(int(self.audited_blocks[row]) - 1, 0)] = True
        eligible[:, 0] = False
        new = mask & eligible & ~self.released
        rows, blocks = np.nonzero(new)
        if rows.size:
            self.released |= new
            self.released_version += 1
        return [(int(r), int(b)) for r, b in zip(rows, blocks)]

    def reassign_rows(self, moved: dict[int, int], new: list[int], empty: list[int]) -> None:
        """The scheduler moved requests between rows: ``moved[row] = old_row``; ``new`` rows hold new
        requests (full reads, audited at their first decode step with a plane); ``empty`` rows none."""
        keep, audit = self.keep.copy(), self.audit_rows.copy()
        released, audited, blocks = self.released.copy(), self.row_audited.copy(), self.audited_blocks.copy()
        for row, old in moved.items():
            keep[row], audit[row] = self.keep[old], self.audit_rows[old]
            released[row], audited[row], blocks[row] = self.released[old], self.row_audited[old], self.audited_blocks[old]
        for row in new:
            keep[row], audit[row] = True, self.audit is not None
            released[row], audited[row], blocks[row] = False, False, 0
        for row in empty:
            keep[row], audit[row] = True, False
            released[row], audited[row], blocks[row] = False, False, 0
        self.keep, self.audit_rows = keep, audit
        if (released != self.released).any():
            self.released_version += 1
        self.released, self.row_audited, self.audited_blocks = released, audited, blocks
        self.version += 1

    # -- the engine-facing view ---------------------------------------------------------------

    def active(self) -> bool:
        return self.deadline_ns > time.monotonic_ns()

    def _ensure_device(self, device: torch.device) -> None:
        if self._table is None:
            self._device = device
            self._table = torch.zeros(self.rows, self.width, dtype=torch.int32, device=device)
            self._lens = torch.zeros(self.rows, dtype=torch.int32, device=device)
            # per-row counters (ekv_build_view adds each row's to its own slot); totals are column sums
            self._counts = torch.zeros(self.rows, len(self.COUNTERS), dtype=torch.int64, device=device)
            self._audited_dev = torch.zeros(self.rows, dtype=torch.uint8, device=device)
            self._decoding_dev = torch.ones(self.rows, dtype=torch.uint8, device=device)

    def build(
        self, table: torch.Tensor, seq_lens: torch.Tensor, query_lens: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """The view buffers (table, lengths) for a batch of ``len(query_lens)`` rows
        (runtime/block_view.py:225-295).  A row computing one token decodes and gets its view; a row
        computing more prefills and reads its whole table."""
        if self.before_build is not None:
            self.before_build()
        live = self.active()  # one reading of the lease decides the step
        self.finish_audit()
        _check_table(table, seq_lens)
        num_reqs = len(query_lens)
        width = int(table.shape[1])
        if width != self.width or num_reqs > self.rows:
            raise ValueError(f"batch ({num_reqs} rows, {width} blocks) exceeds view ({self.rows}, {self.width})")
        self._ensure_device(table.device)
        assert self._table is not None and self._lens is not None and self._counts is not None
        decode = np.asarray(query_lens.numpy() == 1)
        all_decode = bool(decode.all())
        servable = decode | (self.final_prefill[:num_reqs] & self.prefill_audit)
        self.final_prefill[:] = False
        audited = np.zeros(self.rows, dtype=bool)
        audited[:num_reqs] = self.audit_rows[:num_reqs] & servable
        if audited.any() and not self.may_audit():
            audited[:] = False
        if (audited[:num_reqs] & ~decode).any() and self.on_prefill_audit is not None:
            self.on_prefill_audit()
        self.audit_rows[audited] = False
        self.audit_step = bool(audited.any())
        self._audit_pending = self.audit_step
        self._pending_rows = audited
        if self.audit_step:
            self.start_audit()
            size = self.block_size
            self._pending_blocks[:num_reqs] = ((seq_lens[:num_reqs] + size - 1) // size).cpu().numpy()
        if self.audit is not None:
            starts = np.concatenate(([0], np.cumsum(query_lens.numpy())[:-1]))
            self.audit.select(audited[:num_reqs], starts)
            self.audit.set(self.audit_step)
        if num_reqs == 0:
            return self._table[:0], self._lens[:0]
        committed = self._keep_on(table.device)
        released = self._released_on(table.device) if self.released.any() else None
        audited_dev = None
        if self.audit_step:
            self._audited_dev[:num_reqs].copy_(torch.from_numpy(audited[:num_reqs].astype(np.uint8)))
            audited_dev = self._audited_dev
        decoding_dev = None
        if not all_decode:
            self._decoding_dev[:num_reqs].copy_(torch.from_numpy(decode.astype(np.uint8)))
            decoding_dev = self._decoding_dev
        ekv_hip.call(
            "ekv_build_view",
            table.data_ptr(), table.stride(0), seq_lens.data_ptr(),
            committed.data_ptr(), committed.stride(0),
            ekv_hip.ptr(released), released.stride(0) if released is not None else 0,
            ekv_hip.ptr(audited_dev), ekv_hip.ptr(decoding_dev), int(live),
            num_reqs, width, self.block_size,
            self._table.data_ptr(), self._table.stride(0), self._lens.data_ptr(), self._counts.data_ptr(),
            ekv_hip.stream_handle(),
        )
        return self._table[:num_reqs], self._lens[:num_reqs]

    @property
    def buffers(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The view's table and lengths: the buffers the engine's kernels read and graphs capture."""
        if self._table is None or self._lens is None:
            raise RuntimeError("the view has built no batch yet")
        return self._table, self._lens

    def reads(self) -> tuple[int, int]:
        """The blocks read and the blocks full reads would have read, over every decode step."""
        if self._counts is None:
            return 0, 0
        values = self._counts.sum(dim=0).tolist()
        return int(values[0]), int(values[1])

    def read_breakdown(self) -> dict[str, int]:
        if self._counts is None:
            return dict.fromkeys(self.COUNTERS, 0)
        return dict(zip(self.COUNTERS, (int(x) for x in self._counts.sum(dim=0).tolist())))

    def skip(self, seq_lens: torch.Tensor, query_lens: torch.Tensor) -> None:
        """A shared-prefix batch reads the engine's table and records nothing; its decode rows count as
        full reads (runtime/block_view.py:352-361)."""
        self.finish_audit()
        self.audit_step = False
        if self.audit is not None:
            self.audit.set(False)
        num_reqs = len(query_lens)
        if num_reqs == 0:
            return
        if num_reqs > self.rows:
            raise ValueError(f"batch of {num_reqs} rows exceeds the view's {self.rows} rows")
        self._ensure_device(seq_lens.device)
        assert self._counts is not None and self._decoding_dev is not None
        decode = np.asarray(query_lens.numpy() == 1)
        self._decoding_dev[:num_reqs].copy_(torch.from_numpy(decode.astype(np.uint8)))
        lens = seq_lens[:num_reqs].to(torch.int32).contiguous()
        # no table: every row reads in full and only the counters move
        ekv_hip.call(
            "ekv_build_view",
            0, 0, lens.data_ptr(), 0, 0, 0, 0, 0, self._decoding_dev.data_ptr(), 1,
            num_reqs, 1, self.block_size, 0, 0, 0, self._counts.data_ptr(), ekv_hip.stream_handle(),
        )

    def may_audit(self) -> bool:
        return self.audit_gate is None or self.audit_gate()

    def start_audit(self) -> None:
        self.audits_started += 1
        if self.on_audit_start is not None:
            self.on_audit_start()

    def finish_audit(self) -> None:
        """Count the previous step as a completed audit once the device has written it; only audit
        steps pay the synchronisation (runtime/block_view.py:373-389)."""
        if not self._audit_pending:
            return
        if self._device is not None and self._device.type == "cuda":
            torch.cuda.synchronize(self._device)
        self.last_audit_rows = self._pending_rows
        self.row_audited |= self._pending_rows
        self.audited_blocks[self._pending_rows] = self._pending_blocks[self._pending_rows]
        self.audits_completed += 1
        self._audit_pending = False

    def _keep_on(self, device: torch.device) -> torch.Tensor:
        if self._device_keep is None or self._device_version != self.version:
            self._device_keep = torch.from_numpy(self.keep.astype(np.uint8)).to(device)
            self._device_version = self.version
        return self._device_keep

    def _released_on(self, device: torch.device) -> torch.Tensor:
        if self._device_released is None or self._released_device_version != self.released_version:
            self._device_released = torch.from_numpy(self.released.astype(np.uint8)).to(device)
            self._released_device_version = self.released_version
        return self._device_released


# -- engine installation (vLLM glue; runtime/block_view.py:404-626) --------------------------------

_view: DecodeView | None = None
_plane: AuditPlane | None = None
_layers: tuple[str, ...] = ()


def _enabled(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0", "false")


def _audit_plane(builder, cam) -> AuditPlane | None:
    """The plane that records the statistic: the audit kernel's (``EKV_AUDIT_KERNEL``), the pass's
    (``EKV_ATTN_SHARE``) or none; asking for both is an error."""
    if _enabled("EKV_ATTN_SHARE") and _enabled("EKV_AUDIT_KERNEL"):
        raise RuntimeError("EKV_ATTN_SHARE and EKV_AUDIT_KERNEL both record the statistic: set one")
    if _enabled("EKV_AUDIT_KERNEL"):
        from runtime.audit_kernel import RecordingPlane

        model, parallel = builder.vllm_config.model_config, builder.vllm_config.parallel_config
        return RecordingPlane(
            layers=model.get_num_layers_by_block_type(parallel, "attention"),
            rows=builder.vllm_config.scheduler_config.max_num_seqs,
            width=cam.block_table_tensor.shape[1],
            group_rows=model.get_num_attention_heads(parallel) // model.get_num_kv_heads(parallel),
            block_size=builder.kv_cache_spec.block_size,
        )
    return AuditPlane() if _enabled("EKV_ATTN_SHARE") else None


def require_supported_attention(builder) -> None:
    """Refuse a cache group the view cannot trim exactly: anything but plain full causal decoder
    self-attention in one cache group (runtime/block_view.py:436-469)."""
    from vllm.v1.attention.backend import AttentionType
    from vllm.v1.kv_cache_interface import FullAttentionSpec

    spec = builder.kv_cache_spec
    if type(spec) is not FullAttentionSpec:
        raise RuntimeError(f"the view supports full causal attention only; this cache group is {type(spec).__name__}")
    if spec.sliding_window is not None or spec.attention_chunk_size is not None:
        raise RuntimeError("the view does not support a sliding window or chunked attention in a cache group")
    layers = builder.vllm_config.compilation_config.static_forward_context
    for name in builder.layer_names:
        layer = layers[name]
        if layer.sliding_window is not None:
            raise RuntimeError(f"layer {name} has a sliding window: the view cannot trim its blocks exactly")
        if getattr(layer.impl, "alibi_slopes", None) is not None:
            raise RuntimeError(f"layer {name} has a position bias (ALiBi): the view cannot trim its blocks")
        if layer.attn_type != AttentionType.DECODER:
            raise RuntimeError(f"layer {name} is {layer.attn_type.value} attention: the view supports decoder attention")


def _view_for(builder, cam) -> DecodeView:
    """The process's view, created by the first batch with the engine's rows, width and block size."""
    global _view, _plane, _layers
    layers = tuple(builder.layer_names)
    if _view is None:
        require_supported_attention(builder)
        _plane = _audit_plane(builder, cam)
        prefill_audit = _enabled("EKV_PREFILL_AUDIT")
        if prefill_audit and not _enabled("EKV_ATTN_SHARE"):
            raise RuntimeError("EKV_PREFILL_AUDIT needs the compiler pass's statistic (EKV_ATTN_SHARE)")
        _view = DecodeView(
            rows=builder.vllm_config.scheduler_config.max_num_seqs,
            width=cam.block_table_tensor.shape[1],
            block_size=builder.kv_cache_spec.block_size,
            audit=_plane,
            prefill_audit=prefill_audit,
        )
        if prefill_audit:
            assert _plane is not None
            _view.on_prefill_audit = _plane.require_newest_rows
        _layers = layers
    if layers != _layers:
        raise RuntimeError("a block-table view supports one KV-cache group; this model has several")
    return _view


def _query_lens(cam) -> torch.Tensor:
    starts = cam.query_start_loc_cpu[: cam.num_reqs + 1]
    return starts[1:] - starts[:-1]


def install_decode_view() -> int:
    """Give every attention batch of the Triton and FlashInfer backends its view; returns the builders
    patched (runtime/block_view.py:504-560).  Install before the engine is created."""
    from vllm.v1.attention.backends.flashinfer import FlashInferMetadataBuilder
    from vllm.v1.attention.backends.triton_attn import TritonAttentionMetadataBuilder

    patched = 0
    triton_build = TritonAttentionMetadataBuilder.build
    if not getattr(triton_build, "_ekv_decode_view", False):

        def build_triton(self, common_prefix_len, common_attn_metadata, fast_build=False):
            metadata = triton_build(self, common_prefix_len, common_attn_metadata, fast_build)
            cam = common_attn_metadata
            view = _view_for(self, cam)
            if common_prefix_len > 0:
                view.skip(cam.seq_lens, _query_lens(cam))
                return metadata
            metadata.block_table, metadata.seq_lens = view.build(cam.block_table_tensor, cam.seq_lens, _query_lens(cam))
            return metadata

        build_triton._ekv_decode_view = True  # type: ignore[attr-defined]
        TritonAttentionMetadataBuilder.build = build_triton
        patched += 1

    flashinfer_build = FlashInferMetadataBuilder.build
    if not getattr(flashinfer_build, "_ekv_decode_view", False):

        def build_flashinfer(self, common_prefix_len, common_attn_metadata, fast_build=False):
            cam = common_attn_metadata
            view = _view_for(self, cam)
            if common_prefix_len > 0:
                view.skip(cam.seq_lens, _query_lens(cam))
                return flashinfer_build(self, common_prefix_len, cam, fast_build)
            table, lens = view.build(cam.block_table_tensor, cam.seq_lens, _query_lens(cam))
            seen = cam.replace(block_table_tensor=table, seq_lens=lens, max_seq_len=int(lens.max()), _seq_lens_cpu=None)
            return flashinfer_build(self, common_prefix_len, seen, fast_build)

        build_flashinfer._ekv_decode_view = True  # type: ignore[attr-defined]
        FlashInferMetadataBuilder.build = build_flashinfer
        patched += 1
    return patched


def install_audit_kernel() -> int:
    """Record the statistic after each attention layer of the Triton and FlashInfer backends; returns
    the implementations patched (runtime/block_view.py:563-596)."""
    from vllm.v1.attention.backends.flashinfer import FlashInferImpl
    from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl

    from runtime.audit_kernel import RecordingPlane

    patched = 0
    for impl in (TritonAttentionImpl, FlashInferImpl):
        original = impl.forward
        if getattr(original, "_ekv_audit_kernel", False):
            continue

        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, _original=original, **kwargs):
            output = _original(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs)
            if attn_metadata is not None:  # a profiling run has no batch
                view = current_view()
                if not isinstance(view.audit, RecordingPlane):
                    raise RuntimeError("the audit kernel is installed but the view has no recording plane")
                table, lens = view.buffers
                view.audit.record(layer.layer_name, table, lens, query, kv_cache, self.scale)
            return output

        forward._ekv_audit_kernel = True  # type: ignore[attr-defined]
        impl.forward = forward
        patched += 1
    return patched


def current_view() -> DecodeView:
    """The process's view; it exists once the engine has built its first attention batch."""
    if _view is None:
        raise RuntimeError("no attention batch has been built: install the decode view before the engine starts")
    return _view


def attach_audit_plane(runner) -> DecodeView:
    """The view, with the audit plane given the engine's KV-cache addresses (runtime/block_view.py:608-626)."""
    from runtime.audit_kernel import RecordingPlane

    view = current_view()
    if isinstance(_plane, RecordingPlane):
        layers = runner.compilation_config.static_forward_context
        _plane.attach([layers[name].kv_cache.data_ptr() for name in _plane.layer_names])
    elif _plane is not None:
        _plane.attach([cache.data_ptr() for cache in runner.kv_caches if cache is not None])
    return view
