"""The serving process's switch for the attention-share statistic.

Whatever records the statistic -- the compiler pass's instrumented kernels or this package's audit
kernel -- publishes one block of device memory per process, described by a JSON line in
``$EKV_RUNTIME_DIR/ekv_pass_<pid>.json``:

* ``stat_flag_dev``: a device ``uint32``; the recording kernels store nothing while it is 0;
* ``layer_table_dev``: a device ``uint64[tile_lse_layers]`` of per-layer KV-cache base addresses,
  through which the pass numbers the layer of a launch.

``AuditPlane`` is the engine's handle on that block (the contract of runtime/audit.py:26-113):
``attach`` writes the engine's cache addresses into the table once the caches exist, ``set`` turns
recording on for an audit step and off after it, and ``require_newest_rows`` refuses a prefill
audit unless every recording kernel stores only from the program holding a request's newest
query tokens.  Device writes go through libekv_hip.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass

import numpy as np

import ekv_hip
from observe.zero_touch import runtime_dir


@dataclass(frozen=True)
class StatBlock:
    """The device addresses of one process's published statistic block."""

    flag: int
    table: int
    layers: int


def _json_lines(path: str) -> list[dict]:
    with open(path) as f:
        return [json.loads(text) for text in f if text.strip()]


def published_block(pid: int) -> StatBlock | None:
    """The first descriptor of process ``pid`` that names a flag, or None while there is none
    (runtime/audit.py:39-53)."""
    try:
        records = _json_lines(os.path.join(runtime_dir(), f"ekv_pass_{pid}.json"))
    except FileNotFoundError:
        return None
    for record in records:
        flag = int(record.get("stat_flag_dev", 0) or 0)
        if flag:
            return StatBlock(flag, int(record["layer_table_dev"]), int(record["tile_lse_layers"]))
    return None


class AuditPlane:
    """The flag and layer table of one serving process's statistic block."""

    def __init__(self, pid: int | None = None) -> None:
        self.pid = os.getpid() if pid is None else pid
        ekv_hip.load()  # a missing library is an error at construction, not at the first audit step
        self._flag_dev = 0  # device address of the flag, 0 until known
        self._table_dev = 0  # device address of the layer table
        self._layers = 0  # entries of the layer table
        self._attached = False
        self._recording: bool | None = None  # the value last written to the flag
        self._newest_rows_ok = False

    # -- the block ---------------------------------------------------------------------------

    def _discover(self) -> bool:
        """Look the block up in the published descriptors; True once it is known."""
        block = published_block(self.pid)
        if block is None:
            return False
        self._flag_dev, self._table_dev, self._layers = block.flag, block.table, block.layers
        return True

    def _known(self) -> bool:
        return bool(self._flag_dev) or self._discover()

    def _copy_to_device(self, device: int, data: np.ndarray) -> None:
        """Write ``data``'s bytes at device address ``device`` (a synchronous copy)."""
        ekv_hip.h2d(device, np.ascontiguousarray(data).tobytes())

    # -- the engine-facing protocol ----------------------------------------------------------

    def require_newest_rows(self) -> None:
        """Refuse a prefill audit unless every kernel that records the statistic records it only from
        the program holding a request's newest query tokens (runtime/audit.py:62-81).  In a prefill step
        several programs serve one request, and each would store its own query rows into the request's
        cells.  The coverage file is read once; after a success the answer is kept."""
        if self._newest_rows_ok:
            return
        records = _json_lines(os.path.join(runtime_dir(), f"ekv_coverage_{self.pid}.json"))
        recorders = [r for r in records if int(r.get("attn_share_sites", 0) or 0)]
        if not recorders:
            raise RuntimeError("no kernel that records the attention statistic has compiled, so a prefill "
                               "step cannot be audited yet")
        every_program = [r["kernel"] for r in recorders if not int(r.get("attn_share_newest_rows", 0) or 0)]
        if every_program:
            raise RuntimeError(f"a prefill step cannot be audited: kernels {every_program} store the statistic "
                               "from every program of a request, not only the one with its newest tokens")
        self._newest_rows_ok = True

    def select(self, audited: np.ndarray, token_start: np.ndarray) -> None:
        """The rows to record next step and the token of each row's query.  The pass records every
        row its kernels see, so this plane has nothing to store."""

    def attach(self, cache_addresses: list[int]) -> bool:
        """Store the engine's per-layer KV-cache addresses in the layer table; False while no block is
        published, True once the table holds them (runtime/audit.py:86-100).  Later calls do nothing."""
        if self._attached:
            return True
        if not self._known():
            return False
        count = len(cache_addresses)
        if count > self._layers:
            raise ValueError(f"{count} KV caches do not fit the layer table of {self._layers} entries")
        entries = np.zeros(self._layers, dtype=np.uint64)
        entries[:count] = np.asarray(cache_addresses, dtype=np.uint64)
        self._copy_to_device(self._table_dev, entries)
        self._attached = True
        return True

    def set(self, on: bool) -> None:
        """Record (``on``) or not in the launches that follow (runtime/audit.py:102-113).  The flag is
        written only when the value changes; turning recording off before any block exists does
        nothing, turning it on then, or before ``attach``, is an error."""
        on = bool(on)
        if self._recording is on:
            return
        if not self._known():
            if not on:
                return
            raise RuntimeError(f"process {self.pid} has published no statistic block, so an audit step "
                               "cannot start")
        if on and not self._attached:
            raise RuntimeError("the layer table holds no KV-cache addresses yet: attach them before an "
                               "audit step")
        self._copy_to_device(self._flag_dev, np.array([int(on)], dtype=np.uint32))
        self._recording = on
