"""The serving-process side of the attention-share statistic: the audit flag and the layer table.

A recording kernel stores the statistic only while a device flag is set, and the compiler pass
numbers layers by the position of a KV-cache address in a per-layer table; both live in device
memory described by the descriptor file the recorder publishes.  ``AuditPlane`` fills the table
once the engine's caches exist and flips the flag for audit steps.  Its protocol -- ``set``,
``select``, ``attach``, ``require_newest_rows`` and their errors -- follows runtime/audit.py:26-113;
the device copies go through libekv_hip instead of libcudart.
"""

from __future__ import annotations

import json
import os

import numpy as np

import ekv_hip
from observe.zero_touch import runtime_dir


class AuditPlane:
    """Fills the layer table and switches the audit flag of one serving process."""

    def __init__(self, pid: int | None = None) -> None:
        self.pid = os.getpid() if pid is None else pid
        ekv_hip.load()  # fails here, not at the first audit step, if the library is missing
        self._flag_dev = 0
        self._table_dev = 0
        self._layers = 0
        self._table_filled = False
        self._flag_on: bool | None = None
        self._newest_rows_checked = False

    def _discover(self) -> bool:
        """Read the published descriptor of the statistic block; False until one exists
        (runtime/audit.py:39-53)."""
        path = os.path.join(runtime_dir(), f"ekv_pass_{self.pid}.json")
        try:
            with open(path) as f:
                records = [json.loads(line) for line in f if line.strip()]
        except FileNotFoundError:
            return False
        for record in records:
            if int(record.get("stat_flag_dev", 0)):
                self._flag_dev = int(record["stat_flag_dev"])
                self._table_dev = int(record["layer_table_dev"])
                self._layers = int(record["tile_lse_layers"])
                return True
        return False

    def _copy_to_device(self, device: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        ekv_hip.h2d(device, data.tobytes())

    def require_newest_rows(self) -> None:
        """Fail unless every recording kernel records only from the program holding a request's newest
        query tokens, which a prefill audit needs (runtime/audit.py:62-81).  Checked once."""
        if self._newest_rows_checked:
            return
        path = os.path.join(runtime_dir(), f"ekv_coverage_{self.pid}.json")
        with open(path) as f:
            records = [json.loads(line) for line in f if line.strip()]
        recording = [r for r in records if int(r.get("attn_share_sites", 0))]
        if not recording:
            raise RuntimeError("a prefill audit was requested before any kernel that records the statistic compiled")
        unsafe = [r["kernel"] for r in recording if not int(r.get("attn_share_newest_rows", 0))]
        if unsafe:
            raise RuntimeError(
                f"kernels {unsafe} record the statistic from every program of a request: a prefill step "
                "cannot be an audit step with them"
            )
        self._newest_rows_checked = True

    def select(self, audited: np.ndarray, token_start: np.ndarray) -> None:
        """Choose the rows to record next step.  A recorder that records every row it is given needs none."""

    def attach(self, cache_addresses: list[int]) -> bool:
        """Write each layer's KV-cache base address into the layer table; True once it is filled
        (runtime/audit.py:86-100)."""
        if self._table_filled:
            return True
        if not self._flag_dev and not self._discover():
            return False
        if len(cache_addresses) > self._layers:
            raise ValueError(
                f"the layer table holds {self._layers} layers, the engine has {len(cache_addresses)}"
            )
        table = np.zeros(self._layers, dtype=np.uint64)
        table[: len(cache_addresses)] = np.asarray(cache_addresses, dtype=np.uint64)
        self._copy_to_device(self._table_dev, table)
        self._table_filled = True
        return True

    def set(self, on: bool) -> None:
        """Turn recording on or off for the launches that follow; copies only on a change
        (runtime/audit.py:102-113)."""
        if on == self._flag_on:
            return
        if not self._flag_dev and not self._discover():
            if on:
                raise RuntimeError("an audit step was requested but no statistic buffers were published")
            return
        if on and not self._table_filled:
            raise RuntimeError("an audit step was requested before the layer table was filled")
        self._copy_to_device(self._flag_dev, np.array([1 if on else 0], dtype=np.uint32))
        self._flag_on = on
