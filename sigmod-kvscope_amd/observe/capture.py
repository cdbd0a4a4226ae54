"""The per-row cycle deltas of a serving process's audit timer, for a reader in that process or in
another one (the cycle half of observe/capture.py:24-99; the capture-buffer half belongs to the
compiler pass, which this package does not build).

A recording plane with a timer publishes a descriptor line with ``timer_dev``, ``timer_ipc`` and
``timer_bytes``.  ``Capture.cycle_deltas`` reads every such buffer (directly in the serving process,
through its IPC handle from another) and returns the cycles each row gained since the previous call.
"""

from __future__ import annotations

import os

import numpy as np

from observe.hip import Hip
from observe.zero_touch import pub_path, read_json_lines


class Capture:
    def __init__(self, pid: int) -> None:
        self.pid = pid
        self.local = pid == os.getpid()
        self.hip = Hip()
        self._timers: dict[int, int] = {}  # the descriptor's timer address -> this process's address
        self._previous: dict[int, np.ndarray] = {}

    def _entries(self, key: str) -> list[dict]:
        """The process's descriptor lines that carry a non-zero ``key`` (observe/capture.py:31-33)."""
        try:
            records = read_json_lines(pub_path(self.pid))
        except FileNotFoundError:
            return []
        return [e for e in records if int(e.get(key, 0) or 0)]

    def _read(self, entry: dict) -> tuple[int, np.ndarray]:
        """The current counts of one published timer, keyed by its address in the serving process."""
        key = int(entry["timer_dev"])
        if key not in self._timers:
            self._timers[key] = key if self.local else self.hip.ipc_open(str(entry["timer_ipc"]))
        size = int(entry["timer_bytes"]) // 8 * 8
        return key, np.frombuffer(self.hip.d2h(self._timers[key], size), dtype=np.int64).copy()

    def cycle_deltas(self) -> dict[int, int]:
        """{row: cycles} gained since the previous call, rows that gained only (observe/capture.py:77-99).
        The first read of a timer is its baseline and adds nothing; a line without ``timer_bytes`` is
        skipped."""
        gained = np.zeros(0, dtype=np.int64)
        for entry in self._entries("timer_dev"):
            if not int(entry.get("timer_bytes", 0) or 0):
                continue
            key, now = self._read(entry)
            before, self._previous[key] = self._previous.get(key), now
            if before is None:
                continue
            step = np.maximum(now - before, 0)
            if len(step) > len(gained):
                gained = np.concatenate([gained, np.zeros(len(step) - len(gained), dtype=np.int64)])
            gained[: len(step)] += step
        return {int(row): int(gained[row]) for row in np.flatnonzero(gained)}
