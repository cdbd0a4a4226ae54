"""Where the serving process publishes the descriptors of its statistic buffers.

Only the descriptor-file format is kept from the reference's external readers
(observe/zero_touch.py:48-63): one JSON object per line, appended, in
``$EKV_RUNTIME_DIR`` (default ``/tmp``) as ``ekv_pass_<pid>.json``, with a sibling
``ekv_coverage_<pid>.json``.  The timer readers (``find_published``, ``read_pass_cycles``) read the
per-row cycle counter a recording plane publishes there, over HIP.
"""

from __future__ import annotations

import glob
import json
import os
from dataclasses import dataclass


def runtime_dir() -> str:
    """``$EKV_RUNTIME_DIR`` when set and not blank, else ``/tmp`` (observe/zero_touch.py:48-53)."""
    directory = os.environ.get("EKV_RUNTIME_DIR", "").strip()
    return directory or "/tmp"


def pub_path(pid: int) -> str:
    """The descriptor file of process ``pid`` (observe/zero_touch.py:56-57)."""
    return os.path.join(runtime_dir(), f"ekv_pass_{pid}.json")


def read_json_lines(path: str) -> list[dict]:
    """Every record of an append-only JSON-lines file, blank lines skipped (observe/zero_touch.py:60-63)."""
    with open(path) as f:
        return [json.loads(line) for line in f if line.strip()]


_OPENED: dict[tuple[int, int], int] = {}  # (pid, timer_dev) -> this process's address of that buffer


def _opened(b: "PassBuffer") -> int:
    """Another process's timer opened once by its IPC handle."""
    import ekv_hip

    key = (b.pid, b.timer_dev)
    if key not in _OPENED:
        _OPENED[key] = ekv_hip.ipc_open(bytes.fromhex(b.timer_ipc))
    return _OPENED[key]


@dataclass(frozen=True)
class PassBuffer:
    """The fields of one published descriptor line that the timer readers use
    (observe/zero_touch.py:28-45): the process, its row count, and the timer's device buffer."""

    pid: int
    max_rows: int
    kernel: str = ""
    timer_dev: int = 0
    timer_ipc: str = ""
    timer_bytes: int = 0


def find_published(pid: int | None = None, out_dir: str | None = None) -> list[PassBuffer]:
    """Every descriptor line of process ``pid`` (every process when None) that names its pid and row
    count, in file order (observe/zero_touch.py:66-97); lines without them are skipped, as the
    reference skips them."""
    base = out_dir or runtime_dir()
    pattern = os.path.join(base, f"ekv_pass_{pid}.json" if pid else "ekv_pass_*.json")
    found = []
    for path in sorted(glob.glob(pattern)):
        try:
            records = read_json_lines(path)
        except (ValueError, OSError):
            continue
        for m in records:
            try:
                found.append(PassBuffer(int(m["pid"]), int(m["max_rows"]), str(m.get("kernel", "")),
                                        int(m.get("timer_dev", 0) or 0), str(m.get("timer_ipc", "")),
                                        int(m.get("timer_bytes", 0) or 0)))
            except (KeyError, TypeError, ValueError):
                continue
    return found


def read_pass_cycles(pid: int | None = None, kernel: str | None = None) -> dict[int, int]:
    """{row: accumulated cycles} of the first published timer (of a kernel whose name contains
    ``kernel``, when given), rows with a positive count only (observe/zero_touch.py:190-225).  The
    buffer is device memory: read with a device-to-host copy in the publishing process, through its
    IPC handle from another.  Empty when no timer is published.  Read after a completion sync: the
    counters are cumulative and written by device atomics."""
    import numpy as np

    import ekv_hip

    for b in find_published(pid):
        if not b.timer_dev or (kernel is not None and kernel not in b.kernel):
            continue
        address = b.timer_dev if b.pid == os.getpid() else _opened(b)
        size = (b.timer_bytes // 8) * 8
        counts = np.frombuffer(ekv_hip.d2h(address, size), dtype=np.int64)
        return {row: int(counts[row]) for row in range(min(b.max_rows, len(counts))) if counts[row] > 0}
    return {}
