"""Where the serving process publishes the descriptors of its statistic buffers.

Only the descriptor-file format is kept from the reference's external readers
(observe/zero_touch.py:48-63): one JSON object per line, appended, in
``$EKV_RUNTIME_DIR`` (default ``/tmp``) as ``ekv_pass_<pid>.json``, with a sibling
``ekv_coverage_<pid>.json``.
"""

from __future__ import annotations

import json
import os


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
