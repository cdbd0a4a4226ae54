"""The cycle readers in a process of their own, reading another process's audit timer through its
published descriptor and IPC handle (observe/zero_touch.py:190-225, observe/capture.py:77-99 of the
reference).  Run by tests/test_gpu_timer_readers.py: prints the baseline read as one JSON line, waits
for a line on stdin (the serving process ran another step), then prints the deltas."""

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for path in (os.path.join(ROOT, "sigmod-kvscope_amd"), ROOT):
    sys.path.insert(0, path)

from observe.capture import Capture  # noqa: E402
from observe.zero_touch import read_pass_cycles  # noqa: E402


def main() -> None:
    pid = int(sys.argv[1])
    capture = Capture(pid)
    baseline = capture.cycle_deltas()  # the first call takes the baseline
    print(json.dumps({"baseline": baseline, "cycles": read_pass_cycles(pid, kernel="ekv_audit")}), flush=True)
    sys.stdin.readline()
    print(json.dumps({"deltas": capture.cycle_deltas(), "cycles": read_pass_cycles(pid)}), flush=True)


if __name__ == "__main__":
    main()
