"""The controller side of the cross-process share test: read another process's statistic planes
by IPC handle and write the live rows' shares, normalised on this process's device, to a .npy
file (observe/controller.py:92-136 of the reference reads them the same way, on the host).

Usage: python ipc_controller.py <serving pid> <out.npy> <row blocks, comma separated>"""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "sigmod-kvscope_amd"))
sys.path.insert(0, ROOT)

from observe.hip import Hip  # noqa: E402
from observe.tile_shares import DeviceTileShareSource, share_descriptor  # noqa: E402


def main() -> None:
    pid, out = int(sys.argv[1]), sys.argv[2]
    row_blocks = np.array([int(x) for x in sys.argv[3].split(",")])
    entry = share_descriptor(pid)
    source = DeviceTileShareSource(Hip(), entry, pid)
    assert source.base != int(entry["tile_lse_dev"]) or pid == os.getpid()
    np.save(out, source.read(len(row_blocks), row_blocks))


if __name__ == "__main__":
    main()
