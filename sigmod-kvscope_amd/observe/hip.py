"""The part of the HIP runtime a controller process needs: open another process's device buffer
by IPC handle and copy device memory to the host.

It stands where observe/cuda.py:12-58 stands in the reference, with the same methods, so the
readers that take a ``cuda`` object (``observe.tile_shares.read_tile_rows``) take this one.
"""

from __future__ import annotations

import ctypes

import ekv_hip


class Hip:
    def __init__(self) -> None:
        count = ctypes.c_int(0)
        ekv_hip.call("ekv_device_count", ctypes.byref(count))
        if count.value < 1:
            raise RuntimeError("no HIP device is visible")

    def ipc_open(self, hex_handle: str) -> int:
        """The local address of another process's allocation, from its 64-byte handle in hex."""
        raw = bytes.fromhex(hex_handle)
        if len(raw) != 64:
            raise ValueError(f"an IPC handle has 64 bytes, got {len(raw)}")
        return ekv_hip.ipc_open(raw)

    def d2h(self, dev: int, n_bytes: int) -> bytes:
        return ekv_hip.d2h(dev, n_bytes)

    def d2h_many(self, requests: list[tuple[int, int]]) -> list[bytes]:
        return [ekv_hip.d2h(dev, size) for dev, size in requests]
