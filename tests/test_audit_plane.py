"""AuditPlane's protocol on the host (runtime/audit.py:29-113 of the reference): the descriptor lookup,
attach's one-time table fill, set's change-only flag writes and its errors, and the prefill check
of require_newest_rows (tests/test_block_view.py:315-330 of the reference).  The device writes are
recorded instead of made, so this runs without a GPU."""

import json
import os

import numpy as np
import pytest

from runtime.audit import AuditPlane, published_block


def plane_with_writes(monkeypatch, tmp_path):
    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))
    plane = AuditPlane()
    writes = []
    monkeypatch.setattr(plane, "_copy_to_device", lambda device, data: writes.append((device, np.array(data))))
    return plane, writes


def publish(tmp_path, pid, **fields):
    with open(os.path.join(tmp_path, f"ekv_pass_{pid}.json"), "a") as f:
        f.write(json.dumps(fields) + "\n")


def test_nothing_published(monkeypatch, tmp_path):
    plane, writes = plane_with_writes(monkeypatch, tmp_path)
    assert published_block(plane.pid) is None
    assert plane.attach([1, 2]) is False
    plane.set(False)  # nothing to switch off
    with pytest.raises(RuntimeError, match="published no statistic block"):
        plane.set(True)
    assert writes == []


def test_attach_then_set_writes_on_change_only(monkeypatch, tmp_path):
    plane, writes = plane_with_writes(monkeypatch, tmp_path)
    publish(tmp_path, plane.pid, host_va=1, other=5)  # a record without a flag is skipped
    publish(tmp_path, plane.pid, stat_flag_dev=4096, layer_table_dev=8192, tile_lse_layers=3)
    with pytest.raises(RuntimeError, match="attach"):
        plane.set(True)  # the table is not filled yet
    with pytest.raises(ValueError, match="4 KV caches"):
        plane.attach([11, 12, 13, 14])
    assert plane.attach([11, 12]) is True
    assert len(writes) == 1 and writes[0][0] == 8192 and writes[0][1].tolist() == [11, 12, 0]
    assert writes[0][1].dtype == np.uint64
    assert plane.attach([99]) is True and len(writes) == 1  # filled once
    plane.set(True)
    plane.set(True)
    plane.set(np.bool_(True))
    plane.set(False)
    plane.set(False)
    plane.set(True)
    flags = [(d, w.tolist()) for d, w in writes[1:]]
    assert flags == [(4096, [1]), (4096, [0]), (4096, [1])]
    assert all(w.dtype == np.uint32 for _, w in writes[1:])


def test_newest_rows_check(monkeypatch, tmp_path):
    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))

    def outcome(entries):
        path = os.path.join(tmp_path, f"ekv_coverage_{os.getpid()}.json")
        with open(path, "w") as f:
            f.writelines(json.dumps(e) + "\n" for e in entries)
        try:
            AuditPlane().require_newest_rows()
            return "ok"
        except RuntimeError:
            return "refused"

    safe = {"kernel": "attention", "attn_share_sites": 1, "attn_share_newest_rows": 1}
    unsafe = {"kernel": "extend", "attn_share_sites": 1, "attn_share_newest_rows": 0}
    other = {"kernel": "gather", "attn_share_sites": 0}
    assert outcome([safe, other]) == "ok"
    assert outcome([safe, unsafe]) == "refused"
    assert outcome([other]) == "refused"  # nothing records yet
    plane = AuditPlane()
    with open(os.path.join(tmp_path, f"ekv_coverage_{os.getpid()}.json"), "w") as f:
        f.write(json.dumps(safe) + "\n")
    plane.require_newest_rows()
    with open(os.path.join(tmp_path, f"ekv_coverage_{os.getpid()}.json"), "w") as f:
        f.write(json.dumps(unsafe) + "\n")
    plane.require_newest_rows()  # checked once


# -- RecordingPlane's host rules, without a device ------------------------------------------------


def host_plane(rows):
    """A RecordingPlane with host tensors in place of its device buffers, for its host-side rules."""
    import torch

    from runtime.audit_kernel import RecordingPlane

    plane = RecordingPlane.__new__(RecordingPlane)
    plane.rows = rows
    plane._select = torch.zeros(rows, dtype=torch.uint8)
    plane._token = torch.zeros(rows, dtype=torch.int32)
    plane._pending = []
    plane._plan_stale = False
    return plane


def test_select_clears_the_rows_past_a_shrinking_batch():
    plane = host_plane(8)
    plane.select(np.ones(8, bool), np.arange(8) * 3)
    assert plane._select.tolist() == [1] * 8 and plane._token.tolist() == [0, 3, 6, 9, 12, 15, 18, 21]
    plane._plan_stale = False
    plane.select(np.array([1, 0, 1, 1], bool), np.array([5, 6, 7, 8]))
    # rows 4-7 are no longer selected and their old query tokens are gone
    assert plane._select.tolist() == [1, 0, 1, 1, 0, 0, 0, 0]
    assert plane._token.tolist() == [5, 6, 7, 8, 0, 0, 0, 0]
    assert plane._plan_stale  # the next record rebuilds the step plan
    plane.select(np.zeros(0, bool), np.zeros(0, np.int64))
    assert plane._select.tolist() == [0] * 8
    with pytest.raises(ValueError, match="exceed"):
        plane.select(np.ones(9, bool), np.arange(9))
    with pytest.raises(ValueError, match="query tokens"):
        plane.select(np.ones(4, bool), np.arange(3))


def test_a_statistic_block_of_2_gib_is_refused_before_allocating():
    from runtime.audit_kernel import IPC_LIMIT_BYTES, RecordingPlane

    # 32 layers x 256 rows x 8192 blocks x 4 query rows x 2 planes x 4 B = 2.15 GB: refused with the limit named
    with pytest.raises(ValueError, match=str(IPC_LIMIT_BYTES)):
        RecordingPlane(32, 256, 8192, 4, 16)
    # one cell fewer per block stays under it (the size rule alone; not constructed here)
    assert 2 * 32 * 256 * 8192 * 3 * 4 < IPC_LIMIT_BYTES
    with pytest.raises(ValueError, match="IPC"):
        RecordingPlane(1, 1 << 16, 1 << 12, 2, 16)  # exactly 2 GiB


def test_the_timer_is_published_with_the_keys_its_readers_need(monkeypatch, tmp_path):
    """The timer's descriptor line carries pid, kernel, max_rows, timer_dev, timer_ipc and
    timer_bytes (mlir_pass/lib/eKVTimer.cpp:588-590), on a line of its own, and the readers find it."""
    import ekv_hip
    from observe.zero_touch import find_published
    from runtime.audit_kernel import RecordingPlane

    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))
    monkeypatch.setattr(ekv_hip, "ipc_handle", lambda address: address.to_bytes(64, "little"))
    plane = RecordingPlane.__new__(RecordingPlane)
    plane.pid = 4242
    plane.rows, plane.width, plane._layers, plane.cells = 6, 10, 3, 4
    plane._lse, plane._flag_dev, plane._table_dev, plane._cycles_dev = 1 << 20, 1 << 21, 1 << 22, 1 << 23
    plane._publish()
    lines = [json.loads(t) for t in open(os.path.join(tmp_path, "ekv_pass_4242.json"))]
    assert len(lines) == 2
    stat, timer = lines
    assert "pid" not in stat and "timer_dev" not in stat  # a capture-buffer reader never takes the planes
    assert stat["tile_lse_dev"] == 1 << 20 and stat["stat_flag_dev"] == 1 << 21
    assert timer["pid"] == 4242 and timer["max_rows"] == 6 and timer["timer_dev"] == 1 << 23
    assert timer["timer_bytes"] == 6 * 8 and timer["kernel"] == "ekv_audit_tile_lse"
    assert bytes.fromhex(timer["timer_ipc"]) == (1 << 23).to_bytes(64, "little")
    found = find_published(4242)
    assert len(found) == 1 and found[0].timer_dev == 1 << 23 and found[0].timer_bytes == 48
    assert found[0].max_rows == 6 and found[0].pid == 4242
    # no timer: only the statistic line
    plane._cycles_dev = 0
    plane.pid = 4243
    plane._publish()
    assert find_published(4243) == []
