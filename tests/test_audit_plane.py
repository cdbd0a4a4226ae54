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
