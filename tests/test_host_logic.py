"""Host-side logic of the drop-in modules that needs no device: DecodeView's controller-facing state
(runtime/block_view.py:133-218), Request and allocate's argument rules (observe/allocation.py:31-76),
the descriptor helpers."""

import numpy as np
import pytest

from observe import allocation
from observe.zero_touch import pub_path, read_json_lines
from runtime.block_view import DecodeView


class FakePlane:
    def set(self, on):
        pass

    def select(self, audited, token_start):
        pass


def test_view_writes_validate_their_shapes():
    view = DecodeView(rows=2, width=4, block_size=16)
    with pytest.raises(ValueError):
        view.write_row_controls(np.ones((2, 4)), np.zeros((2, 4), dtype=np.float32))
    with pytest.raises(ValueError):
        view.write_row_controls(np.ones((3, 4)))
    with pytest.raises(ValueError):
        view.write_audit_rows(np.array([True, False]))  # no plane to switch the statistic on
    with pytest.raises(ValueError):
        DecodeView(rows=2, width=4, block_size=16, prefill_audit=True)
    with pytest.raises(ValueError):
        DecodeView(rows=0, width=4, block_size=16)


def test_release_rules_and_row_moves():
    view = DecodeView(rows=2, width=4, block_size=16, audit=FakePlane())
    ask = np.array([[1, 1, 1, 1], [0, 0, 0, 0]], dtype=np.uint8)
    assert view.write_release(ask) == []  # before any audit
    view.row_audited[0] = True
    view.audited_blocks[0] = 4
    assert view.write_release(ask) == [(0, 1), (0, 2)]  # never block 0 nor the last audited block
    assert view.write_release(ask) == []
    view.reassign_rows({1: 0, 0: 1}, [], [])
    assert view.released[1].tolist() == [False, True, True, False]
    view.reassign_rows({}, [1], [])
    assert not view.released[1].any() and not view.row_audited[1] and view.audit_rows[1]


def test_request_pins_and_shares():
    r = allocation.Request(scores=np.array([0.0, 2.0, 2.0, -1.0]))
    assert r.pinned_mask().tolist() == [True, False, False, True]
    assert r.shares().tolist() == [0.0, 0.5, 0.5, 0.0]
    assert allocation.Request(scores=np.zeros(4)).shares().tolist() == [0.25] * 4


def test_allocate_argument_rules():
    reqs = [allocation.Request(scores=np.ones(5)), allocation.Request(scores=np.ones(5))]
    with pytest.raises(ValueError):
        allocation.allocate(reqs, 3, "uniform")
    with pytest.raises(ValueError):
        allocation.allocate(reqs, -1, "uniform")
    with pytest.raises(ValueError):
        allocation.allocate([allocation.Request(scores=np.ones(4), weight=2.0), reqs[0]], 5, "uniform")
    assert all(m.all() for m in allocation.allocate(reqs, 10, "uniform"))


def test_descriptor_paths(tmp_path, monkeypatch):
    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))
    path = pub_path(42)
    assert path == f"{tmp_path}/ekv_pass_42.json"
    with open(path, "w") as f:
        f.write('{"a": 1}\n\n{"b": 2}\n')
    assert read_json_lines(path) == [{"a": 1}, {"b": 2}]


def test_skip_rejects_a_batch_wider_than_the_view():
    # the per-row read counters have one slot per view row: a larger batch is refused before any
    # device work (DecodeView.skip, runtime/block_view.py:352-361)
    import torch

    view = DecodeView(rows=2, width=4, block_size=16)
    with pytest.raises(ValueError):
        view.skip(torch.tensor([16, 32, 48], dtype=torch.int32), torch.ones(3, dtype=torch.int32))


def test_uniform_keep_rejects_masks_of_another_shape():
    # the ranking reads scores and masks for every b < width, so masks must be [rows, width]
    import torch

    scores = torch.zeros(2, 8, dtype=torch.float32)
    blocks = torch.tensor([4, 8], dtype=torch.int32)
    with pytest.raises(ValueError):
        allocation.uniform_keep(scores, blocks, pinned=torch.zeros(2, 4, dtype=torch.uint8))
    with pytest.raises(ValueError):
        allocation.uniform_keep(scores, blocks, released=torch.zeros(3, 8, dtype=torch.uint8))
    with pytest.raises(ValueError):
        allocation.uniform_keep(scores, blocks, measured=torch.zeros(3, dtype=torch.uint8))


def test_device_wrappers_refuse_host_tensors_and_wrong_shapes():
    # every device wrapper checks its tensors before any launch: a host tensor or a short mask is a
    # ValueError, not a device read of a host address or past a buffer (runs without a GPU)
    import torch

    from runtime.block_view import compact_block_table, uniform_view

    s = torch.zeros(3, 8)
    n = torch.ones(3, dtype=torch.int32)
    t = torch.zeros(3, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="device"):
        allocation.uniform_keep(s, n)
    with pytest.raises(ValueError, match="device"):
        allocation.uniform_keep(s.double(), n)
    with pytest.raises(ValueError, match="device"):
        allocation.sum_keep(s, n, budget=3)
    with pytest.raises(ValueError, match="device"):
        allocation.maxmin_keep(s, n, budget=3)
    with pytest.raises(ValueError, match="device"):
        uniform_view(s, n, t, n, 16)
    with pytest.raises(ValueError, match="device"):
        compact_block_table(t, n, torch.ones(3, 8, dtype=torch.bool), 16)
    with pytest.raises(ValueError):
        allocation.uniform_keep(torch.zeros(3, 8, dtype=torch.int32), n)  # integer scores
    with pytest.raises(ValueError):
        allocation.uniform_keep(s.reshape(-1), n)  # not [rows, width]


def test_shape_checks_name_the_tensor():
    # shapes and dtypes are checked before the device: a pinned mask narrower than the scores, a
    # blocks vector of another length, weights of another dtype, rows that are not contiguous
    import torch

    s = torch.zeros(4, 8)
    n = torch.ones(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="pinned must have shape"):
        allocation.uniform_keep(s, n, pinned=torch.ones(4, 7, dtype=torch.uint8))
    with pytest.raises(ValueError, match="blocks must have shape"):
        allocation.uniform_keep(s, torch.ones(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="weights must be"):
        allocation.sum_keep(s, n, budget=4, weights=torch.ones(4, dtype=torch.float32))
    with pytest.raises(ValueError, match="contiguous"):
        allocation.uniform_keep(torch.zeros(8, 4).t(), n)
