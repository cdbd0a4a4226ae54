"""The engine's audit-step protocol with a real recording plane, on the GPU: DecodeView.build selects the
audited rows and switches the flag through AuditPlane.set, the layers record into the plane through
the view's buffers, and the next build completes the audit and switches the flag off
(runtime/block_view.py:225-295, 373-389; runtime/audit.py:86-113; runtime/audit_kernel.py:190-222)."""

import time

import numpy as np
import pytest
import torch

import workloads
from oracle import audit as oa
from oracle import tile_shares as ots
from runtime.audit_kernel import RecordingPlane
from runtime.block_view import DecodeView

pytestmark = pytest.mark.gpu


def test_audit_step_through_the_view():
    batch, kv, q = workloads.config1()
    layers, rows = 3, batch.rows
    kv_t = torch.from_numpy(kv).to(torch.bfloat16).cuda()
    q_t = torch.from_numpy(q).to(torch.bfloat16).cuda()
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    plane = RecordingPlane(layers, rows, batch.width, batch.group_rows, batch.block_size)
    flag_writes = []
    copy = plane._copy_to_device

    def counted(device, data):
        if device == plane._flag_dev:
            flag_writes.append(int(np.asarray(data).reshape(-1)[0]))
        copy(device, data)

    plane._copy_to_device = counted
    with pytest.raises(RuntimeError, match="attach"):
        plane.set(True)  # the layer table is empty
    assert flag_writes == []
    view = DecodeView(rows, batch.width, batch.block_size, audit=plane)
    assert plane.attach([kv_t.data_ptr()] * layers)
    view.write_lease_deadline(time.monotonic_ns() + 3600 * 10**9)
    committed = np.zeros((rows, batch.width), dtype=np.uint8)
    committed[:, ::2] = 1  # a live policy that drops every other block
    view.write_row_controls(committed)
    audited = np.array([True, False, True, False])
    view.write_audit_rows(audited)
    decode = torch.ones(rows, dtype=torch.int32)

    def step():
        t, l = view.build(table, lens, decode)
        for layer in range(layers):
            plane.record(f"model.layers.{layer}.attn", t, l, q_t, kv_t, scale)
        torch.cuda.synchronize()
        return plane.read_planes().copy()

    got = step()  # the audit step: rows 0 and 2 read every block and are recorded
    assert view.audit_step and flag_writes == [1]
    want = oa.new_planes(layers, rows, batch.width, batch.group_rows)
    kvh, qh = kv_t.float().cpu().numpy(), q_t.float().cpu().numpy()
    for layer in range(layers):
        oa.tile_lse(want, qh, kvh[:, 0], batch.table, batch.lens, np.arange(rows), audited, 1, layer, scale,
                    batch.block_size, batch.group_rows, [layer % batch.kv_heads])
    assert np.array_equal(np.isnan(got), np.isnan(want)), "the audited rows' cells differ"
    live = ~np.isnan(want[0])
    du = np.abs(ots.log_weights(got[0], got[1], 1)[live] - ots.log_weights(want[0], want[1], 1)[live]).max()
    assert du < 1e-3
    assert np.isnan(got[:, :, 1]).all() and np.isnan(got[:, :, 3]).all(), "an unaudited row was recorded"

    after = step()  # the next step completes the audit and turns recording off
    assert view.audits_completed == 1 and view.last_audit_rows.tolist() == audited.tolist()
    assert not view.audit_step and flag_writes == [1, 0]
    assert np.array_equal(after, got, equal_nan=True), "a launch with the flag off changed the planes"
    step()  # still off: no flag write
    assert flag_writes == [1, 0]
    assert view.row_audited.tolist() == audited.tolist()
    assert view.audited_blocks[audited].tolist() == batch.blocks[audited].tolist()
