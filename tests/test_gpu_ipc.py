"""The controller path across processes: a serving process records the audit statistic and
publishes its descriptor; a controller process opens the planes by IPC handle and normalises the
live rows' shares on its own device (observe/controller.py:92-136, observe/tile_shares.py:26-52
and runtime/audit_kernel.py:160-180 of the reference).  Compared with the oracle within 1e-4."""

import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import workloads
from oracle import tile_shares as ots
from runtime.audit_kernel import TILE_BLOCKS, RecordingPlane

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_controller_reads_the_planes_of_another_process(tmp_path, monkeypatch):
    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))
    batch, kv, q = workloads.config1()
    plane = RecordingPlane(3, batch.rows, batch.width, batch.group_rows, batch.block_size)
    kv_t = torch.from_numpy(kv).cuda()
    # the engine's protocol: two of the three layers' caches attached (the controller counts the
    # filled entries as the layers that ran), the rows selected, the flag set
    plane.attach([kv_t.data_ptr(), kv_t.data_ptr() + 1])
    plane.select(np.ones(batch.rows, bool), np.arange(batch.rows))
    plane.set(True)
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    for layer in range(2):  # two of the three layers run
        plane.record(f"layer.{layer}", table, lens, torch.from_numpy(q).cuda(), kv_t, batch.head_dim ** -0.5)
    torch.cuda.synchronize()
    row_blocks = batch.blocks.copy()
    row_blocks[1] = 0  # a row without blocks is not read
    out = tmp_path / "shares.npy"
    done = subprocess.run(
        [sys.executable, os.path.join(HERE, "ipc_controller.py"), str(os.getpid()), str(out),
         ",".join(str(int(x)) for x in row_blocks)],
        env=dict(os.environ), capture_output=True, text=True, timeout=240,
    )
    assert done.returncode == 0, done.stdout[-2000:] + done.stderr[-2000:]
    got = np.load(out)
    planes = plane.read_planes()
    wanted = np.flatnonzero(row_blocks > 0)
    want = ots.normalize(ots.read_rows(planes, 2, wanted, TILE_BLOCKS), row_blocks[wanted], TILE_BLOCKS)
    assert np.isnan(got[1]).all()
    err = float(np.nanmax(np.abs(got[wanted] - want)))
    print(f"shares read across processes: max |d share| {err:.2e}", flush=True)
    assert np.array_equal(np.isnan(got[wanted]), np.isnan(want)) and err < 1e-4
