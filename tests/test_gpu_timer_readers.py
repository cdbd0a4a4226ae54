"""The per-row timer read the way the reference's consumers read it: the descriptor line found by pid,
``timer_bytes`` bytes read in the serving process (``read_pass_cycles``) and, from another process,
through ``timer_ipc`` with per-step deltas (``Capture.cycle_deltas``); observe/zero_touch.py:66-93,
:190-225 and observe/capture.py:77-99 of the reference, with the pass's keys
(mlir_pass/lib/eKVTimer.cpp:588-590).  The deltas equal the differences of the plane's own reads and
satisfy the reader contract (oracle.cycles: no negative delta, shares partition unity)."""

import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from cases import audit_on
from oracle import cycles as oc
from observe.zero_touch import find_published, read_pass_cycles
from runtime.audit_kernel import RecordingPlane

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_cycles_through_the_descriptor_in_process_and_across_processes(tmp_path, monkeypatch):
    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))
    rng = np.random.default_rng(17)
    rows, width, bs, kvh, g, dim, layers = 24, 16, 16, 2, 4, 128, 4
    lens = torch.from_numpy(rng.integers(1, width * bs + 1, size=rows).astype(np.int32)).cuda()
    pool = 2 * rows * width + 1
    table = torch.from_numpy((1 + rng.permutation(pool - 1)[: rows * width]).reshape(rows, width).astype(np.int32)).cuda()
    kv = torch.randn(pool, 2, bs, kvh, dim, device="cuda", dtype=torch.bfloat16)
    q = torch.randn(rows, kvh * g, dim, device="cuda", dtype=torch.bfloat16)
    plane = RecordingPlane(layers, rows, width, g, bs, timer=True)
    audit_on(plane)

    def step(select):
        plane.select(select, np.arange(rows))
        for layer in range(layers):
            plane.record(f"layer.{layer}", table, lens, q, kv, dim ** -0.5)
        torch.cuda.synchronize()
        return plane.read_cycles().astype(np.int64)

    c0 = step(np.ones(rows, bool))
    published = find_published(os.getpid())
    assert len(published) == 1 and published[0].timer_bytes == rows * 8
    assert read_pass_cycles(os.getpid()) == {r: int(c0[r]) for r in range(rows) if c0[r] > 0}
    assert (c0 > 0).all()

    reader = subprocess.Popen([sys.executable, os.path.join(HERE, "timer_reader.py"), str(os.getpid())],
                              stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                              env=dict(os.environ))
    try:
        first = json.loads(reader.stdout.readline() or "null")
        assert first is not None, reader.stderr.read()[-2000:]
        assert first["baseline"] == {}
        assert {int(k): v for k, v in first["cycles"].items()} == {r: int(c0[r]) for r in range(rows)}
        chosen = rng.random(rows) < 0.5
        c1 = step(chosen)  # another step: only the chosen rows gain
        reader.stdin.write("\n")
        reader.stdin.flush()
        second = json.loads(reader.stdout.readline() or "null")
        assert second is not None, reader.stderr.read()[-2000:]
        assert reader.wait(timeout=60) == 0
    finally:
        if reader.poll() is None:
            reader.kill()
    deltas = {int(k): v for k, v in second["deltas"].items()}
    want = oc.delta(c0, c1)  # raises on a negative delta
    assert deltas == want
    assert set(deltas) == set(np.flatnonzero(chosen).tolist()), "a row that was not audited gained cycles"
    shares = oc.shares(deltas)
    assert abs(sum(shares.values()) - 1.0) < 1e-12
    assert {int(k): v for k, v in second["cycles"].items()} == {r: int(c1[r]) for r in range(rows)}
    print(f"{len(deltas)} rows' cycle deltas read across processes", flush=True)
