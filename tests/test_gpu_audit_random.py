"""The audit kernel on seeded random batches against the float64 oracle (runtime/audit_kernel.py:34-109
of the reference). Every case draws the key type (f16 / bf16 / fp8 on the MFMA form, fp32 on the VALU
form), head dim, block size, query group, KV heads, rows and lengths (empty, partial and multi-tile rows),
the selected rows, a permuted query-token index per row, one KV group per layer or every KV head, and the
workgroup grid (the minimum of tiles per wave). The written cells must match the oracle's and the
records must agree within 1e-3."""

import numpy as np
import pytest
import torch

from oracle import audit as oa
from oracle import tile_shares as ots
from runtime.audit_kernel import RecordingPlane
from cases import audit_on

pytestmark = pytest.mark.gpu
FP8 = getattr(torch, "float8_e4m3fn", None)


def draw(seed):
    rng = np.random.default_rng(7000 + seed)
    kind = ["bf16", "f16", "fp8", "bf16", "f32"][seed % 5]
    dtype = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "fp8": FP8}[kind]
    d = int(rng.choice([64, 128] if kind == "f32" else [64, 128, 256]))
    bs = int(rng.choice([16, 32]))
    G = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 4]))
    rows = int(rng.integers(1, 121))
    max_blocks = int(rng.integers(1, 41))
    lens = rng.integers(0, max_blocks * bs + 1, size=rows).astype(np.int32)
    lens[rng.random(rows) < 0.1] = 0
    n = (lens + bs - 1) // bs
    width = max(int(n.max()), 1) + int(rng.integers(0, 3))
    pool = int(n.sum()) + 2
    ids = rng.permutation(np.arange(1, pool))
    table = np.zeros((rows, width), dtype=np.int32)
    cursor = 0
    for r in range(rows):
        table[r, : n[r]] = ids[cursor : cursor + n[r]]
        cursor += int(n[r])
    select = rng.random(rows) < 0.8
    tokens = rows + int(rng.integers(0, 8))
    qrow = rng.permutation(tokens)[:rows].astype(np.int32)
    every_head = bool(rng.random() < 0.3)
    chunk = int(rng.choice([0, 1, 5, 60, 1000]))
    layer = int(rng.integers(0, 4))
    return dict(kind=kind, dtype=dtype, d=d, bs=bs, G=G, hkv=hkv, rows=rows, lens=lens, width=width, pool=pool,
                table=table, select=select, tokens=tokens, qrow=qrow, every_head=every_head, chunk=chunk,
                layer=layer, rng=rng)


@pytest.mark.parametrize("seed", range(20))
def test_random_batch_against_the_oracle(seed):
    c = draw(seed)
    if c["dtype"] is None:
        pytest.skip("this torch has no float8_e4m3fn")
    rng, d, bs, G, hkv, rows = c["rng"], c["d"], c["bs"], c["G"], c["hkv"], c["rows"]
    print(f"seed {seed}: {c['kind']} d {d} block {bs} G {G} kv heads {hkv} rows {rows} width {c['width']} "
          f"every head {c['every_head']} chunk {c['chunk']}", flush=True)
    kv = torch.from_numpy(rng.standard_normal((c["pool"], 2, bs, hkv, d), dtype=np.float32))
    k_scale = 1.0
    if c["kind"] == "fp8":
        k_scale = 4.0 / 448.0
        kv = (kv / k_scale).clamp(-448, 448).to(FP8)
    else:
        kv = kv.to(c["dtype"])
    qdtype = torch.bfloat16 if c["kind"] == "fp8" else c["dtype"]
    q = torch.from_numpy(rng.standard_normal((c["tokens"], hkv * G, d), dtype=np.float32)).to(qdtype)
    layers = c["layer"] + 1
    plane = RecordingPlane(layers, rows, c["width"], G, bs, kv_heads=hkv if c["every_head"] else None)
    audit_on(plane)
    plane.select(c["select"], c["qrow"])
    scale = d ** -0.5
    plane.launch(c["layer"], torch.from_numpy(c["table"]).cuda(), torch.from_numpy(c["lens"]).cuda(), q.cuda(),
                 kv.cuda()[:, 0], scale, k_scale=k_scale, chunk_tiles=c["chunk"])
    torch.cuda.synchronize()
    got = plane.read_planes()
    heads = list(range(hkv)) if c["every_head"] else [c["layer"] % hkv]
    want = oa.new_planes(layers, rows, c["width"], G * len(heads))
    oa.tile_lse(want, q.float().numpy(), kv[:, 0].float().numpy(), c["table"], c["lens"], c["qrow"], c["select"], 1,
                c["layer"], scale, bs, G, heads, k_scale=k_scale)
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0])), "written cells differ"
    live = ~np.isnan(want[0])
    if not live.any():
        return
    dm = np.abs(got[0][live] - want[0][live]).max()
    du = np.abs(ots.log_weights(got[0], got[1], 1)[live].astype(np.float64)
                - ots.log_weights(want[0], want[1], 1)[live]).max()
    assert dm < 1e-3 and du < 1e-3, (dm, du)
