"""GPU SGLang index-list compaction (ekv_compact_slots through the drop-in SlotCompactor) bit-exact
against the oracle: the reference test's cases, int32 and int64 slots, padding and audited rows,
counters accumulated over calls, nothing written past the list, and a 256-row batch of up to 8192
tokens per row (runtime/sglang_compact.py and tests/test_sglang_view.py of the reference)."""

import numpy as np
import pytest
import torch

from oracle import sglang_compact as osc
from runtime.sglang_compact import SlotCompactor

pytestmark = pytest.mark.gpu
BLOCK = 16
WIDTH = 20


def run(compactor, lens, keep, padding=0, audited=None, active=True, seed=0, dtype=torch.int64):
    rng = np.random.default_rng(seed)
    full_lens = list(lens) + [1] * padding  # a CUDA graph fills the batch with one-token rows
    indptr = np.array([0, *np.cumsum(full_lens).tolist()], dtype=np.int32)
    slots = rng.permutation(max(10_000, int(indptr[-1])))[: indptr[-1]].astype(np.int64)
    want = osc.compact(indptr, slots, keep, audited, active, len(lens), len(full_lens), compactor.block_tokens)
    d_indptr = torch.from_numpy(indptr).cuda()
    d_slots = torch.from_numpy(np.concatenate([slots, np.full(7, -1)])).to(dtype).cuda()  # a longer buffer
    audit = None if audited is None else torch.from_numpy(audited.astype(np.uint8)).cuda()
    before = compactor.counts.cpu().numpy().copy()
    lens_out = compactor.compact(d_indptr, d_slots, torch.from_numpy(keep).cuda(), audit, active, len(lens),
                                 len(full_lens), int(indptr[-1]))
    torch.cuda.synchronize()
    new_indptr = d_indptr.cpu().numpy()
    got_slots = d_slots.cpu().numpy()
    assert new_indptr.tolist() == want["new_indptr"]
    assert lens_out.cpu().numpy().tolist() == want["lens"]
    total = want["new_indptr"][-1]
    assert np.array_equal(got_slots[:total], want["out"].astype(got_slots.dtype))
    assert got_slots[total : indptr[-1]].tolist() == slots[total:].astype(got_slots.dtype).tolist()  # old values
    assert got_slots[indptr[-1] :].tolist() == [-1] * 7  # nothing after the list is written
    table = compactor.table.cpu().numpy()
    for row, chosen in enumerate(want["table"]):
        assert table[row, : len(chosen)].tolist() == chosen, row
    assert (compactor.counts.cpu().numpy() - before).tolist() == want["counts"]
    return want["counts"]


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_reference_cases(dtype):
    c = SlotCompactor(WIDTH, BLOCK, torch.device("cuda"))
    lens = [5, 16, 17, 100, 33]
    blocks = sum(-(-n // BLOCK) for n in lens)
    assert run(c, lens, np.ones((len(lens), WIDTH), dtype=bool), dtype=dtype) == [blocks, blocks, 0, blocks, 0]
    lens = [200, 64, 150, 17, 1]
    counts = run(c, lens, (np.arange(WIDTH)[None, :] % 2 == 0).repeat(len(lens), axis=0), seed=1, dtype=dtype)
    assert counts[0] < counts[1]
    lens = [200, 150, 90]
    keep = np.zeros((len(lens), WIDTH), dtype=bool)
    assert run(c, lens, keep, audited=np.array([False, True, False]), seed=2, dtype=dtype)[2] == -(-150 // BLOCK)
    counts = run(c, lens, keep, active=False, seed=3, dtype=dtype)
    assert counts[0] == counts[1] == counts[4]
    run(c, [35], np.zeros((1, WIDTH), dtype=bool), dtype=dtype)
    rng = np.random.default_rng(7)
    for seed in range(20):
        rows = int(rng.integers(1, 9))
        keep = rng.random((rows, WIDTH)) < rng.random()
        audited = rng.random(rows) < 0.3 if seed % 2 else None
        run(c, rng.integers(1, BLOCK * WIDTH, rows).tolist(), keep, int(rng.integers(0, 4)), audited, seed=seed,
            dtype=dtype)


def test_no_rows():
    c = SlotCompactor(WIDTH, BLOCK, torch.device("cuda"))
    indptr = torch.zeros(1, dtype=torch.int32, device="cuda")
    slots = torch.full((4,), -1, dtype=torch.int64, device="cuda")
    lens = c.compact(indptr, slots, torch.zeros(0, WIDTH, dtype=torch.bool, device="cuda"), None, True, 0, 0, 0)
    torch.cuda.synchronize()
    assert lens.numel() == 0 and indptr.tolist() == [0] and slots.tolist() == [-1] * 4


def test_large_batch():
    # 256 decode rows of up to 8192 tokens (width 512 blocks), a CUDA graph's 8 padding rows
    rng = np.random.default_rng(11)
    width = 512
    c = SlotCompactor(width, BLOCK, torch.device("cuda"))
    lens = rng.integers(1, width * BLOCK + 1, size=256).tolist()
    keep = rng.random((264, width)) < 0.5
    audited = rng.random(256) < 0.1
    counts = run(c, lens, keep, padding=8, audited=audited, seed=5)
    assert counts[0] < counts[1]


def test_rows_past_the_lds_offsets():
    # 8192 rows (more than the 6000 whose offsets the gather keeps in LDS): the offsets go through
    # memory; 16 padding rows and audited rows, int64 and int32 slots
    rng = np.random.default_rng(13)
    width = 24
    c = SlotCompactor(width, BLOCK, torch.device("cuda"))
    rows = 8192
    lens = rng.integers(1, width * BLOCK + 1, size=rows).tolist()
    lens[5] = BLOCK  # one block
    keep = rng.random((rows + 16, width)) < 0.4
    audited = rng.random(rows) < 0.05
    for dtype, seed in ((torch.int64, 21), (torch.int32, 22)):
        print(f"{rows} rows, {dtype}", flush=True)
        counts = run(c, lens, keep, padding=16, audited=audited, seed=seed, dtype=dtype)
        assert counts[0] < counts[1]
