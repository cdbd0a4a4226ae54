"""The oracle of the SGLang index-list compaction against the reads each request makes (its kept
blocks in order, the first and last always kept) and the read counters' known answers
(tests/test_sglang_view.py:18-115 of the reference)."""

import numpy as np

from oracle import sglang_compact as osc

BLOCK = 16
WIDTH = 20


def reads(indptr, slots, keep, lens, whole):
    """The slots each request reads: its kept blocks in order, the first and last block always kept."""
    out = []
    for row, length in enumerate(lens):
        blocks = -(-length // BLOCK)
        kept = [b for b in range(blocks) if keep[row, b] or whole[row] or b in (0, blocks - 1)]
        out.append([slots[indptr[row] + p] for b in kept for p in range(b * BLOCK, (b + 1) * BLOCK) if p < length])
    return out


def run(lens, keep, padding=0, audited=None, active=True, seed=0):
    rng = np.random.default_rng(seed)
    full_lens = list(lens) + [1] * padding
    indptr = [0, *np.cumsum(full_lens).tolist()]
    slots = rng.permutation(10_000)[: indptr[-1]]
    whole = np.zeros(len(lens), dtype=bool) if audited is None else audited[: len(lens)].copy()
    whole |= not active
    got = osc.compact(indptr, slots, keep, audited, active, len(lens), len(full_lens), BLOCK)
    expected = reads(indptr, slots, keep, lens, whole) + [[slots[indptr[len(lens) + i]]] for i in range(padding)]
    assert got["new_indptr"] == [0, *np.cumsum([len(r) for r in expected]).tolist()]
    assert got["lens"] == [len(r) for r in expected]
    for row, want in enumerate(expected):
        assert got["out"][got["new_indptr"][row] : got["new_indptr"][row + 1]].tolist() == want, row
    return got["counts"]


def test_keep_all_is_the_identity():
    lens = [5, 16, 17, 100, 33]
    blocks = sum(-(-n // BLOCK) for n in lens)
    assert run(lens, np.ones((len(lens), WIDTH), dtype=bool)) == [blocks, blocks, 0, blocks, 0]


def test_half_reads_less_than_full():
    lens = [200, 64, 150, 17, 1]
    keep = (np.arange(WIDTH)[None, :] % 2 == 0).repeat(len(lens), axis=0)
    counts = run(lens, keep, seed=1)
    assert counts[0] < counts[1]


def test_audited_and_inactive_rows_read_everything():
    lens = [200, 150, 90]
    keep = np.zeros((len(lens), WIDTH), dtype=bool)
    counts = run(lens, keep, audited=np.array([False, True, False]), seed=2)
    assert counts[2] == -(-150 // BLOCK)
    counts = run(lens, keep, active=False, seed=3)
    assert counts[0] == counts[1] == counts[4]


def test_partial_last_block_is_kept():
    run([35], np.zeros((1, WIDTH), dtype=bool))


def test_random_batches_with_padding_rows():
    rng = np.random.default_rng(7)
    for seed in range(40):
        rows = int(rng.integers(1, 9))
        keep = rng.random((rows, WIDTH)) < rng.random()
        audited = rng.random(rows) < 0.3 if seed % 2 else None
        run(rng.integers(1, BLOCK * WIDTH, rows).tolist(), keep, int(rng.integers(0, 4)), audited, seed=seed)
