"""The seeded workload generators: shapes, determinism, non-overlapping tables."""

import numpy as np

import workloads


def test_config1_shapes():
    batch, kv, q = workloads.config1()
    assert batch.lens.tolist() == [17, 64, 200, 512]
    assert kv.shape == (256, 2, 16, 2, 64) and q.shape == (4, 8, 64)
    assert batch.blocks.tolist() == [2, 4, 13, 32]
    used = np.concatenate([batch.table[r, :n] for r, n in enumerate(batch.blocks)])
    assert len(set(used.tolist())) == len(used) and 0 not in used


def test_config2_is_deterministic_and_non_overlapping():
    a, b = workloads.config2_batch(), workloads.config2_batch()
    assert np.array_equal(a.lens, b.lens) and np.array_equal(a.table, b.table)
    assert a.rows == 128 and a.width == 512 and a.lens.min() >= 512 and a.lens.max() <= 8192
    used = np.concatenate([a.table[r, :n] for r, n in enumerate(a.blocks)])
    assert len(np.unique(used)) == len(used) and used.min() >= 1 and used.max() < 100_000


def test_config3_mix():
    batch = workloads.config3_batch()
    assert (batch.lens == 131072).sum() == 8 and batch.rows == 128
    short = batch.lens[batch.lens != 131072]
    assert short.min() >= 1024 and short.max() <= 4096
    rate = sum(len(h) for h in batch.extra["heavy"]) / batch.lens.sum()
    assert 0.004 < rate < 0.006


def test_config4_inputs():
    c = workloads.config4()
    blocks, shares = c["blocks"], c["shares"]
    assert shares.shape == (1024, 8192) and shares.dtype == np.float32
    assert ((c["seq_lens"] + 15) // 16 == blocks).all()
    sums = shares.sum(axis=1, dtype=np.float64)
    assert np.abs(sums - 1).max() < 1e-4
    assert all((shares[r, n:] == 0).all() for r, n in enumerate(blocks[:50]))
    assert (shares == 0).sum() > blocks.size  # exact zeros beyond the rows, and ties inside them


def test_config5_structure():
    batch = workloads.config5_batch()
    assert batch.rows == 256 and batch.block_size == 32 and batch.width == 1024
    assert batch.pool_blocks == int(batch.blocks.sum()) + 1
