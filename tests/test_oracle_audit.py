"""The audit oracle pinned by brute force on tiny inputs, by the closed form that its records
normalise to the true attention share, and by the flag / row-selection gates
(runtime/audit_kernel.py:62-109, tests/_audit_kernel_live_check.py:117-143 of the reference)."""

import math

import numpy as np

import workloads
from oracle import audit, tile_shares


def brute_force(q, kv, table, length, token, group, group_rows, scale, block_size):
    """m and l of every tile of one row, one key at a time in plain Python floats."""
    tile_tokens = 2 * block_size
    out = []
    for start in range(0, length, tile_tokens):
        per_q = []
        for g in range(group_rows):
            scores = []
            for pos in range(start, min(start + tile_tokens, length)):
                blk = int(table[pos // block_size])
                k = kv[blk, 0, pos % block_size, group]
                qq = q[token, group * group_rows + g]
                scores.append(scale * math.fsum(float(a) * float(b) for a, b in zip(qq, k)))
            m = max(scores)
            per_q.append((m, math.fsum(math.exp(s - m) for s in scores)))
        out.append(per_q)
    return out


def test_brute_force_on_config1_row0_and_row2():
    batch, kv, q = workloads.config1()
    planes = audit.new_planes(2, batch.rows, batch.width, batch.group_rows)
    scale = batch.head_dim ** -0.5
    for layer in (0, 1):
        audit.tile_lse(planes, q, kv[:, 0], batch.table, batch.lens, np.arange(batch.rows), np.ones(batch.rows),
                       1, layer, scale, batch.block_size, batch.group_rows, [layer % batch.kv_heads])
    for layer in (0, 1):
        for row in (0, 2):
            want = brute_force(q, kv, batch.table[row], int(batch.lens[row]), row, layer % batch.kv_heads,
                               batch.group_rows, scale, batch.block_size)
            n_blocks = -(-int(batch.lens[row]) // batch.block_size)
            for b in range(n_blocks):
                for g in range(batch.group_rows):
                    m, l = want[b // 2][g]
                    assert abs(planes[0, layer, row, b, g] - m) < 1e-5
                    assert abs(planes[1, layer, row, b, g] - l) < 1e-5 * max(1.0, l)
            assert np.isnan(planes[:, layer, row, n_blocks:]).all()  # cells past the row stay unwritten


def test_records_normalise_to_the_true_share():
    # u = m + log l is the log-sum-exp of each tile, so the normalised records are the exact share per tile
    batch, kv, q = workloads.config1()
    scale = batch.head_dim ** -0.5
    planes = audit.new_planes(1, batch.rows, batch.width, batch.group_rows)
    audit.tile_lse(planes, q, kv[:, 0], batch.table, batch.lens, np.arange(batch.rows), np.ones(batch.rows),
                   1, 0, scale, batch.block_size, batch.group_rows, [0])
    u = tile_shares.log_weights(planes[0], planes[1], 2)
    shares = tile_shares.normalize(u, batch.blocks, 2)
    for row in range(batch.rows):
        length = int(batch.lens[row])
        pos = np.arange(length)
        k = kv[batch.table[row, pos // batch.block_size], 0, pos % batch.block_size, 0]
        true = audit.true_block_shares(q[row, : batch.group_rows], k, scale, batch.block_size)
        n = len(true)
        tiles_true = np.add.reduceat(true, np.arange(0, n, 2))
        tiles_obs = np.add.reduceat(shares[row, :n], np.arange(0, n, 2))
        assert 0.5 * np.abs(tiles_true - tiles_obs).sum() < 1e-6  # far inside the 1e-3 TV gate


def test_flag_and_row_selection_gate_the_records():
    batch, kv, q = workloads.config1()
    scale = batch.head_dim ** -0.5
    off = audit.new_planes(1, batch.rows, batch.width, batch.group_rows)
    audit.tile_lse(off, q, kv[:, 0], batch.table, batch.lens, np.arange(4), np.ones(4), 0, 0, scale,
                   batch.block_size, batch.group_rows, [0])
    assert np.isnan(off).all()
    part = audit.new_planes(1, batch.rows, batch.width, batch.group_rows)
    audit.tile_lse(part, q, kv[:, 0], batch.table, batch.lens, np.arange(4), np.array([1, 0, 1, 1]), 1, 0, scale,
                   batch.block_size, batch.group_rows, [0])
    assert np.isnan(part[:, 0, 1]).all() and not np.isnan(part[:, 0, 0, 0]).all()


def test_all_heads_mode_stacks_the_groups():
    batch, kv, q = workloads.config1()
    scale = batch.head_dim ** -0.5
    one = [audit.new_planes(1, batch.rows, batch.width, batch.group_rows) for _ in range(batch.kv_heads)]
    for g in range(batch.kv_heads):
        audit.tile_lse(one[g], q, kv[:, 0], batch.table, batch.lens, np.arange(4), np.ones(4), 1, 0, scale,
                       batch.block_size, batch.group_rows, [g])
    every = audit.new_planes(1, batch.rows, batch.width, batch.group_rows * batch.kv_heads)
    audit.tile_lse(every, q, kv[:, 0], batch.table, batch.lens, np.arange(4), np.ones(4), 1, 0, scale,
                   batch.block_size, batch.group_rows, list(range(batch.kv_heads)))
    stacked = np.concatenate(one, axis=-1)
    assert np.array_equal(np.isnan(stacked), np.isnan(every))
    assert np.nanmax(np.abs(stacked - every)) == 0.0


def test_torch_cpu_form_matches_the_numpy_oracle():
    import torch

    batch, kv, q = workloads.config1()
    scale = batch.head_dim ** -0.5
    a = audit.new_planes(1, batch.rows, batch.width, batch.group_rows)
    b = audit.new_planes(1, batch.rows, batch.width, batch.group_rows)
    audit.tile_lse(a, q, kv[:, 0], batch.table, batch.lens, np.arange(4), np.ones(4), 1, 0, scale, batch.block_size,
                   batch.group_rows, [1])
    audit.tile_lse_torch(b, torch.from_numpy(q), torch.from_numpy(kv[:, 0].copy()), batch.table, batch.lens,
                         np.arange(4), np.ones(4), 0, scale, batch.block_size, batch.group_rows, 1)
    assert np.array_equal(np.isnan(a), np.isnan(b))
    live = ~np.isnan(a[0])
    assert np.abs(a[0][live] - b[0][live]).max() < 1e-4
    assert np.abs(np.log(a[1][live]) - np.log(b[1][live])).max() < 1e-4
