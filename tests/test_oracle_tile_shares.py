"""The share-normalisation oracle against the reference's known answers and closed forms
(tests/test_tile_shares.py of the reference)."""

import numpy as np
import pytest

from cases import block_lse, lse_of, softmax_mass
from oracle import tile_shares as ots


def test_known_answers(known_answers):
    for case in known_answers["tile_shares"]:
        got = ots.normalize(lse_of(case), np.array(case["row_blocks"]), case["tile_blocks"], case["aggregate"])
        want = np.array(case["expected"], dtype=np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want)), case["name"]
        assert np.nanmax(np.abs(np.nan_to_num(got - want))) <= case["tol"], case["name"]


def test_shares_equal_the_softmax_mass_of_each_block():
    # closed form: normalised block log-sum-exps are the softmax mass of the blocks (test_tile_shares.py:33-45)
    rng = np.random.default_rng(0)
    layers, rows, qrows, sizes = 3, 2, 4, [16, 16, 16, 7]
    lse = np.zeros((layers, rows, len(sizes), qrows), dtype=np.float32)
    expected = np.zeros((rows, len(sizes)))
    for layer in range(layers):
        for row in range(rows):
            for q in range(qrows):
                scores = rng.normal(0, 3, sum(sizes))
                lse[layer, row, :, q] = block_lse(scores, sizes)
                expected[row] += softmax_mass(scores, sizes) / (layers * qrows)
    got = ots.normalize(lse, np.full(rows, len(sizes)), 1)
    assert np.abs(got - expected).max() < 1e-5


def test_rows_sum_to_one_and_offsets_cancel():
    rng = np.random.default_rng(1)
    lse = rng.normal(0, 4, (4, 3, 10, 2)).astype(np.float32)
    got = ots.normalize(lse, np.full(3, 10), 1)
    assert np.abs(got.sum(axis=1) - 1).max() < 1e-12
    shifted = lse.copy()
    shifted[1, 0, :, 1] += 40.0  # another running max leaves that record's shares unchanged
    assert np.abs(ots.normalize(shifted, np.full(3, 10), 1) - got).max() < 1e-6


def test_partial_tail_regain_equals_dropping_the_missing_block():
    # a row of 5 blocks in tiles of 2: the last tile's mass must land on block 4 alone, which is the same as
    # normalising per-tile masses directly -- an independent construction
    rng = np.random.default_rng(2)
    masses = rng.uniform(0.1, 5, size=3)
    lse = np.repeat(np.log(masses / 2), 2).astype(np.float32).reshape(1, 1, 6, 1)
    got = ots.normalize(lse, np.array([5]), 2)[0]
    want = np.array([masses[0] / 2, masses[0] / 2, masses[1] / 2, masses[1] / 2, masses[2], 0]) / masses.sum()
    assert np.abs(got - want).max() < 1e-6


def test_read_rows_layout_and_empty_tiles():
    # observe/tile_shares.py:129-173 read through d2h_many; the plane layout [2][layer][row][block][q]
    table_layers, layers, rows, width, group, tile_blocks = 4, 3, 5, 4, 2, 2
    cells = table_layers * rows * width * group
    rng = np.random.default_rng(3)
    m = rng.normal(0, 3, cells).astype(np.float32)
    total = rng.uniform(0.5, 9, cells).astype(np.float32)
    total[7] = 0.0  # a tile with no keys
    planes = np.concatenate([m, total]).reshape(2, table_layers, rows, width, group)
    got = ots.read_rows(planes, layers, np.arange(2), tile_blocks)
    assert got.shape == (layers, 2, width, group)
    assert got[0, 0, 3, 1] == -np.inf  # flat cell 7 is layer 0, row 0, block 3, query row 1
    assert np.isclose(got[2, 1, 0, 0], m[(2 * rows + 1) * width * group] + np.log(total[(2 * rows + 1) * width * group]) - np.log(2))
    with pytest.raises(ValueError):
        ots.read_rows(planes, layers, np.array([2, 1]), tile_blocks)


def test_errors():
    with pytest.raises(ValueError):
        ots.normalize(np.zeros((1, 1, 2, 1)), np.array([2]), 1, "median")
    with pytest.raises(ValueError):
        ots.normalize(np.zeros((2, 3, 4)), np.array([1, 1, 1]), 1)
    with pytest.raises(ValueError):
        ots.normalize(np.zeros((1, 3, 4, 1)), np.array([4, 4]), 1)
