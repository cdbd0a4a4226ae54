"""CPU restatement of the audit statistic, tile_lse_kernel (runtime/audit_kernel.py:34-109).

For each selected row (``select[r] != 0``) while the flag is set (``:64-65``), each tile of
``tile_blocks`` blocks that starts before the row's length (``:67-69``) and each query row of the
audited KV head, the tile max ``m`` and ``l = sum exp(s - m)`` of ``s = scale * <q, k>`` over the
tile's keys at positions < length (``:70-96``) are stored into every block of the tile that the
row reaches (``:97-109``): plane 0 = m, plane 1 = l, at ``[layer][row][block][cell]``.

This restatement gathers each row's keys position by position through its block table and
computes in float64; cells it does not write keep their value (NaN in a fresh plane).
"""

from __future__ import annotations

import numpy as np


def new_planes(layers: int, rows: int, width: int, cells: int) -> np.ndarray:
    """A fresh statistic block: ``float32[2, layers, rows, width, cells]``, every cell NaN
    (the 0xFF fill, runtime/audit_kernel.py:137)."""
    return np.full((2, layers, rows, width, cells), np.nan, dtype=np.float32)


def tile_lse(
    planes: np.ndarray,
    q: np.ndarray,
    keys,
    table: np.ndarray,
    lens: np.ndarray,
    qrow: np.ndarray,
    select: np.ndarray,
    flag: int,
    layer: int,
    scale: float,
    block_size: int,
    group_rows: int,
    groups: list[int],
    tile_blocks: int = 2,
    k_scale: float = 1.0,
    key_heads: list[int] | None = None,
) -> None:
    """Record one layer into ``planes`` in place.

    ``q``: ``[tokens, q_heads, dim]``; ``keys``: indexable as ``keys[block, pos, head, :]``
    (``[blocks, block_size, kv_heads, dim]``).  ``groups`` lists the audited KV heads; head
    ``groups[h]`` writes cells ``h * group_rows .. + group_rows``.  ``k_scale`` dequantises keys;
    ``key_heads[h]`` is head ``groups[h]``'s index in ``keys`` when only some heads were copied.
    Lengths past ``width * block_size`` are clipped to it (the reference would read past the row)."""
    if flag == 0:
        return
    rows, width = planes.shape[2], planes.shape[3]
    tile_tokens = tile_blocks * block_size
    for r in range(rows):
        if select[r] == 0:
            continue
        length = int(min(max(int(lens[r]), 0), width * block_size))
        if length == 0:
            continue
        n_blocks = -(-length // block_size)
        positions = np.arange(length)
        block_ids = table[r, positions // block_size]
        for h, g in enumerate(groups):
            kh = g if key_heads is None else key_heads[h]
            k = np.asarray(keys[block_ids, positions % block_size, kh, :], dtype=np.float64) * k_scale
            qg = np.asarray(q[int(qrow[r]), g * group_rows : (g + 1) * group_rows, :], dtype=np.float64)
            scores = (qg @ k.T) * scale  # [group_rows, length]
            n_tiles = -(-length // tile_tokens)
            padded = np.full((group_rows, n_tiles * tile_tokens), -np.inf)
            padded[:, :length] = scores
            tiles = padded.reshape(group_rows, n_tiles, tile_tokens)
            m = tiles.max(axis=2)  # [group_rows, n_tiles]
            total = np.exp(tiles - m[:, :, None]).sum(axis=2)
            tile_of_block = np.arange(n_blocks) // tile_blocks
            cells = slice(h * group_rows, (h + 1) * group_rows)
            planes[0, layer, r, :n_blocks, cells] = m[:, tile_of_block].T
            planes[1, layer, r, :n_blocks, cells] = total[:, tile_of_block].T


def true_block_shares(q: np.ndarray, k: np.ndarray, scale: float, block_size: int) -> np.ndarray:
    """The float64 attention share of each block for one sequence and one KV group: the mean over the
    group's query rows of the softmax weight summed per block (tests/_attn_share_live_check.py:175-184).

    ``q``: ``[group_rows, dim]``; ``k``: ``[length, dim]``."""
    s = (np.asarray(q, np.float64) @ np.asarray(k, np.float64).T) * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    p = p.mean(axis=0)
    n_blocks = -(-len(p) // block_size)
    return np.pad(p, (0, n_blocks * block_size - len(p))).reshape(n_blocks, block_size).sum(axis=1)


def tile_lse_torch(planes, q, keys, table, lens, qrow, select, layer, scale, block_size, group_rows, group,
                   key_head=None, tile_blocks=2):
    """The same statistic with PyTorch on the host CPU, float32 as the reference's kernel accumulates,
    for the CPU baseline: ``keys`` a CPU tensor ``[blocks, block_size, heads, dim]`` (any float dtype),
    ``q`` a CPU tensor ``[tokens, q_heads, dim]``; one KV group; ``planes`` a NumPy block as above."""
    import torch

    kh = group if key_head is None else key_head
    width = planes.shape[3]
    tile_tokens = tile_blocks * block_size
    flat = keys[:, :, kh, :].reshape(-1, keys.shape[-1])  # [blocks * block_size, dim]
    for r in range(planes.shape[2]):
        if select[r] == 0:
            continue
        length = int(min(max(int(lens[r]), 0), width * block_size))
        if length == 0:
            continue
        n_blocks = -(-length // block_size)
        pos = torch.arange(length)
        rows_of = torch.from_numpy(table[r, :n_blocks].astype("int64"))[pos // block_size] * block_size + pos % block_size
        k = flat.index_select(0, rows_of).float()
        qg = q[int(qrow[r]), group * group_rows : (group + 1) * group_rows].float()
        s = (qg @ k.T) * scale
        n_tiles = -(-length // tile_tokens)
        padded = torch.full((group_rows, n_tiles * tile_tokens), float("-inf"))
        padded[:, :length] = s
        t = padded.view(group_rows, n_tiles, tile_tokens)
        m = t.amax(dim=2)
        total = torch.exp(t - m[:, :, None]).sum(dim=2)
        tile_of_block = torch.arange(n_blocks) // tile_blocks
        planes[0, layer, r, :n_blocks, :group_rows] = m[:, tile_of_block].T.numpy()
        planes[1, layer, r, :n_blocks, :group_rows] = total[:, tile_of_block].T.numpy()
