"""Seeded synthetic inputs of the five benchmark configurations of the audit / view hot path.

Structure (lengths, block tables, queries, shares) comes from ``numpy.random.default_rng(1000 + c)``
for configuration ``c``.  The paged KV pools of the large configurations are generated on the
device with a seeded ``torch.Generator`` (gigabytes of N(0, 1) would take minutes on the host);
tests copy back only the blocks they check.  Block 0 of every pool is unused and each request's
blocks come from a permutation of ``1 .. pool - 1``, as the reference's live checks lay out
their caches.

  1  4 rows, L = {17, 64, 200, 512}, bs 16, 8 query / 2 KV heads, d 64, fp32, pool 256
  2  Llama-3-8B decode: 128 rows, L ~ U[512, 8192], 32 / 8 heads, d 128, bf16, bs 16, pool 100k
  3  skewed: 8 rows of 131072 + 120 rows of truncated Zipf(1.2) on [1024, 4096], 0.5 % planted
     heavy-hitter keys (k <- 4 |k| qbar / |qbar|), Llama-3-8B heads, bf16, bs 16
  4  view build: 1024 rows of U[1, 8192] blocks, ids from a 2M pool, Dirichlet(0.1) float32 shares
  5  32-layer step: 256 rows, L ~ U[2048, 32768], 32 / 8 heads, d 128, bs 32, fp8 e4m3 keys
     with one per-tensor scale, bf16 queries
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def rng_for(config: int) -> np.random.Generator:
    return np.random.default_rng(1000 + config)


@dataclass
class Batch:
    """A paged decode batch: lengths, block tables and the pool they index."""

    lens: np.ndarray  # int32 [rows]
    table: np.ndarray  # int32 [rows, width]
    block_size: int
    pool_blocks: int
    q_heads: int
    kv_heads: int
    head_dim: int
    seed: int
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return int(self.lens.shape[0])

    @property
    def width(self) -> int:
        return int(self.table.shape[1])

    @property
    def group_rows(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def blocks(self) -> np.ndarray:
        return (self.lens.astype(np.int64) + self.block_size - 1) // self.block_size

    def key_bytes(self, elem_bytes: int, audited_heads: int = 1) -> int:
        """Bytes of keys one audit launch reads."""
        return int(self.lens.astype(np.int64).sum()) * self.head_dim * elem_bytes * audited_heads


def _tables(rng: np.random.Generator, lens: np.ndarray, block_size: int, width: int, pool: int) -> np.ndarray:
    """Non-overlapping block tables: consecutive slices of a permutation of 1 .. pool - 1."""
    n = (lens.astype(np.int64) + block_size - 1) // block_size
    if int(n.sum()) > pool - 1:
        raise ValueError(f"{int(n.sum())} blocks do not fit a pool of {pool}")
    ids = rng.permutation(np.arange(1, pool, dtype=np.int32))
    table = np.zeros((len(lens), width), dtype=np.int32)
    cursor = 0
    for r, count in enumerate(n.tolist()):
        table[r, :count] = ids[cursor : cursor + count]
        cursor += count
    return table


def config1() -> tuple[Batch, np.ndarray, np.ndarray]:
    """The small CPU-runnable audit: (batch, kv_cache float32 [256, 2, 16, 2, 64], q float32 [4, 8, 64])."""
    rng = rng_for(1)
    lens = np.array([17, 64, 200, 512], dtype=np.int32)
    bs, hq, hkv, d, pool = 16, 8, 2, 64, 256
    kv = rng.standard_normal((pool, 2, bs, hkv, d), dtype=np.float32)
    q = rng.standard_normal((len(lens), hq, d), dtype=np.float32)
    table = _tables(rng, lens, bs, 32, pool)
    return Batch(lens, table, bs, pool, hq, hkv, d, seed=1001), kv, q


def config2_batch() -> Batch:
    """Llama-3-8B decode shape, one layer's structure."""
    rng = rng_for(2)
    lens = rng.integers(512, 8193, size=128).astype(np.int32)
    bs = 16
    return Batch(lens, _tables(rng, lens, bs, 8192 // bs, 100_000), bs, 100_000, 32, 8, 128, seed=1002)


def queries(batch: Batch, layers: int, seed_offset: int = 0) -> np.ndarray:
    """float32 N(0, 1) queries ``[layers, rows, q_heads, head_dim]`` (one decode token per row)."""
    rng = np.random.default_rng(batch.seed + 7919 * (seed_offset + 1))
    return rng.standard_normal((layers, batch.rows, batch.q_heads, batch.head_dim), dtype=np.float32)


def config3_batch() -> Batch:
    """8 rows of 131072 tokens and 120 rows of truncated Zipf(1.2) lengths on [1024, 4096], shuffled."""
    rng = rng_for(3)
    support = np.arange(1024, 4097)
    p = support.astype(np.float64) ** -1.2
    short = rng.choice(support, size=120, p=p / p.sum())
    lens = np.concatenate([np.full(8, 131072), short]).astype(np.int32)
    lens = lens[rng.permutation(len(lens))]
    bs = 16
    batch = Batch(lens, _tables(rng, lens, bs, 131072 // bs, 100_000), bs, 100_000, 32, 8, 128, seed=1003)
    # positions of planted heavy hitters: 0.5 % of every row's keys
    batch.extra["heavy"] = [np.flatnonzero(rng.random(int(n)) < 0.005).astype(np.int64) for n in lens]
    return batch


def config4() -> dict[str, np.ndarray | int]:
    """The view-build inputs: blocks per row, tables, lengths and float32 Dirichlet(0.1) shares."""
    rng = rng_for(4)
    rows, width, bs = 1024, 8192, 16
    blocks = rng.integers(1, width + 1, size=rows).astype(np.int32)
    table = rng.integers(1, 2_000_000, size=(rows, width), dtype=np.int32)
    seq_lens = ((blocks.astype(np.int64) - 1) * bs + rng.integers(1, bs + 1, size=rows)).astype(np.int32)
    shares = np.zeros((rows, width), dtype=np.float32)
    for r, n in enumerate(blocks.tolist()):
        g = rng.standard_gamma(0.1, size=n)  # Dirichlet(0.1 * 1_n) = normalised Gamma(0.1)
        shares[r, :n] = (g / g.sum()).astype(np.float32)
    return {"blocks": blocks, "table": table, "seq_lens": seq_lens, "shares": shares, "block_size": bs}


def config5_batch() -> Batch:
    """256 rows of U[2048, 32768] tokens, block size 32, fp8 keys (structure only)."""
    rng = rng_for(5)
    lens = rng.integers(2048, 32769, size=256).astype(np.int32)
    bs = 32
    n = int(((lens.astype(np.int64) + bs - 1) // bs).sum())
    batch = Batch(lens, _tables(rng, lens, bs, 32768 // bs, n + 1), bs, n + 1, 32, 8, 128, seed=1005)
    batch.extra["k_scale"] = 6.0 / 448.0  # N(0, 1) / s fills the e4m3 range up to 6 sigma
    return batch


# -- device pools ------------------------------------------------------------------------------

def device_pool(batch: Batch, dtype, seed: int, device="cuda", chunk_blocks: int = 8192):
    """A paged KV cache ``[pool, 2, block, kv_heads, head_dim]`` of N(0, 1) on the device.

    fp8 pools hold ``N(0, 1) / k_scale`` rounded to e4m3 (saturated at +-448)."""
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (batch.pool_blocks, 2, batch.block_size, batch.kv_heads, batch.head_dim)
    fp8 = getattr(torch, "float8_e4m3fn", None)
    pool = torch.empty(shape, dtype=dtype, device=device)
    for start in range(0, batch.pool_blocks, chunk_blocks):
        stop = min(start + chunk_blocks, batch.pool_blocks)
        part = torch.randn((stop - start, *shape[1:]), generator=gen, dtype=torch.float32, device=device)
        if fp8 is not None and dtype == fp8:
            part = (part / batch.extra["k_scale"]).clamp_(-448.0, 448.0)
        pool[start:stop] = part.to(dtype)
    return pool


def plant_heavy_hitters(batch: Batch, pool, q) -> None:
    """Config 3's heavy hitters: each chosen key of every KV head h becomes ``4 |k| qbar_h / |qbar_h|``,
    ``qbar_h`` the mean of the row's query heads of group h (``q``: device ``[rows, q_heads, d]``)."""
    import torch

    g = batch.group_rows
    for r, positions in enumerate(batch.extra["heavy"]):
        if positions.size == 0:
            continue
        pos = torch.from_numpy(positions).to(pool.device)
        blocks = torch.from_numpy(batch.table[r]).to(pool.device).long()[pos // batch.block_size]
        offs = pos % batch.block_size
        qbar = q[r].float().reshape(batch.kv_heads, g, batch.head_dim).mean(dim=1)  # [kv_heads, d]
        direction = qbar / qbar.norm(dim=1, keepdim=True)
        k = pool[blocks, 0, offs].float()  # [count, kv_heads, d]
        norms = k.norm(dim=2, keepdim=True)
        pool[blocks, 0, offs] = (4.0 * norms * direction[None]).to(pool.dtype)


def host_keys(batch: Batch, pool, rows: list[int] | None = None, heads: list[int] | None = None):
    """The keys the given rows read, copied to the host as float32 with a compact table:
    (keys [used, block, kv_heads', d], table' [rows, width]) where table' indexes the compact pool."""
    import torch

    rows = list(range(batch.rows)) if rows is None else rows
    n = batch.blocks
    used = np.unique(np.concatenate([batch.table[r, : n[r]] for r in rows] + [np.zeros(1, np.int32)]))
    remap = np.zeros(int(batch.table.max()) + 1, dtype=np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    keys = pool[torch.from_numpy(used.astype(np.int64)).to(pool.device), 0]
    if heads is not None:
        keys = keys[:, :, heads]
    table = np.zeros_like(batch.table)
    for r in rows:
        table[r, : n[r]] = remap[batch.table[r, : n[r]]]
    return keys.float().cpu().numpy(), table
