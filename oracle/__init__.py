"""Oracle: a CPU restatement of KVScope's audit / tile-share / ranking / view hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it, and only as the reference the results are compared with (or,
in ``bench.py``, as the timed CPU baseline) -- never as the thing measured or shipped.  The product path is the HIP library
(``sigmod-kvscope_amd/``) and fails loudly without it.

Modules, each citing the reference file:line it follows:
  audit        tile_lse_kernel's per-tile max / sum-exp   (runtime/audit_kernel.py:34-109)
  tile_shares  read_tile_rows + normalize_tile_lse         (observe/tile_shares.py:58-173)
  allocation   Request / allocate(..., "uniform")          (observe/allocation.py:39-91)
  controller   Controller._allocate's pins, cap, budget    (observe/controller.py:398-451)
  block_view   compact_block_table, DecodeView keep / count (runtime/block_view.py:36-56, 225-329)
  cycles       the per-row cycle-accumulator invariants     (observe/cycles.py:1-45, 116-239)

How each is pinned (known answers of the reference's tests, closed forms, brute force) is in
``tests/test_oracle_*.py``.  ``oracle/_ref`` does not exist: the reference's path is Python
(plus a Triton kernel), not C/C++ compiled from a few files.
"""
