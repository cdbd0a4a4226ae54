"""GPU `sum` split (ekv_rank_sum through allocate and sum_keep) bit-exact against the oracle:
the reference test's tied integer scores with weights, explicit pins, float64 scores, rows past
NumPy's 8192-value reduction run, and the view-build configuration at full size
(observe/allocation.py:55-123 and tests/test_allocation.py:170-250 of the reference)."""

import numpy as np
import pytest
import torch

import workloads
from cases import random_requests
from observe import allocation
from oracle import allocation as oa

pytestmark = pytest.mark.gpu


def same(got, want):
    return len(got) == len(want) and all(np.array_equal(a, b) for a, b in zip(got, want))


@pytest.mark.parametrize("seed", range(40))
def test_sum_with_ties_and_weights(seed):
    rng = np.random.default_rng(seed)
    reqs = []
    for _ in range(int(rng.integers(1, 9))):
        n = int(rng.integers(3, 40))
        scores = rng.integers(0, 4, size=n).astype(float)  # many equal scores, so many ties
        reqs.append(allocation.Request(scores=scores, weight=float(rng.choice([1.0, 2.0, 0.5]))))
    total = sum(len(r.scores) for r in reqs)
    must = sum(int(r.pinned_mask().sum()) for r in reqs)
    budget = int(rng.integers(must, max(total, must + 1)))
    got = allocation.allocate(reqs, budget, "sum")
    want = oa.allocate_sum([r.scores for r in reqs], [r.pinned_mask() for r in reqs], [r.weight for r in reqs], budget)
    assert same(got, want)


def test_sum_float64_scores_and_explicit_pins():
    rng = np.random.default_rng(3)
    for trial in range(60):
        scores, pinned = random_requests(rng, int(rng.integers(1, 7)), 50, ties=trial % 2 == 0)
        scores = [s.astype(np.float64) * (1 + 1e-9 * rng.random(len(s))) for s in scores]  # not float32 values
        weights = [float(rng.choice([1.0, 3.0, 0.25])) for _ in scores]
        total = sum(len(s) for s in scores)
        must = sum(int(p.sum()) for p in pinned)
        budget = int(rng.integers(must, max(total, must + 1)))
        reqs = [allocation.Request(scores=s, weight=w, pinned=p) for s, w, p in zip(scores, weights, pinned)]
        assert same(allocation.allocate(reqs, budget, "sum"), oa.allocate_sum(scores, pinned, weights, budget)), trial


def test_sum_row_totals_are_numpy_sums_bit_for_bit():
    # every ranking divides by NumPy's float64 sum of the clamped scores; a total one ulp off would
    # shift each share by about an ulp, which the keep masks rarely show, so the totals are read back
    # from the workspace (its state block, then one 24-byte statistic per row: the total first) and
    # compared bit for bit: lengths across the leaf sizes (1..128), the pairwise splits and several
    # 8192-value runs, with values over many binades so that the order of the additions shows
    rng = np.random.default_rng(21)
    lengths = [1, 2, 7, 8, 9, 15, 16, 17, 127, 128, 129, 136, 255, 256, 257, 1000, 1024, 4095, 4096,
               4097, 8191, 8192, 8193, 12288, 16385, 20000]
    width = max(lengths)
    rows = len(lengths)
    scores = np.zeros((rows, width))
    for r, n in enumerate(lengths):
        scores[r, :n] = rng.random(n) * 10.0 ** rng.integers(-12, 4, size=n)
        scores[r, : n : 5] *= -1.0  # clamped to 0
    state = allocation.sum_workspace_bytes(0) - 256
    stat = 24
    workspace = torch.zeros(allocation.sum_workspace_bytes(rows), dtype=torch.uint8, device="cuda")
    s_dev = torch.from_numpy(scores).cuda()
    b_dev = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    allocation.sum_keep(s_dev, b_dev, budget=sum(lengths) // 2, workspace=workspace)
    torch.cuda.synchronize()
    raw = workspace.cpu().numpy()
    base = (-workspace.data_ptr()) % 256 + state
    for r, n in enumerate(lengths):
        got = raw[base + r * stat: base + r * stat + 8].view(np.float64)[0]
        want = np.maximum(scores[r, :n], 0.0).sum()
        assert got.tobytes() == np.float64(want).tobytes(), (n, got, want)


def test_sum_rows_past_one_reduction_run():
    # rows of more than 8192 blocks: NumPy's total adds two runs' pairwise sums
    rng = np.random.default_rng(8)
    scores = [rng.random(n) * rng.choice([1e-3, 1.0, 7.0]) for n in (8191, 8192, 8193, 12288, 9000)]
    pinned = [oa.default_pins(len(s)) for s in scores]
    weights = [1.0, 2.0, 0.5, 1.0, 1.5]
    total = sum(len(s) for s in scores)
    for frac in (0.1, 0.5, 0.9):
        budget = int(frac * total)
        reqs = [allocation.Request(scores=s, weight=w) for s, w in zip(scores, weights)]
        assert same(allocation.allocate(reqs, budget, "sum"), oa.allocate_sum(scores, pinned, weights, budget)), frac


def test_sum_rows_wider_than_a_register_row():
    # rows past 12288 blocks and past the 14-bit block field of the narrower tie key (16384): the tie
    # passes cover 18 bits of block; integer scores force ties at the threshold across requests, and
    # NumPy's totals add several 8192-value runs
    rng = np.random.default_rng(16)
    for sizes in ((16384, 12289, 300), (16385, 32768, 5000), (40000, 17, 20000)):
        scores = [rng.integers(0, 5, size=n).astype(float) * rng.choice([1e-3, 1.0]) for n in sizes]
        scores[0][::7] = 2.0  # many equal gains
        pinned = [oa.default_pins(len(x)) for x in scores]
        weights = [1.0, 2.0, 1.0][: len(sizes)]
        total = sum(sizes)
        for frac in (0.2, 0.5):
            budget = int(frac * total)
            reqs = [allocation.Request(scores=x, weight=w) for x, w in zip(scores, weights)]
            print(f"sizes {sizes} budget {budget}", flush=True)
            assert same(allocation.allocate(reqs, budget, "sum"), oa.allocate_sum(scores, pinned, weights, budget))


def test_sum_view_build_configuration():
    # 1024 rows of U[1, 8192] blocks with Dirichlet(0.1) float32 shares: budgets 0.2 / 0.5 / 0.8
    c = workloads.config4()
    shares, blocks = c["shares"], c["blocks"]
    sizes = blocks.tolist()
    total = int(blocks.sum())
    scores = [shares[r, : sizes[r]] for r in range(len(sizes))]
    pinned = [oa.default_pins(n) for n in sizes]
    s_dev, b_dev = torch.from_numpy(shares).cuda(), torch.from_numpy(blocks).cuda()
    for frac in (0.2, 0.5, 0.8):
        budget = int(np.ceil(frac * total))
        keep, summary = allocation.sum_keep(s_dev, b_dev, budget=budget)
        got = keep.cpu().numpy()
        want = oa.allocate_sum(scores, pinned, [1.0] * len(sizes), budget)
        bad = sum(int((got[r, : sizes[r]].astype(bool) != want[r]).sum()) for r in range(len(sizes)))
        print(f"sum at {frac}: budget {budget}, kept {sum(int(w.sum()) for w in want)}, mismatched {bad}", flush=True)
        assert bad == 0 and int(summary[0]) == budget and int(summary[3]) == 0
        assert all(got[r, sizes[r]:].all() for r in range(len(sizes))), "a position past a row is kept"


def test_sum_select_ending_at_the_first_digit():
    # the free blocks are exactly the open blocks of the top bucket of the first digit (shares near 1/k
    # against shares 1e-10 times smaller, 33 binades apart): the select ends at the first pass, so the
    # keep kernel writes every block itself; a budget one block larger ends it in a later pass
    rng = np.random.default_rng(5)
    scores, pinned = [], []
    for n in (40, 300, 3000, 9000):
        big = int(rng.integers(5, n - 5))
        x = np.concatenate([1.0 + rng.random(big), 1e-10 * (1.0 + rng.random(n - big))])
        scores.append(rng.permutation(x))
        pinned.append(oa.default_pins(n))
    must = sum(int(p.sum()) for p in pinned)
    top = sum(int(((x >= 1.0) & ~p).sum()) for x, p in zip(scores, pinned))
    for budget in (must + top, must + top + 1, must + top - 1):
        reqs = [allocation.Request(scores=x) for x in scores]
        assert same(allocation.allocate(reqs, budget, "sum"), oa.allocate_sum(scores, pinned, [1.0] * 4, budget)), budget


def test_sum_more_than_65536_requests():
    # 70000 requests: the tie key's request field takes 17 bits; integer scores tie across requests
    rng = np.random.default_rng(31)
    rows, width = 70000, 6
    scores = rng.integers(0, 3, size=(rows, width)).astype(np.float64)
    sizes = rng.integers(1, width + 1, size=rows)
    pinned = [oa.default_pins(int(n)) for n in sizes]
    total = int(sizes.sum())
    s_dev = torch.from_numpy(scores).cuda()
    b_dev = torch.from_numpy(sizes.astype(np.int32)).cuda()
    must = sum(int(p.sum()) for p in pinned)
    for frac in (0.3, 0.6):
        budget = must + int(frac * (total - must))
        keep, summary = allocation.sum_keep(s_dev, b_dev, budget=budget)
        got = keep.cpu().numpy()
        want = oa.allocate_sum([scores[r, : sizes[r]] for r in range(rows)], pinned, [1.0] * rows, budget)
        bad = sum(int((got[r, : sizes[r]].astype(bool) != want[r]).sum()) for r in range(rows))
        print(f"sum over {rows} requests at {frac}: mismatched {bad}", flush=True)
        assert bad == 0 and int(summary[4]) == rows


def test_maxmin_more_than_65536_requests():
    # 70000 requests: the bisection's state in memory, its summed count and active requests packed
    rng = np.random.default_rng(32)
    rows, width = 70000, 6
    scores = rng.random((rows, width)) * rng.choice([1e-3, 1.0], size=(rows, 1))
    sizes = rng.integers(1, width + 1, size=rows)
    pinned = [oa.default_pins(int(n)) for n in sizes]
    total = int(sizes.sum())
    s_dev = torch.from_numpy(scores).cuda()
    b_dev = torch.from_numpy(sizes.astype(np.int32)).cuda()
    must = sum(int(p.sum()) for p in pinned)
    budget = must + int(0.5 * (total - must))
    keep, summary = allocation.maxmin_keep(s_dev, b_dev, budget=budget)
    got = keep.cpu().numpy()
    want = oa.allocate_maxmin([scores[r, : sizes[r]] for r in range(rows)], pinned, budget)
    bad = sum(int((got[r, : sizes[r]].astype(bool) != want[r]).sum()) for r in range(rows))
    print(f"maxmin over {rows} requests: mismatched {bad}", flush=True)
    assert bad == 0 and int(summary[4]) == rows


def test_sum_summary_flags_a_budget_below_the_pins():
    scores = torch.ones(2, 5, dtype=torch.float64, device="cuda")
    blocks = torch.tensor([5, 5], dtype=torch.int32, device="cuda")
    keep, summary = allocation.sum_keep(scores, blocks, budget=3)  # 4 pinned blocks
    assert int(summary[3]) == 1 and int(summary[2]) == 4
    with pytest.raises(ValueError):
        allocation.allocate([allocation.Request(scores=np.ones(5))] * 2, 3, "sum")


# ---- maxmin ----------------------------------------------------------------------------------

def test_maxmin_running_totals_are_numpy_cumsums_bit_for_bit():
    # the running totals of each request's open shares sorted by share (np.cumsum) are read back from
    # the workspace (the last rows x width float64 array before its 256-byte tail) and compared bit for
    # bit: shares with full mantissas, whose sums round to ties about half the time while a share is
    # within a binade of the total; coarse integer scores (many equal shares); exact binary fractions;
    # shares across 300 decades; zero plateaus; lengths on both sides of the 1024-value chunks; a NaN
    # score (every share NaN) and a +inf score (zero shares, then one NaN, which sorts last)
    rng = np.random.default_rng(33)
    lengths = [1, 2, 3, 17, 1023, 1024, 1025, 1026, 2047, 2049, 3000, 4096, 5000, 8191, 8192, 8192,
               6000, 7000, 8000, 300, 9000, 12288, 2500, 3100]
    width = max(lengths)
    rows = len(lengths)
    scores = np.zeros((rows, width))
    for r, n in enumerate(lengths):
        kind = r % 6
        if kind == 0:
            x = rng.dirichlet(np.full(n, 0.1))
        elif kind == 1:
            x = rng.integers(1, 9, size=n).astype(np.float64)
        elif kind == 2:
            x = np.full(n, 0.25)
        elif kind == 3:
            x = rng.random(n) * 10.0 ** rng.uniform(-300, 0, size=n)
        elif kind == 4:
            x = rng.random(n)
            x[rng.random(n) < 0.7] = 0.0
        else:
            x = rng.dirichlet(np.full(n, 10.0))
        if r == len(lengths) - 2:
            x = rng.random(n)
            x[n // 3] = np.nan
        elif r == len(lengths) - 1:
            x = rng.random(n)
            x[n // 2] = np.inf
        scores[r, :n] = x
    need = allocation.maxmin_workspace_bytes(rows, width)
    workspace = torch.zeros(need, dtype=torch.uint8, device="cuda")
    s_dev = torch.from_numpy(scores).cuda()
    b_dev = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    total = sum(lengths)
    must = sum(min(n, 2) for n in lengths)
    allocation.maxmin_keep(s_dev, b_dev, budget=must + (total - must) // 2, workspace=workspace)
    torch.cuda.synchronize()
    raw = workspace.cpu().numpy()
    cells = rows * width * 8
    prefix = (-workspace.data_ptr()) % 256 + need - 256 - (cells + 255) // 256 * 256
    for r, n in enumerate(lengths):
        with np.errstate(invalid="ignore"):
            sh = oa.shares(scores[r, :n])  # inf / inf is NaN
        open_sh = sh[~oa.default_pins(n)]
        nan = np.isnan(open_sh)
        want = np.cumsum(np.concatenate([np.sort(open_sh[~nan])[::-1], open_sh[nan]]))
        got = raw[prefix + r * width * 8: prefix + (r * width + len(want)) * 8].view(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want)), (n, r)
        fin = ~np.isnan(want)
        assert got[fin].tobytes() == want[fin].tobytes(), (n, r % 6, int(np.argmax(got != want)))


@pytest.mark.parametrize("seed", range(40))
def test_maxmin_random_requests(seed):
    rng = np.random.default_rng(seed)
    scores, pinned = random_requests(rng, int(rng.integers(1, 9)), 40)
    total = sum(len(s) for s in scores)
    must = sum(int(p.sum()) for p in pinned)
    budget = int(rng.integers(must, max(total, must + 1)))
    reqs = [allocation.Request(scores=s, pinned=p) for s, p in zip(scores, pinned)]
    assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget))


def test_maxmin_identical_requests_and_edges():
    # identical requests reach the level together: the leftover goes one block each by index
    rng = np.random.default_rng(4)
    s = rng.dirichlet(np.full(30, 0.3))
    scores = [s.copy() for _ in range(12)]
    pinned = [oa.default_pins(30) for _ in scores]
    must = sum(int(p.sum()) for p in pinned)
    for budget in (must, must + 1, must + 7, must + 100, 360 - 1, 360):
        reqs = [allocation.Request(scores=x) for x in scores]
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), budget
    with pytest.raises(ValueError):
        allocation.allocate([allocation.Request(scores=np.ones(5))] * 2, 3, "maxmin")


@pytest.mark.parametrize("rows", [12, 1500, 3000])
def test_maxmin_leftover_over_plateaus_and_ties(rows):
    # a large leftover: requests whose remaining shares are zero (a plateau the level bisection stops
    # below) take every block they have left at one level; equal shares, shares too small to move the
    # level and distinct ones mixed across requests; 1500 and 3000 requests put 2 and 4 on a thread
    rng = np.random.default_rng(rows)
    scores = []
    for r in range(rows):
        n = int(rng.integers(3, 60))
        kind = r % 4
        if kind == 0:
            x = np.zeros(n)
            x[0] = 1.0  # one block carries everything: the rest are a zero plateau
        elif kind == 1:
            x = np.ones(n)  # equal shares
        elif kind == 2:
            x = np.full(n, 1e-30)
            x[0] = 1.0  # shares below the level's last bit once the first block is kept
        else:
            x = rng.random(n)
        scores.append(x)
    pinned = [oa.default_pins(len(x)) for x in scores]
    total = sum(len(x) for x in scores)
    must = sum(int(q.sum()) for q in pinned)
    for frac in (0.3, 0.6, 0.95):
        budget = max(must, int(frac * total))
        reqs = [allocation.Request(scores=x) for x in scores]
        print(f"{rows} requests, budget {budget} of {total}", flush=True)
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), frac


@pytest.mark.parametrize("sizes", [(12289, 300, 5000), (20000, 16384, 17, 9000), (65535, 40000, 12288),
                                   (65536, 100000, 7), (262144, 70000)])
def test_maxmin_rows_wider_than_a_sort_in_lds(sizes):
    # requests past 12288 blocks sort in global memory and search their running
    # totals in memory; ties (integer scores), explicit pins and a zero tail
    rng = np.random.default_rng(sum(sizes))
    scores = [rng.integers(0, 6, size=n).astype(float) * rng.choice([1e-3, 1.0]) for n in sizes]
    scores[0][-(len(scores[0]) // 5):] = 0.0
    pinned = [oa.default_pins(len(x)) for x in scores]
    pinned[1] = pinned[1].copy()
    pinned[1][:: 97] = True
    total = sum(sizes)
    must = sum(int(q.sum()) for q in pinned)
    for frac in (0.2, 0.55, 0.9):
        budget = max(must, int(frac * total))
        reqs = [allocation.Request(scores=x, pinned=q) for x, q in zip(scores, pinned)]
        print(f"sizes {sizes}, budget {budget}", flush=True)
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), frac


def test_maxmin_float64_scores_zero_rows_and_long_rows():
    rng = np.random.default_rng(6)
    scores = [rng.random(n) * (1 + 1e-9 * rng.random(n)) for n in (8191, 8193, 12288, 50)]
    scores.append(np.zeros(40))  # no evidence: equal shares
    scores.append(np.array([0.0, -1.0, 2.0, np.float64(1e-300)]))
    pinned = [oa.default_pins(len(s)) for s in scores]
    pinned[3] = rng.random(50) < 0.3  # explicit pins
    total = sum(len(s) for s in scores)
    for frac in (0.05, 0.3, 0.7, 0.95):
        budget = max(int(frac * total), sum(int(p.sum()) for p in pinned))
        reqs = [allocation.Request(scores=s, pinned=p) for s, p in zip(scores, pinned)]
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), frac


@pytest.mark.parametrize("spread", [2.0 ** -40, 2.0 ** -30, 2.0 ** -26])
def test_maxmin_shares_that_differ_only_in_low_bits(spread):
    # the per-request sort orders the top 40 bits of each share's key first and sorts again on all 64
    # bits only when two neighbours agree there but are out of order below: shares a few float64
    # ulps apart (1 + k * spread, a handful of distinct values per row) take that second sort, next to
    # rows whose shares differ high up
    rng = np.random.default_rng(int(-np.log2(spread)))
    scores = []
    for n in (8192, 4096, 3000, 1024, 700, 64):
        s = 0.5 * (1.0 + rng.integers(0, 7, size=n) * spread)
        if n == 3000:
            s = rng.random(n)  # no close neighbours: the first sort stands
        scores.append(s)
    pinned = [oa.default_pins(len(s)) for s in scores]
    total = sum(len(s) for s in scores)
    for frac in (0.1, 0.5, 0.9):
        budget = max(int(frac * total), sum(int(q.sum()) for q in pinned))
        reqs = [allocation.Request(scores=s, pinned=q) for s, q in zip(scores, pinned)]
        print(f"spread {spread}, budget {budget}", flush=True)
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), frac


def test_maxmin_ties_in_rows_sorted_in_lds():
    # each request's blocks are sorted in LDS (a stable radix sort by share desc, so equal shares keep
    # block order): rows full of exactly equal shares must keep the stable order the reference's
    # argsort gives
    rng = np.random.default_rng(9)
    scores = [np.round(rng.random(n) * 8) / 8 for n in (8192, 4097, 1000, 64)]  # 9 distinct values
    scores.append(np.full(300, 0.25))
    scores.append(np.zeros(40))
    pinned = [oa.default_pins(len(s)) for s in scores]
    pinned[2] = rng.random(1000) < 0.2
    total = sum(len(s) for s in scores)
    for frac in (0.1, 0.4, 0.6, 0.9):
        budget = max(int(frac * total), sum(int(p.sum()) for p in pinned))
        reqs = [allocation.Request(scores=s, pinned=p) for s, p in zip(scores, pinned)]
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), frac


def test_maxmin_view_build_configuration():
    c = workloads.config4()
    shares, blocks = c["shares"], c["blocks"]
    sizes = blocks.tolist()
    total = int(blocks.sum())
    scores = [shares[r, : sizes[r]] for r in range(len(sizes))]
    pinned = [oa.default_pins(n) for n in sizes]
    s_dev, b_dev = torch.from_numpy(shares).cuda(), torch.from_numpy(blocks).cuda()
    for frac in (0.2, 0.5, 0.8):
        budget = int(np.ceil(frac * total))
        keep, summary = allocation.maxmin_keep(s_dev, b_dev, budget=budget)
        got = keep.cpu().numpy()
        want = oa.allocate_maxmin(scores, pinned, budget)
        bad = sum(int((got[r, : sizes[r]].astype(bool) != want[r]).sum()) for r in range(len(sizes)))
        print(f"maxmin at {frac}: budget {budget}, kept {sum(int(w.sum()) for w in want)}, mismatched {bad}",
              flush=True)
        assert bad == 0 and int(summary[3]) == 0


@pytest.mark.parametrize("rows", [1500, 3000, 6000, 8192, 8193, 20000])
def test_maxmin_many_requests(rows):
    # past 1024 requests each bisection thread carries 2, 4 or 8 of them; past 8192 the bisection
    # keeps every request's state in the workspace
    rng = np.random.default_rng(rows)
    sizes = rng.integers(1, 30, size=rows)
    scores = [rng.random(int(n)) for n in sizes]
    scores[5] = np.zeros(int(sizes[5]))
    pinned = [oa.default_pins(int(n)) for n in sizes]
    total, must = int(sizes.sum()), sum(int(p.sum()) for p in pinned)
    for frac in (0.3, 0.75):
        budget = max(int(frac * total), must)
        reqs = [allocation.Request(scores=s, pinned=p) for s, p in zip(scores, pinned)]
        assert same(allocation.allocate(reqs, budget, "maxmin"), oa.allocate_maxmin(scores, pinned, budget)), frac
