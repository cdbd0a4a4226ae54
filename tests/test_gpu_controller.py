"""The controller's keep rule under the `sum` and `maxmin` objectives on the device
(observe.controller.keep_rows -> ekv_controller_keep) against oracle.controller.keep_rows, which
restates Controller._allocate (observe/controller.py:398-451): known answers of the reference's
controller tests (which run under its default objective, `sum`), the tie between requests counted
among each request's remaining blocks, random batches with every input of the rule, and the
1024-row view-build configuration at cap 256.  Keep masks and budgets must be bit-identical."""

import numpy as np
import pytest
import torch

import workloads
from observe.controller import keep_rows
from oracle import controller as oc

pytestmark = pytest.mark.gpu


def run(shares, lengths, evidence, fraction, recent, cap, audited=None, released=None, weights=None,
        objective="sum"):
    dev = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
    keep, summary = keep_rows(dev(shares), dev(lengths.astype(np.int32)), dev(evidence.astype(np.uint8)), fraction,
                              objective=objective, recent_blocks=recent, cap_above_blocks=cap,
                              audited_blocks=dev(None if audited is None else audited.astype(np.int32)),
                              released=dev(None if released is None else released.astype(np.uint8)),
                              weights=dev(weights))
    want, budget = oc.keep_rows(np.asarray(shares, np.float64), lengths, evidence, fraction, recent, cap, audited,
                                released, objective=objective, weights=weights)
    got = keep.cpu().numpy()
    s = summary.cpu().numpy()
    assert np.array_equal(got, want), np.argwhere(got != want)[:8].tolist()
    if budget:
        assert s[0] == budget and s[3] == 0
    return got, s


def diffuse(n, width):
    s = np.zeros(width)
    s[:n] = 1.0 / n
    return s


def concentrated(n, width):
    s = np.zeros(width)
    s[:n] = 0.02 / (n - 1)
    s[3] = 0.98
    s[:n] /= s[:n].sum()
    return s


@pytest.mark.parametrize("objective", ["sum", "maxmin"])
def test_reference_controller_cases(objective, known_answers):
    width = 16
    shares = np.stack([diffuse(14, width), diffuse(6, width), np.zeros(width)])
    for case, cap in ((known_answers["controller"]["cap_trims_only_long_requests"], 8),
                      (known_answers["controller"]["without_a_cap_both_are_trimmed"], 0)):
        keep, summary = run(shares, np.array(case["lengths"]), np.array([1, 1, 0]), case["fraction"],
                            case["recent_blocks"], cap, objective=objective)
        if cap:
            assert keep[0, :14].sum() == case["kept_long"] and keep[1, :6].sum() == case["short_reads_in_full"]
            assert summary[4] == 1  # only the long request is allocated
        else:
            assert keep[0, :14].sum() + keep[1, :6].sum() == case["kept_total"]
    shares = np.stack([concentrated(12, width), diffuse(12, width)])
    keep, _ = run(shares, np.array([12, 12]), np.array([1, 1]), 0.5, 1, 0, objective=objective)
    kept = keep[:, :12].sum(axis=1)
    assert kept[0] < kept[1] and keep[0, 3] and keep[:, 0].all() and keep[:, 11].all()


def test_sum_tie_counts_the_requests_remaining_blocks():
    width = 6
    shares = np.array([[0.25, 0.125, 0.9, 0.125, 0.375, 0.125],
                       [0.25, 0.125, 0.0625, 0.0625, 0.375, 0.125]])
    released = np.zeros((2, width), dtype=bool)
    released[0, 2] = True
    keep, summary = run(shares, np.array([6, 6]), np.array([1, 1]), 0.4, 0, 0, released=released)
    assert summary[0] == 5
    assert np.flatnonzero(keep[0]).tolist() == [0, 5] and np.flatnonzero(keep[1]).tolist() == [0, 4, 5]


@pytest.mark.parametrize("seed", range(30))
def test_random_batches(seed):
    rng = np.random.default_rng(900 + seed)
    rows = int(rng.integers(1, 40))
    width = int(rng.choice([1, 5, 64, 300, 1025]))
    objective = "sum" if seed % 2 == 0 else "maxmin"
    lengths = rng.integers(0, width + 8, size=rows)
    evidence = rng.random(rows) < 0.85
    cap = int(rng.choice([0, 0, 3, width // 2]))
    recent = int(rng.integers(0, 5))
    audited = rng.integers(0, width + 4, size=rows) if seed % 3 else None
    released = (rng.random((rows, width)) < rng.choice([0.0, 0.1, 0.4])) if seed % 4 else None
    dtype = np.float32 if seed % 5 else np.float64
    shares = rng.dirichlet(np.full(width, 0.3), size=rows).astype(dtype)
    if seed % 7 == 0:
        shares[:, ::3] = shares[:, :1]  # ties inside a request and across requests
    weights = None
    if objective == "sum" and seed % 6:
        weights = rng.choice([0.5, 1.0, 2.0, 3.0], size=rows).astype(np.float64)
    fraction = float(rng.choice([0.05, 0.3, 0.5, 0.8, 1.0]))
    print(f"seed {seed}: {objective} rows {rows} width {width} cap {cap} recent {recent} fraction {fraction}",
          flush=True)
    run(shares, lengths, evidence, fraction, recent, cap, audited, released, weights, objective)


@pytest.mark.parametrize("rows", [8193, 12000])
def test_maxmin_more_requests_than_the_bisection_registers(rows):
    # past 8192 measured rows the bisection keeps each request's state in the workspace
    rng = np.random.default_rng(rows)
    width = 24
    lengths = rng.integers(0, width + 4, size=rows)
    evidence = rng.random(rows) < 0.9
    shares = rng.dirichlet(np.full(width, 0.3), size=rows)
    shares[::11, ::2] = shares[::11, :1]  # ties inside requests
    for fraction in (0.3, 0.7):
        print(f"maxmin: {rows} rows, fraction {fraction}", flush=True)
        run(shares, lengths, evidence, fraction, 2, 3, None, None, None, "maxmin")


@pytest.mark.parametrize("objective", ["sum", "maxmin"])
def test_view_build_configuration_at_cap_256(objective):
    c = workloads.config4()
    rows = c["blocks"].shape[0]
    print(f"{objective}: {rows} rows", flush=True)
    keep, summary = run(c["shares"], c["blocks"].astype(np.int64), np.ones(rows, bool), 0.5, 4, 256,
                        objective=objective)
    assert summary[4] == int((c["blocks"] > 256).sum())


def test_sum_rows_wider_than_a_register_row():
    # the default objective on rows past 16384 blocks (the wider tie key): released blocks, audit
    # lengths, a row under the cap and one without evidence, weights
    rng = np.random.default_rng(21)
    rows, width = 5, 20000
    shares = rng.integers(0, 4, size=(rows, width)).astype(np.float64)  # equal gains: ties at the cut
    lengths = np.array([20000, 16385, 300, 19999, 12000])
    evidence = np.array([1, 1, 1, 0, 1])
    audited = np.array([19000, 16385, 300, 0, 11000])
    released = (rng.random((rows, width)) < 0.05).astype(np.uint8)
    weights = np.array([1.0, 2.0, 0.5, 1.0, 1.5])
    for fraction in (0.3, 0.6):
        run(shares, lengths, evidence, fraction, 4, 256, audited=audited, released=released, weights=weights)


@pytest.mark.parametrize("width", [30000, 70000])
def test_maxmin_rows_wider_than_a_sort_in_lds(width):
    # the maxmin rule on rows past 12288 blocks (the sort in global memory), and past 65535
    # (level positions in 32 bits)
    rng = np.random.default_rng(22)
    rows = 4
    shares = rng.random((rows, width))
    lengths = np.array([width, 12289, 20000, 500])
    evidence = np.array([1, 1, 1, 1])
    audited = np.array([width - 1000, 12289, 15000, 500])
    released = (rng.random((rows, width)) < 0.03).astype(np.uint8)
    for fraction in (0.3, 0.7):
        run(shares, lengths, evidence, fraction, 4, 256, audited=audited, released=released, objective="maxmin")
