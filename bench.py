"""Benchmark of the audit / share / ranking / view hot path on one MI355X.

Workload: the Llama-3-8B decode shape -- 128 rows with contexts U[512, 8192] tokens, 32 query /
8 KV heads, head_dim 128, bf16, block size 16, a pool of 100k blocks per layer, 32 layers.  A step
is one decode step's worth of the path: the audit kernel after each of the 32 layers (layer L reads
KV group L mod 8 of its own cache; the caches rotate over 4 distinct pools so that the 144 MB a
launch reads is never served by the 256 MB Infinity Cache), the share normalisation over the 32
layers, the uniform ranking at budget 0.5 (first block and 4 newest pinned) and the block-table
view build.  The layers go through RecordingPlane.record, as the engine's hook calls it: the step
plan at the first layer (each audit workgroup's tiles, built once per step from the view buffers by
ekv_audit_plan) and one audit launch over the 32 layers at the last (ekv_audit_tile_lse_layers),
which under the capture reads each layer's query in place (eager steps stage them first).  The step is captured once into a HIP
graph and replayed (the launches are identical every step; the audit flag lives on the device).

value = audited KV bytes (algorithmic, below) per step / step time.  Per layer:
  B = sum_r L_r*d*2 (keys) + sum_r n_r*4 (table) + R*G*d*2 (queries) + R*8 (lengths, token)
      + 2*sum_r n_r*G*4 (m and l cells written)
roofline.achieved = 32 B / the duration of the step's audit launch, timed with HIP events on the
launch stream; roofline.frac counts the step plan into that time.  The
CPU baseline is the reference's CPU path restated by the oracle (PyTorch-CPU audit, NumPy
normalisation, ranking and compaction) on the same step, each stage the median of 5 runs.

Only one GPU is used: ``--gpus N`` with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sigmod-kvscope_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
LAYERS = 32
POOLS = 4
FRACTION = 0.5
RECENT = 4


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-repeats", type=int, default=5, help="timed repetitions of each CPU-baseline stage")
    ap.add_argument("--chunk-tiles", type=int, default=0)
    ap.add_argument("--profile-only", action="store_true", help="run the graph replays only (for rocprof)")
    ap.add_argument("--objectives-only", action="store_true",
                    help="time the 1024 x 8192 view build and the sum / maxmin objectives only (for rocprof)")
    return ap.parse_args()


def audit_bytes(batch, audited_heads: int = 1, key_bytes: int = 2, query_bytes: int = 2) -> int:
    lens = batch.lens.astype("int64")
    n = batch.blocks.astype("int64")
    g, d = batch.group_rows, batch.head_dim
    return int(
        lens.sum() * d * key_bytes * audited_heads
        + n.sum() * 4
        + batch.rows * g * audited_heads * d * query_bytes
        + batch.rows * 8
        + 2 * n.sum() * g * audited_heads * 4
    )


def graph_launch_us(launches, count: int, reps: int) -> float:
    """Mean duration (us) of one of the ``count`` launches that ``launches(stream)`` makes, from a
    HIP graph of them replayed ``reps`` times and timed with events on the replay stream."""
    import torch

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launches(int(torch.cuda.current_stream().cuda_stream))
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * count)


def other_audit_shapes() -> dict:
    """The audit kernel on the skewed long-context mix and on the 256-row fp8 full step (per-row
    timer on): one KV group per launch, layers rotating over pools larger than the Infinity Cache."""
    import numpy as np
    import torch

    import workloads
    from runtime.audit_kernel import RecordingPlane

    out = {}
    # skewed mix: 8 rows of 131072 tokens + 120 Zipf(1.2) rows on [1024, 4096], bf16, 2 pools
    b3 = workloads.config3_batch()
    pools = [workloads.device_pool(b3, torch.bfloat16, seed=b3.seed + i) for i in range(2)]
    q3 = torch.from_numpy(workloads.queries(b3, 8)).to(torch.bfloat16).cuda()
    plane = RecordingPlane(8, b3.rows, b3.width, b3.group_rows, b3.block_size)
    plane.attach([pool.data_ptr() for pool in pools])
    plane.select(np.ones(b3.rows, bool), np.arange(b3.rows))
    plane.set(True)
    t3, l3 = torch.from_numpy(b3.table).cuda(), torch.from_numpy(b3.lens).cuda()
    plane.plan(t3, l3)  # the step plan the launches share
    us = graph_launch_us(lambda s: [plane.launch(layer, t3, l3, q3[layer], pools[layer % 2][:, 0],
                                                 b3.head_dim ** -0.5, planned=True, stream=s) for layer in range(8)],
                         8, 10)
    entries3 = [plane.direct(layer, q3[layer], pools[layer % 2][:, 0], b3.head_dim ** -0.5) for layer in range(8)]
    us_batched = graph_launch_us(lambda s: plane.launch_layers(entries3, pools[0][:, 0], q3[0], staged=False,
                                                               stream=s), 8, 10)
    bytes3 = audit_bytes(b3)
    out["skewed_long_context_bf16"] = {"bytes_per_layer": bytes3, "us_per_layer_launch": round(us, 2),
                                       "us_per_layer_in_8_layer_launch": round(us_batched, 2),
                                       "gbs": round(bytes3 / us_batched / 1e3, 1),
                                       "frac": round(bytes3 / us_batched / 1e3 / HBM_PEAK_GBS, 4),
                                       "frac_per_layer_launch": round(bytes3 / us / 1e3 / HBM_PEAK_GBS, 4)}
    del pools, q3, plane
    torch.cuda.empty_cache()
    # full step: 256 rows of U[2048, 32768] tokens, block 32, fp8 keys with a per-tensor scale, 32 layers
    b5 = workloads.config5_batch()
    fp8 = torch.float8_e4m3fn
    pools = [workloads.device_pool(b5, fp8, seed=b5.seed + i) for i in range(2)]
    q5 = torch.from_numpy(workloads.queries(b5, LAYERS)).to(torch.bfloat16).cuda()
    plane = RecordingPlane(LAYERS, b5.rows, b5.width, b5.group_rows, b5.block_size, timer=True)
    plane.attach([pools[layer % 2].data_ptr() for layer in range(LAYERS)])
    plane.select(np.ones(b5.rows, bool), np.arange(b5.rows))
    plane.set(True)
    t5, l5 = torch.from_numpy(b5.table).cuda(), torch.from_numpy(b5.lens).cuda()
    k_scale = b5.extra["k_scale"]
    plane.plan(t5, l5)
    us = graph_launch_us(lambda s: [plane.launch(layer, t5, l5, q5[layer], pools[layer % 2][:, 0],
                                                 b5.head_dim ** -0.5, k_scale=k_scale, planned=True, stream=s)
                                    for layer in range(LAYERS)], LAYERS, 5)
    entries5 = [plane.direct(layer, q5[layer], pools[layer % 2][:, 0], b5.head_dim ** -0.5, k_scale=k_scale)
                for layer in range(LAYERS)]
    us_batched = graph_launch_us(lambda s: plane.launch_layers(entries5, pools[0][:, 0], q5[0], staged=False,
                                                               stream=s), LAYERS, 5)
    bytes5 = audit_bytes(b5, key_bytes=1)
    out["full_step_fp8_256_rows"] = {"bytes_per_layer": bytes5, "us_per_layer_launch": round(us, 2),
                                     "us_per_layer_in_32_layer_launch": round(us_batched, 2),
                                     "ms_per_step": round(us_batched * LAYERS / 1e3, 3),
                                     "gbs": round(bytes5 / us_batched / 1e3, 1),
                                     "frac": round(bytes5 / us_batched / 1e3 / HBM_PEAK_GBS, 4),
                                     "frac_per_layer_launch": round(bytes5 / us / 1e3 / HBM_PEAK_GBS, 4), "timer": True}
    del pools, q5, plane
    torch.cuda.empty_cache()
    return out


class Step:
    """Preallocated buffers and the launches of one step."""

    def __init__(self, batch, chunk_tiles: int):
        import numpy as np
        import torch

        import ekv_hip
        import workloads
        from runtime.audit_kernel import RecordingPlane

        self.ekv = ekv_hip
        self.batch = batch
        self.chunk = chunk_tiles
        dev = "cuda"
        self.pools = [workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + 101 * p) for p in range(POOLS)]
        self.keys = [pool[:, 0] for pool in self.pools]
        qs = workloads.queries(batch, LAYERS)
        self.q = [torch.from_numpy(qs[layer]).to(torch.bfloat16).to(dev) for layer in range(LAYERS)]
        self.table = torch.from_numpy(batch.table).to(dev)
        self.lens = torch.from_numpy(batch.lens).to(dev)
        self.blocks = torch.from_numpy(batch.blocks.astype(np.int32)).to(dev)
        self.plane = RecordingPlane(LAYERS, batch.rows, batch.width, batch.group_rows, batch.block_size)
        self.plane.attach([self.pools[layer % POOLS].data_ptr() for layer in range(LAYERS)])
        self.plane.select(np.ones(batch.rows, bool), np.arange(batch.rows))
        self.plane.set(True)
        R, W = batch.rows, batch.width
        self.shares = torch.empty(R, W, dtype=torch.float32, device=dev)
        need = int(self.ekv.load().ekv_tile_shares_workspace(R, W, LAYERS))
        self.shares_ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)  # zeroed once
        self.keep = torch.empty(R, W, dtype=torch.uint8, device=dev)
        self.summary = torch.zeros(6, dtype=torch.int64, device=dev)
        self.view = torch.zeros(R, W, dtype=torch.int32, device=dev)
        self.view_lens = torch.zeros(R, dtype=torch.int32, device=dev)
        self.counts = torch.zeros(R, 5, dtype=torch.int64, device=dev)  # per-row view counters
        self.scale = batch.head_dim ** -0.5

    def plan(self, stream: int) -> None:
        # the step plan: the work list the step's audits share, built once from the view buffers
        self.plane.plan(self.table, self.lens, stream=stream)

    def audit(self, layer: int, stream: int, planned: bool = True) -> None:
        """One layer's own audit launch (the per-layer form the batched launch replaces)."""
        self.plane.launch(layer, self.table, self.lens, self.q[layer], self.keys[layer % POOLS], self.scale,
                          planned=planned, chunk_tiles=self.chunk, stream=stream)

    def record_layers(self) -> None:
        """The 32 layers as the engine's hook records them (on the current stream): the plan at the
        first, a staging per layer, one audit launch at the last."""
        for layer in range(LAYERS):
            self.plane.record(f"layer.{layer}", self.table, self.lens, self.q[layer], self.pools[layer % POOLS],
                              self.scale)

    def stage_all(self, stream: int) -> list:
        return [self.plane.stage(layer, self.q[layer], self.keys[layer % POOLS], self.scale, stream=stream)
                for layer in range(LAYERS)]

    def direct_all(self) -> list:
        return [self.plane.direct(layer, self.q[layer], self.keys[layer % POOLS], self.scale) for layer in range(LAYERS)]

    def launch_all(self, entries: list, stream: int, staged: bool = False) -> None:
        self.plane.launch_layers(entries, self.keys[0], self.q[0], staged=staged, stream=stream)

    def shares_rank_view(self, stream: int) -> None:
        b, p = self.batch, self.plane
        plane_stride, layer_stride, row_stride = p.strides
        self.ekv.call(
            "ekv_tile_shares_ws", p.lse_address, plane_stride, layer_stride, row_stride, LAYERS, p.cells, b.width,
            0, self.blocks.data_ptr(), b.rows, 2, self.ekv.AGG_MEAN, self.shares.data_ptr(), b.width,
            self.shares_ws.data_ptr(), self.shares_ws.numel(), stream,
        )
        self.rank_view(stream)

    def rank_view(self, stream: int) -> None:
        # the uniform ranking and DecodeView.build on its keep (live decoding rows, with the read
        # counters), in one kernel: the same keep, view, lengths and counters as ekv_rank_uniform
        # followed by ekv_build_view
        b = self.batch
        self.ekv.call(
            "ekv_rank_uniform_view", self.shares.data_ptr(), b.width, self.blocks.data_ptr(), 0, 0, RECENT,
            b.rows, b.width, FRACTION, -1, self.keep.data_ptr(), b.width, self.summary.data_ptr(),
            self.table.data_ptr(), b.width, self.lens.data_ptr(), b.block_size, self.view.data_ptr(), b.width,
            self.view_lens.data_ptr(), self.counts.data_ptr(), stream,
        )

    def run(self, stream: int) -> None:
        """One step on the current stream (``stream`` is its handle)."""
        self.record_layers()
        self.shares_rank_view(stream)


def time_events(fn, repeats: int, stream) -> list[float]:
    """Durations (ms) of ``fn`` bracketed by events on ``stream``."""
    import torch

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
    for i in range(repeats):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def copy_peak_gbs() -> float:
    """Measured streaming peak: a 1 GiB -> 1 GiB float32 negation (the counter calibration
    kernel), read + write bytes / median time."""
    import torch

    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    stream = torch.cuda.current_stream()
    ms = sorted(time_events(lambda: torch.neg(src, out=dst), 11, stream))[5]
    del src, dst
    torch.cuda.empty_cache()
    return 2 * n * 4 / (ms * 1e-3) / 1e9


def profiled_traffic() -> int | None:
    """HBM bytes per audit launch from the committed FETCH_SIZE / WRITE_SIZE summary of this
    workload (scaled by the calibration kernel), or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "tile_lse_llama3_decode_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        return None
    return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(step: Step, repeats: int) -> dict:
    """The reference's CPU path on the same step, stage by stage: the oracle's PyTorch-CPU audit of
    the 32 layer launches (gather through the table, matmul, tile max / sum exp), the float64 NumPy
    read and normalisation of the 32 layers' records, the controller's uniform ranking (budget 0.5,
    block 0 and the 4 newest pinned) and the compaction of the block table.  Each stage is timed as
    the median of ``repeats`` runs after one warm-up, in this process, on the same seeded inputs."""
    import numpy as np
    import torch

    from oracle import audit as oracle_audit
    from oracle import block_view as oracle_view
    from oracle import controller as oracle_controller
    from oracle import tile_shares as oracle_shares
    import workloads

    # the host's CPU share for this process: its affinity, capped by OMP_NUM_THREADS when set
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(affinity, omp) if omp > 0 else affinity
    torch.set_num_threads(threads)
    b = step.batch
    host = {}
    for layer in range(LAYERS):  # the keys each launch reads, gathered to host memory once (not timed)
        pool, group = layer % POOLS, layer % b.kv_heads
        if (pool, group) not in host:
            keys, table = workloads.host_keys(b, step.pools[pool], heads=[group])
            host[(pool, group)] = (torch.from_numpy(keys).to(torch.bfloat16), table)
    queries = [step.q[layer].cpu() for layer in range(LAYERS)]
    planes = oracle_audit.new_planes(LAYERS, b.rows, b.width, b.group_rows)

    def audit_step() -> None:
        for layer in range(LAYERS):
            group = layer % b.kv_heads
            keys, table = host[(layer % POOLS, group)]
            oracle_audit.tile_lse_torch(planes, queries[layer], keys, table, b.lens, np.arange(b.rows),
                                        np.ones(b.rows), layer, step.scale, b.block_size, b.group_rows, group,
                                        key_head=0)

    got = step.plane.read_planes()
    shares = None
    keep = None

    def normalise() -> None:
        nonlocal shares
        shares = oracle_shares.normalize(oracle_shares.read_rows(got, LAYERS, np.arange(b.rows), 2), b.blocks, 2)

    def rank() -> None:
        nonlocal keep
        keep, _ = oracle_controller.keep_rows(shares.astype(np.float32), b.blocks, np.ones(b.rows), FRACTION,
                                              RECENT, 0)

    def compact() -> None:
        oracle_view.compact(b.table, b.lens, keep.astype(bool), b.block_size)

    stages = {}
    for name, fn in (("audit_32_layers", audit_step), ("normalise_32_layers", normalise), ("uniform_rank", rank),
                     ("compact", compact)):
        fn()  # warm-up
        times = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        stages[name] = float(np.median(times))
    live = ~np.isnan(planes[0])
    err = float(np.abs(got[0][live] - planes[0][live]).max())  # the CPU records agree with the device's
    audit_s = stages["audit_32_layers"]
    return {
        "value": round(LAYERS * audit_bytes(b) / audit_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"the whole step: the 32 layer launches (all 128 rows, one KV group each) with "
                  f"oracle.audit.tile_lse_torch, median of {repeats} passes after one warm-up; tile max agrees "
                  f"with the GPU to {err:.1e}",
        "cpu_model": cpu_model(),
        "host_logical_cpus": os.cpu_count(),
        "affinity_cpus": affinity,
        "step_stages_s": {k: round(v, 4) for k, v in stages.items()},
        "step_s": round(sum(stages.values()), 4),
    }


def view_build_config(handle: int, stream) -> dict:
    """Medians (ms) of the view build (uniform ranking + compaction) and the sum / maxmin objectives on
    1024 rows x U[1, 8192] blocks at budget 0.5."""
    import numpy as np
    import torch

    import ekv_hip
    import workloads
    from observe.allocation import maxmin_keep, sum_keep

    # ranking + compaction of 1024 rows x up to 8192 blocks
    c4 = workloads.config4()
    s4 = torch.from_numpy(c4["shares"]).cuda()
    n4 = torch.from_numpy(c4["blocks"]).cuda()
    t4 = torch.from_numpy(c4["table"]).cuda()
    l4 = torch.from_numpy(c4["seq_lens"]).cuda()
    k4 = torch.empty_like(s4, dtype=torch.uint8)
    v4 = torch.empty_like(t4)
    vl4 = torch.empty_like(l4)
    sm4 = torch.zeros(6, dtype=torch.int64, device="cuda")

    def rank_c4():
        ekv_hip.call("ekv_rank_uniform", s4.data_ptr(), 8192, n4.data_ptr(), 0, 0, 0, 0, 0, 0, 0, 1024, 8192, 0.5,
                     -1, k4.data_ptr(), 8192, sm4.data_ptr(), handle)

    def compact_c4():
        ekv_hip.call("ekv_compact_view", t4.data_ptr(), 8192, l4.data_ptr(), k4.data_ptr(), 8192, 1024, 8192, 16,
                     v4.data_ptr(), 8192, vl4.data_ptr(), handle)

    def view_build_c4():
        rank_c4()
        compact_c4()

    def fused_c4():  # the same two results from one kernel (ekv_rank_uniform_view)
        ekv_hip.call("ekv_rank_uniform_view", s4.data_ptr(), 8192, n4.data_ptr(), 0, 0, 0, 1024, 8192, 0.5, -1,
                     k4.data_ptr(), 8192, sm4.data_ptr(), t4.data_ptr(), 8192, l4.data_ptr(), 16, v4.data_ptr(),
                     8192, vl4.data_ptr(), 0, handle)

    view_build_c4()
    fused_c4()
    out = {"view_build": float(np.median(time_events(fused_c4, 20, stream))),
           "view_build_two_calls": float(np.median(time_events(view_build_c4, 20, stream))),
           "rank": float(np.median(time_events(rank_c4, 20, stream))),
           "compact": float(np.median(time_events(compact_c4, 20, stream)))}
    # the other objectives on the same rows: sum (global top-k) and maxmin (water level)
    s4_64 = s4.double()
    b4 = int(np.ceil(0.5 * int(c4["blocks"].sum())))
    sum_keep(s4_64, n4, budget=b4)
    out["sum"] = float(np.median(time_events(lambda: sum_keep(s4_64, n4, budget=b4), 10, stream)))
    maxmin_keep(s4_64, n4, budget=b4)
    out["maxmin"] = float(np.median(time_events(lambda: maxmin_keep(s4_64, n4, budget=b4), 5, stream)))
    return out


def calibration_copy() -> int:
    """A plain streaming kernel of known size (one read and one write of 256 MiB, the only negation
    in a profiling run), to scale the memory counters of the kernels around it; returns its bytes
    each way."""
    import torch

    calib_bytes = 256 << 20
    src = torch.ones(calib_bytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    return calib_bytes


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); this library has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import workloads

    torch.cuda.set_device(0)
    if args.objectives_only:
        stream = torch.cuda.current_stream()
        calibration_copy()
        times = view_build_config(int(stream.cuda_stream), stream)
        print(json.dumps({"objectives_only": True, **{k + "_us": round(v * 1e3, 2) for k, v in times.items()}}))
        return
    batch = workloads.config2_batch()
    step = Step(batch, args.chunk_tiles)
    stream = torch.cuda.current_stream()
    handle = int(stream.cuda_stream)

    # eager reference of one step, then the captured graph; every replay must reproduce it
    step.run(handle)
    torch.cuda.synchronize()
    eager = (step.shares.clone(), step.keep.clone(), step.view.clone(), step.view_lens.clone())
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for _ in range(2):
            step.run(int(side.cuda_stream))
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step.run(int(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        now = (step.shares, step.keep, step.view, step.view_lens)
        for a, b in zip(eager, now):
            if not torch.equal(a, b) and not (a.is_floating_point() and torch.equal(torch.nan_to_num(a), torch.nan_to_num(b))):
                raise RuntimeError("a graph replay differs from the eager step")

    if args.profile_only:
        calib_bytes = calibration_copy()
        for _ in range(args.warmup + args.steps):
            graph.replay()
        torch.cuda.synchronize()
        # the event-timed step audit launch in the same run, for comparison with the trace
        entries = step.direct_all()
        launch_us = graph_launch_us(lambda s: step.launch_all(entries, s), 1, 10)
        print(json.dumps({"profile_only": True, "steps": args.steps, "calibration_copy_bytes": calib_bytes,
                          "audit_launch_us_events": round(launch_us, 2)}))
        return

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / args.steps

    # the step's audit launch alone: a graph of it (over the 32 layers' staged queries and the plan the
    # steps above built), replayed and timed with events on the stream it runs on; the 32 stagings and
    # the plan the same way; and for comparison the per-layer launches it replaces (planned, and
    # self-contained: each launch building its work list itself)
    def graph_ms(launches, reps: int) -> float:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launches(int(torch.cuda.current_stream().cuda_stream))
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        for _ in range(reps):
            g.replay()
        a1.record(stream)
        torch.cuda.synchronize()
        return a0.elapsed_time(a1) / reps

    reps = max(10, args.steps // 2)
    entries = step.direct_all()  # the captured step's launch reads the queries in place
    launch_ms = graph_ms(lambda s: step.launch_all(entries, s), reps)
    staged = step.stage_all(handle)  # an eager step stages them first
    torch.cuda.synchronize()
    staged_launch_ms = graph_ms(lambda s: step.launch_all(staged, s, staged=True), reps)
    stage_ms = graph_ms(lambda s: step.stage_all(s), reps) / LAYERS
    plan_ms = float(np.median(time_events(lambda: step.plan(handle), 20, stream)))
    per_layer_ms = graph_ms(lambda s: [step.audit(layer, s) for layer in range(LAYERS)], reps) / LAYERS
    self_contained_ms = graph_ms(lambda s: [step.audit(layer, s, planned=False) for layer in range(LAYERS)],
                                 reps) / LAYERS
    # the other stages of the step
    shares_ms = float(np.median(time_events(lambda: step.ekv.call(
        "ekv_tile_shares_ws", step.plane.lse_address, *step.plane.strides, LAYERS, step.plane.cells, batch.width, 0,
        step.blocks.data_ptr(), batch.rows, 2, step.ekv.AGG_MEAN, step.shares.data_ptr(), batch.width,
        step.shares_ws.data_ptr(), step.shares_ws.numel(), handle),
        20, stream)))
    view_ms = float(np.median(time_events(lambda: step.rank_view(handle), 20, stream)))

    b_launch = audit_bytes(batch)
    b_step = LAYERS * b_launch
    achieved = b_step / (launch_ms * 1e-3) / 1e9
    with_overheads = b_step / ((launch_ms + plan_ms) * 1e-3) / 1e9
    value = b_step / (ms_per_step * 1e-3) / 1e9

    # the every-KV-head audit (1.14 GB of keys per launch): same kernel, all 8 groups per launch
    from runtime.audit_kernel import RecordingPlane

    all_plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size, kv_heads=batch.kv_heads)
    all_plane.attach([step.pools[0].data_ptr()])
    all_plane.select(np.ones(batch.rows, bool), np.arange(batch.rows))
    all_plane.set(True)
    all_plane.plan(step.table, step.lens)
    all_ms = float(np.median(time_events(
        lambda: all_plane.launch(0, step.table, step.lens, step.q[0], step.keys[0], step.scale, planned=True),
        10, stream)))
    all_gbs = audit_bytes(batch, batch.kv_heads) / (all_ms * 1e-3) / 1e9

    c4_times = view_build_config(handle, stream)
    others = other_audit_shapes()
    peak = copy_peak_gbs()
    traffic = profiled_traffic()
    out = {
        "metric": "audit KV GB/s (% HBM peak) at Llama-3-8B decode shape; view build us",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) bf16 keys and queries, seeded tables and lengths",
        "config": {
            "workload": "Llama-3-8B decode audit step: 128 rows, L~U[512,8192], 32q/8kv heads, d=128, bf16, "
                        "block 16, 32 layers (one KV group each, 4 rotating 100k-block pools), shares + uniform "
                        "ranking at 0.5 + view build, HIP-graph replay",
            "rows": batch.rows,
            "layers": LAYERS,
            "audited_tokens": int(batch.lens.sum()),
            "audit_bytes_per_launch": b_launch,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(with_overheads, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(with_overheads / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "ekv_audit_tile_lse_layers (tile_lse_layers_kernel: the step's 32 layers, one KV group each)",
            "bytes_per_launch": b_step,
            "launch_us": round(launch_ms * 1e3, 2),
            "achieved_launch_only": round(achieved, 1),
            "frac_launch_only": round(achieved / HBM_PEAK_GBS, 4),
            "counted_in_frac": "the launch + the step plan (the captured step reads the queries in place: no staging)",
            "traffic_source": "profiles/tile_lse_llama3_decode_traffic.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                              "scaled by a 256 MiB streaming kernel)",
            "measured_copy_peak_gbs": round(peak, 1),
            "frac_of_measured_peak": round(with_overheads / peak, 4),
        },
        "stages_us": {
            "audit_launch_32_layers": round(launch_ms * 1e3, 2),
            "audit_plan_per_step": round(plan_ms * 1e3, 2),
            "query_staging_per_layer_eager": round(stage_ms * 1e3, 2),
            "audit_launch_32_layers_staged_queries": round(staged_launch_ms * 1e3, 2),
            "audit_per_layer_launch": round(per_layer_ms * 1e3, 2),
            "audit_per_layer_launch_self_contained": round(self_contained_ms * 1e3, 2),
            "shares_32_layers": round(shares_ms * 1e3, 2),
            "rank_and_view": round(view_ms * 1e3, 2),
        },
        "every_kv_head_audit": {"bytes_per_launch": audit_bytes(batch, batch.kv_heads), "us": round(all_ms * 1e3, 2),
                                "gbs": round(all_gbs, 1), "frac": round(all_gbs / HBM_PEAK_GBS, 4)},
        "other_audit_shapes": others,
        "view_build_us": {"llama3_step_128_rows": round(view_ms * 1e3, 2),
                          "config_1024x8192_budget_0.5": round(c4_times["view_build"] * 1e3, 2),
                          "config_1024x8192_budget_0.5_two_calls": round(c4_times["view_build_two_calls"] * 1e3, 2),
                          "config_1024x8192_rank": round(c4_times["rank"] * 1e3, 2),
                          "config_1024x8192_compact": round(c4_times["compact"] * 1e3, 2),
                          "config_1024x8192_sum_objective": round(c4_times["sum"] * 1e3, 2),
                          "config_1024x8192_maxmin_objective": round(c4_times["maxmin"] * 1e3, 2)},
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(step, max(5, args.cpu_repeats))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
