#!/usr/bin/env python3
"""Benchmark: QPS at recall@10 >= 0.95 on config 2, plus build vectors/s.

Workload (the configuration the metric is quoted on): 1,000,000 x 128
vectors from a mixture of 1,000 Gaussian clusters (centres U[0,128]^128,
sigma 20, clipped to [0,218], rounded to integers, fp16); 10,000 queries from
the same mixture; Vamana R = 64, alpha = 1.2; k = 10; limit = 2 * beam width.

Procedure
  1. generate the data (seeded, jasper_amd.datasets) and copy it to HBM;
  2. build the graph on the GPU (timed: build vectors/s, device-resident
     input, the reference's batch schedule);
  3. exact ground truth on the GPU;
  4. sweep the beam width over 16..256 and pick the smallest one whose
     recall@10 reaches the target;
  5. a "step" is one search call over all queries at that beam width
     (inputs resident in HBM, output allocation included as in the
     reference's bench); W untimed steps, then K timed steps between
     device synchronisations;
  6. roofline of the search kernel: algorithmic bytes per launch from the
     kernel's own exact work counters (hops, adjacency entries read,
     distinct vectors scored, each at the bytes of the row format the query
     reads: the graph's byte rows, dim bytes, or its fp16 rows, 2 dim bytes)
     divided by the kernel time measured with HIP events on the stream the
     kernel runs on;
  7. CPU baseline (rank 0, N = 1): the exact kNN scan restated from the
     reference's ground-truth arithmetic, on a bounded query sample, all
     host cores.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time

import numpy as np

METRIC = "QPS @ recall@10≥0.95, 1M×128 fp16 synthetic; build vectors/sec"
PEAK_HBM_GBS = 8000.0


def measured_traffic(beam_width: int, n: int, nq: int, row_bytes: int = 256,
                     profile: str = "beam_search_c2_1M_pmc.md"):
    """HBM bytes per launch of a kernel from a committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary, when it covers this exact workload and
    row format; None otherwise (the counters cannot be read from inside this
    process)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", profile)
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r"machine-readable: traffic_bytes_per_launch=(\d+) beam_width=(\d+) n=(\d+) nq=(\d+) "
                  r"row_bytes=(\d+)", text)
    if not m or tuple(int(m.group(i)) for i in range(2, 6)) != (beam_width, n, nq, row_bytes):
        return None
    return int(m.group(1))


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(base: np.ndarray, queries: np.ndarray, target_s: float) -> dict:
    """Exact kNN scan (oracle restatement of the reference ground-truth
    arithmetic) on a query sample sized to about `target_s` seconds."""
    import oracle
    oracle.ensure_built()
    cores = len(os.sched_getaffinity(0))
    vb = base.astype(np.float32)
    qs = queries.astype(np.float32)
    m = 8
    t0 = time.perf_counter()
    oracle.bruteforce_ref(vb, qs[:m], k=10, nthreads=cores)
    dt = time.perf_counter() - t0
    m2 = int(min(len(qs), max(m, m * target_s / max(dt, 1e-3))))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.bruteforce_ref(vb, qs[:m2], k=10, nthreads=cores)
        times.append(time.perf_counter() - t0)
        if sum(times) > 2.5 * target_s:
            break
    t = float(np.median(times))
    return {
        "value": m2 / t,
        "unit": "queries/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"exact L2 kNN scan (||q||^2+||v||^2-2q.v, fp32, top-10) of {m2} of the "
                   f"{len(qs)} queries against all {len(base)} base vectors, median of "
                   f"{len(times)} runs, {cores} threads on {_cpu_model()}"),
    }


def _median_time(fn, runs: int = 3) -> float:
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def cpu_routines(cores: int) -> list:
    """The rest of the reference's CPU path, each on a bounded sample, median
    of 3 warm runs on `cores` threads (the rotation-matrix factorisation and
    best_rescale_factor are sequential in the reference and run on one):
    the config 1 exact scan in full, the host distance routines at d = 128,
    96 and 960 (2M, 2M and 0.5M pairs from fixed pools), RaBitQ one-bit
    quantisation of 250,000 of 1M x 128 rows, the best_rescale_factor loop of
    get_const_scaling_factors (1,000 unit rows) and set_rotation_matrix at
    d = 96, 128 and 960."""
    import oracle
    from jasper_amd import datasets
    oracle.ensure_built()
    items = []
    base1, q1, _ = datasets.config("c1")
    b1, qf = base1.astype(np.float32), q1.astype(np.float32)
    oracle.bruteforce_ref(b1, qf, k=10, nthreads=cores)
    t = _median_time(lambda: oracle.bruteforce_ref(b1, qf, k=10, nthreads=cores))
    items.append({"routine": "exact kNN scan, config 1 in full (100 queries x 10,000 x 128, L2, top-10)",
                  "value": len(q1) / t, "unit": "queries/s", "gflops": 2.0 * len(q1) * len(base1) * 128 / t / 1e9,
                  "cores": cores})
    rng = np.random.default_rng(7)
    for d in (128, 96, 960):
        pool = 1 << 17 if d <= 128 else 1 << 14
        total = 2_000_000 if d <= 128 else 500_000
        a = rng.standard_normal((pool, d)).astype(np.float16).view(np.uint16)
        b = rng.standard_normal((pool, d)).astype(np.float16).view(np.uint16)
        reps = (total + pool - 1) // pool

        def run():
            for _ in range(reps):
                oracle.distance_pairs(a, b, "l2", nthreads=cores)
        run_pairs = reps * pool
        oracle.distance_pairs(a, b, "l2", nthreads=cores)
        t = _median_time(run)
        items.append({"routine": f"host L2 distance routine (distance.cuh l2_distance order), d={d}",
                      "value": run_pairs / t, "unit": "distances/s",
                      "gb_per_s": run_pairs * 4.0 * d / t / 1e9, "sample": f"{run_pairs} pairs from two "
                      f"{pool}-row fp16 pools", "cores": cores})
    x = rng.standard_normal((1_000_000, 128)).astype(np.float32)
    P, _ = oracle.rotation_matrix(128, 42)
    c = x.mean(axis=0)
    xs = x[:250_000]
    oracle.rabitq_quantize(x[:10000], P, c, nthreads=cores)
    t = _median_time(lambda: oracle.rabitq_quantize(xs, P, c, nthreads=cores))
    items.append({"routine": "RaBitQ one-bit quantize (rotation, residual, sign code, f_add, f_rescale) of "
                             "250,000 rows of a 1,000,000 x 128 set (centroid = its mean)",
                  "value": len(xs) / t, "unit": "vectors/s", "cores": cores})
    del x, xs
    o = rng.standard_normal((1000, 128)).astype(np.float32)
    o = np.abs(o / np.linalg.norm(o, axis=1, keepdims=True)).astype(np.float32)
    t = _median_time(lambda: oracle.const_scaling_factor(o, 1))
    items.append({"routine": "best_rescale_factor over get_const_scaling_factors' 1,000 unit rows, d=128, 1 bit",
                  "value": t * 1e3, "unit": "ms", "cores": 1})
    for d in (96, 128, 960):
        t = _median_time(lambda: oracle.rotation_matrix(d, 42), runs=3 if d <= 128 else 1)
        items.append({"routine": f"set_rotation_matrix (N(0,1) matrix, Householder QR, sign fix), d={d}",
                      "value": t * 1e3, "unit": "ms", "cores": 1})
    return items


def general_path_run(args, bw: int, log) -> dict:
    """The same build and search with the integer-row shortcuts off (the
    packed-difference distances and the exact integer Gram prune), in a child
    process (the switch is read once per process): config 2's numbers on the
    path every other dataset takes."""
    import subprocess
    cmd = [sys.executable, "-u", os.path.abspath(__file__), "--int-exact", "0", "--sweep", str(bw), "--steps",
           str(args.steps), "--warmup", str(args.warmup), "--n", str(args.n), "--nq", str(args.nq),
           "--no-cpu-baseline"]
    log(f"general path (JASPER_INT_EXACT=0) at bw={bw} in a child process")
    r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=1200)
    if r.returncode != 0:
        raise RuntimeError(f"general-path run failed with exit code {r.returncode}")
    line = json.loads(r.stdout.strip().splitlines()[-1])
    cfg = line["config"]
    return {"beam_width": cfg["beam_width"], "qps": line["value"], "recall_at_10": cfg["recall_at_10"],
            "ms_per_step": line["ms_per_step"], "kernel_ms": line["roofline"]["kernel_ms"],
            "roofline_frac": line["roofline"]["frac"], "build_vectors_per_s": cfg["build_vectors_per_s"],
            "build_s": cfg["build_s"], "kernel": line["roofline"]["kernel"]}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--target-recall", type=float, default=0.95)
    ap.add_argument("--sweep", default="16,24,32,40,44,48,64,96,128,192,256")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--curve-out", default=None, help="also write the QPS/recall curve as JSON here")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a 512 MiB device-to-device copy (3 times) first: the reference kernel of "
                         "known traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--calibrate-gather", action="store_true",
                    help="gather 1M random rows of 64, 128, 192 and 256 bytes (index_select from 256 MiB "
                         "tables) first: reference kernels of known traffic for the counters of random reads")
    ap.add_argument("--path", default="search",
                    choices=["search", "directional", "pq", "bruteforce", "rotate", "rabitq", "c4", "c5", "c5plain",
                             "updates", "scale", "diskann"],
                    help="search (default, the headline metric) or one of the other hot-path rows, each "
                         "printing its own JSON line: directional (config 3, LSH), pq (PQ-ADC on "
                         "config 3's data), bruteforce (exact k-NN, config 2), rotate (prerotation), "
                         "rabitq (one-bit codes), c4 (config 4: 1M x 960 build + PQ search), c5 "
                         "(config 5: 100M x 128 in-HBM build + LSH k=16 directional search), c5plain (config 5's rows "
                         "without prerotation: plain build and search on byte rows), updates "
                         "(config 2: mark_deleted 10%%, consolidate, append 100k), scale (config 2: the "
                         "partitioned build), diskann (config 2: the DiskANN build)")
    ap.add_argument("--scale-parts", default="4,2,8", help="partition counts of --path scale (first = the line's value)")
    ap.add_argument("--diskann-parts", default="8,4,16", help="shard counts of --path diskann (first = the line's value)")
    ap.add_argument("--c5-n", type=int, default=100_000_000, help="base size of --path c5")
    ap.add_argument("--c4-m", type=int, default=120, help="PQ subspaces of --path c4 (120 = one per 8 dims)")
    ap.add_argument("--rotate-dim", type=int, default=128, help="row dimension of --path rotate (128 or 960)")
    ap.add_argument("--no-build-roofline", action="store_true",
                    help="skip the two extra builds that count the build's work and time its stages (profiler runs)")
    ap.add_argument("--no-general-path", action="store_true",
                    help="skip the child-process run with the integer-row shortcuts off (profiler runs)")
    ap.add_argument("--nq-sweep", default="",
                    help="comma-separated query counts: after the headline measurement, time the search "
                         "kernel at the chosen beam width on that many queries of the same mixture "
                         "(config.nq_sweep: kernel ms and QPS per count)")
    ap.add_argument("--int-exact", type=int, default=1, choices=[0, 1],
                    help="0: run with the integer-row shortcuts off (JASPER_INT_EXACT=0), the general "
                         "distance and prune paths; the default search run also measures this in a child "
                         "process at its chosen beam width")
    args = ap.parse_args()
    if args.int_exact == 0:
        os.environ["JASPER_INT_EXACT"] = "0"  # read by the library at its first range scan

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); every "
              "index here fits one MI355X, and sharding across GPUs is a design, not code.",
              file=sys.stderr)
        return 2

    import torch
    import jasper_amd
    from jasper_amd import datasets

    torch.cuda.init()
    dev = torch.device("cuda:0")
    log = lambda *a: print("[bench]", *a, file=sys.stderr, flush=True)  # noqa: E731

    if args.calibrate_copy:
        src = torch.empty(512 * 2 ** 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("calibration copy: 3 x 512 MiB device-to-device")
    if args.calibrate_gather:
        gen = torch.Generator(device=dev)
        gen.manual_seed(5)
        for row_bytes in (64, 128, 192, 256):
            rows = 256 * 2 ** 20 // row_bytes
            table = torch.empty((rows, row_bytes // 2), dtype=torch.float16, device=dev)
            idx = torch.randperm(rows, device=dev, generator=gen)[:2 ** 20]
            torch.cuda.synchronize()
            out = table.index_select(0, idx)
            torch.cuda.synchronize()
            del table, idx, out
            log(f"calibration gather: 1,048,576 random rows of {row_bytes} B from a {rows}-row table "
                f"({2 ** 20 * row_bytes} B gathered, 8 MiB of int64 indices)")
    if args.path != "search":
        return OTHER_PATHS[args.path](args, torch, jasper_amd, datasets, dev, log)

    t0 = time.perf_counter()
    base = datasets.clustered(args.n, 128, 0)
    queries = datasets.clustered(args.nq, 128, 1)
    log(f"data generated in {time.perf_counter() - t0:.1f}s: base {base.shape}, queries {queries.shape}")
    base_t = torch.from_numpy(base).to(dev)
    q_t = torch.from_numpy(queries).to(dev)
    torch.cuda.synchronize()

    # ---- build
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base_t, n_neighbors=64, distance="l2", alpha=1.2)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    bst = jasper_amd.last_build_stats()
    log(f"build {args.n} vectors in {build_s:.2f}s ({args.n / build_s:.0f} vec/s), "
        f"batches={int(bst['batches'])} max_batch={int(bst['max_batch'])}")
    # the same build again in this process: the first one also pays the
    # one-time loading of the build's code objects at their first launches
    t0 = time.perf_counter()
    g_rep = jasper_amd.Graph.build(base_t, n_neighbors=64, distance="l2", alpha=1.2)
    torch.cuda.synchronize()
    build_repeat_s = time.perf_counter() - t0
    g_rep.free()
    log(f"build again in the same process: {build_repeat_s:.3f}s ({args.n / build_repeat_s:.0f} vec/s)")

    build_total_ms = bst["total_ms"]
    build_roof = None if args.no_build_roofline else build_roofline(jasper_amd, base_t, 64, build_s, build_total_ms,
                                                                     log)

    # ---- ground truth
    t0 = time.perf_counter()
    gt_ids, _ = jasper_amd.generate_groundtruth(base_t, q_t, k=10, distance="l2",
                                                vector_batch_size=250_000)
    gt = gt_ids.numpy()
    log(f"ground truth in {time.perf_counter() - t0:.1f}s")

    def recall_of(ids: np.ndarray) -> float:
        hits = 0
        for a, b in zip(gt, ids):
            hits += len(set(a.tolist()) & set(b.tolist()))
        return hits / (gt.shape[0] * 10)

    # ---- beam-width sweep
    curve = []
    chosen = None
    for bw in [int(x) for x in args.sweep.split(",")]:
        ids, _ = g.search(q_t, k=10, beam_width=bw)
        torch.cuda.synchronize()
        r = recall_of(ids.cpu().numpy())
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            g.search(q_t, k=10, beam_width=bw)
        torch.cuda.synchronize()
        qps = args.nq * reps / (time.perf_counter() - t0)
        curve.append({"beam_width": bw, "recall_at_10": r, "qps": qps})
        log(f"bw={bw:4d} recall@10={r:.4f} qps={qps:,.0f}")
        if chosen is None and r >= args.target_recall:
            chosen = bw
    if chosen is None:
        chosen = curve[-1]["beam_width"]
        log(f"no beam width reached recall {args.target_recall}; using bw={chosen}")

    # ---- timed steps at the chosen beam width
    for _ in range(args.warmup):
        g.search(q_t, k=10, beam_width=chosen)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    last_ids = None
    for e0, e1 in evs:
        e0.record(stream)
        last_ids, _ = g.search(q_t, k=10, beam_width=chosen)
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / args.steps
    kernel_ms = float(np.mean([e0.elapsed_time(e1) for e0, e1 in evs]))
    final_recall = recall_of(last_ids.cpu().numpy())
    qps = args.nq / (ms_per_step / 1000.0)

    # ---- algorithmic bytes per launch (exact work counters of the same traversal)
    st = g.search_stats(q_t, k=10, beam_width=chosen).astype(np.int64)
    hops, deg, scored = st[:, 0].sum(), st[:, 1].sum(), st[:, 2].sum()
    fmt = g.row_format()
    rows_b = query_row_bytes(fmt, queries, 128)
    alg_bytes = algorithmic_bytes(st, 128, args.nq, rows_b)
    achieved = alg_bytes / (kernel_ms / 1000.0) / 1e9
    log(f"bw={chosen}: {ms_per_step:.3f} ms/step, kernel {kernel_ms:.3f} ms, qps={qps:,.0f}, "
        f"recall={final_recall:.4f}, hops/q={hops / args.nq:.1f}, scored/q={scored / args.nq:.1f}, "
        f"predicted adjacency {st[:, 3].sum() / max(hops, 1):.2f} of hops, "
        f"{alg_bytes / args.nq / 1e3:.1f} KB/q, {achieved:.0f} GB/s")

    result = {
        "metric": METRIC,
        "value": qps,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": search_dtype(fmt, queries),
        "data": "synthetic",
        "config": {
            "workload": (f"config 2: {args.n} x 128 clustered integer-valued fp16 (1000 clusters, "
                         f"sigma 20, clipped [0,218]), Vamana R=64 alpha=1.2, {args.nq} queries, "
                         f"k=10, limit=2*bw"),
            "beam_width": chosen,
            "recall_at_10": final_recall,
            "target_recall": args.target_recall,
            "build_vectors_per_s": args.n / build_s,
            "build_s": build_s,
            "build_repeat_vectors_per_s": args.n / build_repeat_s,
            "build_repeat_s": build_repeat_s,
            "build_max_batch": int(bst["max_batch"]),
            "build_roofline": build_roof,
            "storage": ("fp16 vectors; the search reads byte rows (value - lo) for integer rows spanning "
                        "<= 255 values, and queries in that range as bytes (exact u8 dot products, u32 sums)"
                        if fmt["byte_rows"] else "fp16 vectors, fp32 distance arithmetic"),
            "row_bytes_per_scored_vector": float(rows_b.mean()),
            "curve": curve,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": measured_traffic(chosen, args.n, args.nq, int(rows_b.mean())),
            "kernel": "beam_search_kernel<4,0,false,true>" if fmt["byte_rows"] else "beam_search_kernel<4,0,false>",
            "kernel_ms": kernel_ms,
            "algorithmic_bytes_per_launch": alg_bytes,
            "per_query": {"hops": hops / args.nq, "adjacency_entries": deg / args.nq,
                          "vectors_scored": scored / args.nq},
            # what a kernel that fetches every adjacency entry's vector would
            # move (2 dp bytes per entry, the reference-equivalent figure),
            # and the rate it would need to match this launch's time
            "reference_equivalent_bytes_per_launch": int(deg * 2 * 128),
            "reference_equivalent_gbs": deg * 2 * 128 / (kernel_ms / 1000.0) / 1e9,
            # what the two figures are: achieved counts the bytes the
            # algorithm must read; traffic is what rocprofv3's FETCH_SIZE and
            # WRITE_SIZE count leaving L2 for the memory fabric, which
            # includes reads served by the 256 MB Infinity Cache (config 2's
            # 256 MB vector table fits it), scaled by factors measured on a
            # streaming copy
            "notes": "achieved = algorithmic bytes / kernel time; traffic = L2-to-fabric bytes per launch "
                     "(FETCH_SIZE x 2 + WRITE_SIZE, factors from a streaming copy), which counts Infinity "
                     "Cache hits as well as DRAM reads, so neither figure is a DRAM-only measurement",
        },
    }
    if args.nq_sweep:
        result["config"]["nq_sweep"] = nq_sweep(args, torch, g, datasets, dev, chosen, log)
    if args.int_exact == 1 and args.path == "search" and not args.no_general_path:
        result["config"]["general_path"] = general_path_run(args, chosen, log)
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        result["cpu_baseline"] = cpu_baseline(base, queries, args.cpu_seconds)
        log(f"cpu baseline in {time.perf_counter() - t0:.1f}s: {result['cpu_baseline']['value']:.1f} q/s")
        t0 = time.perf_counter()
        result["cpu_baseline"]["routines"] = cpu_routines(result["cpu_baseline"]["cores"])
        log(f"cpu routines in {time.perf_counter() - t0:.1f}s")
    if args.curve_out:
        with open(args.curve_out, "w") as f:
            json.dump(result, f, indent=1)
    print(json.dumps(result), flush=True)
    g.free()
    return 0


# ------------------------------------------------------------------ other rows

def algorithmic_bytes(st, dp, nq, row_bytes=None):
    """Bytes one plain-search launch must move, from its exact work counters
    [nq, 4] (hops, adjacency entries, vectors scored): a 1-byte degree per
    hop, 4 bytes per adjacency entry, row_bytes[q] per distinct vector query q
    scores (2*dp for fp16 rows, dim for byte rows), plus the fp16 query rows
    and the k=10 (id, distance) outputs."""
    hops, deg = st[:, 0].sum(), st[:, 1].sum()
    rb = np.full(len(st), 2 * dp, dtype=np.int64) if row_bytes is None else np.asarray(row_bytes, dtype=np.int64)
    return int(hops * 1 + deg * 4 + (st[:, 2] * rb).sum() + nq * (2 * dp + 8 * 10))


def query_row_bytes(fmt, queries, dim):
    """Bytes per scored row for each query: the byte rows (dim bytes) when
    the graph keeps them and the query is integer-valued with its values and
    the rows' spanning at most the exact span (the search's per-query
    test), else the fp16 rows (2*dim at dim 128)."""
    smax = 2048
    while smax > 0 and dim * smax * smax >= 16777216:
        smax -= 1
    q = queries.astype(np.float32)
    if not fmt["byte_rows"]:
        return np.full(len(q), 2 * dim, dtype=np.int64)
    integer = (q == np.rint(q)).all(axis=1)
    span = np.maximum(q.max(axis=1), fmt["hi"]) - np.minimum(q.min(axis=1), fmt["lo"])
    return np.where(integer & (span <= smax), dim, 2 * dim).astype(np.int64)


def search_dtype(fmt, queries):
    """The arithmetic the plain search uses for these queries: u8 (v_dot4_u32_u8
    with u32 sums, exact) when the graph keeps byte rows and every query's
    values are integers in the rows' byte range [lo, lo + 255], f32 when none
    is, both names otherwise."""
    q = queries.astype(np.float32)
    if not fmt["byte_rows"]:
        return "f32"
    inb = ((q == np.rint(q)) & (q >= fmt["lo"]) & (q <= fmt["lo"] + 255)).all(axis=1)
    return "u8" if inb.all() else ("f32" if not inb.any() else "u8+f32")


def _timed(torch, fn, steps, warmup):
    """Wall ms per call and HIP-event ms per call on the current stream (the
    median over the steps: the first calls after a synchronisation can wait
    on the host's launch, which is not the kernel's time)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    out = None
    for e0, e1 in evs:
        e0.record(stream)
        out = fn()
        e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0 / steps
    ev_ms = float(np.median([a.elapsed_time(b) for a, b in evs]))
    return wall_ms, ev_ms, out


def build_algorithmic_bytes(w: dict, R: int, dp: int, row_bytes: int) -> dict:
    """Bytes a Vamana build must move, per stage, from its work counters
    (jasper_amd.last_build_work): every distinct vector a stage reads at the
    bytes of the row format it reads (row_bytes), adjacency rows at 6 B per
    edge (u32 id + bf16 distance) plus the 1-byte count, visited keys and
    reverse pairs at 8 B.
      search : per row its fp16 query row (2 dp), per pop the count byte, 4 B
               per adjacency entry, row_bytes per distinct vector scored, 8 B
               per popped key written;
      forward: per row its count (read and write) and its R reverse-pair
               slots (8 B each, written), its existing edges (6 B), its
               visited keys (8 B), row_bytes per candidate row, 6 B per edge
               written;
      group  : the reverse pairs read and written once by the sort (16 B each)
               and a 4-byte head per target;
      reverse: per target its count (read and write), its own row and head,
               its existing edges (6 B + the edge's row), its sources (the
               8-byte pair + the source's row), 6 B per edge written."""
    search = (w["search_rows"] * 2 * dp + w["search_hops"] + w["search_adjacency"] * 4
              + w["search_scored"] * row_bytes + w["search_visited"] * 8)
    forward = (w["forward_rows"] * (2 + 8 * R) + w["forward_existing"] * 6 + w["forward_visited"] * 8
               + w["forward_candidates"] * row_bytes + w["forward_selected"] * 6)
    group = w["forward_selected"] * 16 + w["reverse_targets"] * 4
    reverse = (w["reverse_targets"] * (2 + row_bytes + 4) + w["reverse_existing"] * (6 + row_bytes)
               + w["reverse_sources"] * (8 + row_bytes) + w["reverse_selected"] * 6)
    return {"search": search, "forward": forward, "group": group, "reverse": reverse,
            "total": search + forward + group + reverse}


def build_roofline(jasper_amd, base_t, R, build_s, build_total_ms, log) -> dict:
    """Roofline of the build: two more builds of the same rows (the same
    graph), one with work counting (exact per-stage counts) and one with
    per-stage HIP-event times; achieved = algorithmic bytes / time."""
    import torch
    n, dim = base_t.shape
    dp = (dim + 7) // 8 * 8
    jasper_amd.set_build_work_counting(True)
    try:
        g2 = jasper_amd.Graph.build(base_t, n_neighbors=R, distance="l2", alpha=1.2)
        torch.cuda.synchronize()
        w = jasper_amd.last_build_work()
    finally:
        jasper_amd.set_build_work_counting(False)
    fmt = g2.row_format()
    g2.free()
    os.environ["JASPER_BUILD_TIMING"] = "1"
    try:
        g3 = jasper_amd.Graph.build(base_t, n_neighbors=R, distance="l2", alpha=1.2)
        torch.cuda.synchronize()
        st = jasper_amd.last_build_stats()
    finally:
        del os.environ["JASPER_BUILD_TIMING"]
    g3.free()
    row_b = dim if fmt["byte_rows"] else 2 * dp
    b = build_algorithmic_bytes(w, R, dp, row_b)
    stage_ms = {"search": st["search_ms"], "forward": st["prune_ms"], "group": st["group_ms"],
                "reverse": st["reverse_ms"]}
    stages = {k: {"bytes": b[k], "ms": stage_ms[k],
                  "achieved_gbs": b[k] / (stage_ms[k] / 1e3) / 1e9 if stage_ms[k] > 0 else None,
                  "frac": b[k] / (stage_ms[k] / 1e3) / 1e9 / PEAK_HBM_GBS if stage_ms[k] > 0 else None}
              for k in stage_ms}
    ach = b["total"] / (build_total_ms / 1e3) / 1e9
    log(f"build roofline: {b['total'] / n / 1e3:.1f} KB per inserted vector, {b['total'] / 1e9:.2f} GB in "
        f"{build_total_ms:.1f} ms of GPU time: {ach:.0f} GB/s ({ach / PEAK_HBM_GBS:.1%}); stages " +
        ", ".join(f"{k} {v['ms']:.1f} ms {v['achieved_gbs'] or 0:.0f} GB/s" for k, v in stages.items()))
    return {"bound": "hbm", "algorithmic_bytes": b["total"], "bytes_per_vector": b["total"] / n,
            "row_bytes": row_b, "gpu_ms": build_total_ms, "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": ach / PEAK_HBM_GBS, "wall_achieved": b["total"] / build_s / 1e9, "stages": stages,
            "work": w}


def nq_sweep(args, torch, g, datasets, dev, bw, log) -> list:
    """Kernel time of one search launch against the number of queries in it
    (same graph, same beam width, queries of the same mixture from seed 1):
    one wave per query, so the counts around the resident-wave limit show
    whether a launch's last partial round of waves costs a full round."""
    counts = [int(x) for x in args.nq_sweep.split(",") if x]
    q_all = torch.from_numpy(datasets.clustered(max(counts), 128, 1)).to(dev)
    out = []
    for nq in counts:
        q = q_all[:nq].contiguous()
        _, ev_ms, _ = _timed(torch, lambda: g.search(q, k=10, beam_width=bw), 10, 2)
        out.append({"nq": nq, "kernel_ms": ev_ms, "qps": nq / (ev_ms / 1000.0),
                    "us_per_query": ev_ms * 1000.0 / nq})
        log(f"nq={nq:6d} bw={bw}: {ev_ms:.3f} ms, {nq / (ev_ms / 1000.0):,.0f} QPS")
    return out


def _line(args, metric, value, unit, ms, dtype, config, roofline, higher=True):
    return {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": higher, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config, "roofline": roofline}


def _recall(gt, ids):
    hits = 0
    for a, b in zip(gt, ids):
        hits += len(set(a.tolist()) & set(b.tolist()))
    return hits / (gt.shape[0] * gt.shape[1])


def run_directional(args, torch, jasper_amd, datasets, dev, log, use_pq=False):
    """Config 3: 1M x 96 unit vectors, IP, R=64, k_ranks=4 (u8 words),
    prerotated; LSH (or PQ with M=4) directional search over 10k queries."""
    n, nq, dim = args.n, args.nq, 96
    t0 = time.perf_counter()
    base = datasets.unit_sphere(n, dim, 0)
    queries = datasets.unit_sphere(nq, dim, 1)
    log(f"data in {time.perf_counter() - t0:.1f}s")
    base_t = torch.from_numpy(base).to(dev)
    q_t = torch.from_numpy(queries).to(dev)
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base_t, n_neighbors=64, distance="ip", alpha=1.2, build_lsh=not use_pq,
                               build_pq=use_pq, k_ranks=4, prerotate=True, lsh_samples=32768)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    log(f"directional build ({'pq' if use_pq else 'lsh'}) in {build_s:.2f}s")
    gt_ids, _ = jasper_amd.generate_groundtruth(base_t, q_t, k=10, distance="ip")
    gt = gt_ids.numpy()
    fn = g.pq_search if use_pq else g.directional_search
    sweep = [32, 48, 64, 96, 128] if args.sweep == "16,24,32,48,64,96,128,192,256" else \
        [int(x) for x in args.sweep.split(",")]
    curve, chosen = [], None
    for bw in sweep:
        ids, _ = fn(q_t, k=10, beam_width=bw)
        r = _recall(gt, ids.cpu().numpy())
        wall, ev, _ = _timed(torch, lambda: fn(q_t, k=10, beam_width=bw), 3, 1)
        curve.append({"beam_width": bw, "recall_at_10": r, "qps": nq / (wall / 1000.0)})
        log(f"bw={bw} recall={r:.4f} qps={nq / (wall / 1000.0):,.0f}")
        if chosen is None and r >= args.target_recall:
            chosen = bw
    if chosen is None:
        chosen = max(curve, key=lambda c: c["recall_at_10"])["beam_width"]
    wall, ev, _ = _timed(torch, lambda: fn(q_t, k=10, beam_width=chosen), args.steps, args.warmup)
    ids, _ = fn(q_t, k=10, beam_width=chosen)
    rec = _recall(gt, ids.cpu().numpy())
    st = g.directional_stats(q_t, k=10, beam_width=chosen, pq=use_pq).astype(np.int64)
    plain = _sweep(torch, g.exact_search, q_t, gt, (32, 64, 128, 256), log, "c3 exact search on the graph")
    dp, R = 96, 64
    visits, hops, adj = st[:, 0].sum(), st[:, 1].sum(), st[:, 2].sum()
    # per edge: PQ reads M = 4 code bytes (IP: no norm gather); LSH K*P + 2 = 6 (u8 words + bf16 m^2)
    per_edge = 4 if use_pq else 4 * 1 + 2
    alg = int(visits * 2 * dp + hops + adj * (4 + per_edge) + nq * (2 * dp + 8 * 10))
    ach = alg / (ev / 1000.0) / 1e9
    kind = "pq_search" if use_pq else "directional_search"
    res = _line(args, f"QPS @ recall@10, config 3 {kind} (1M x 96 unit vectors, IP, R=64, k_ranks=4, "
                      "prerotated)", nq / (wall / 1000.0), "queries/s", wall, "f16",
                {"workload": f"config 3: {n} x {dim} unit-norm N(0,1) fp16, IP, R=64 alpha=1.2, "
                             f"{'PQ M=4' if use_pq else 'LSH k_ranks=4 u8 words'}, prerotate, {nq} queries, k=10",
                 "beam_width": chosen, "recall_at_10": rec, "build_s": build_s,
                 "build_vectors_per_s": n / build_s, "curve": curve, "curve_exact_search": plain},
                {"bound": "hbm", "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": ach / PEAK_HBM_GBS,
                 "traffic": None if use_pq else measured_traffic(chosen, n, nq, "directional_c3_1M_pmc.md"),
                 "kernel": f"directional_kernel<IP,{'PQ' if use_pq else 'LSH'}>",
                 "kernel_ms": ev, "algorithmic_bytes_per_launch": alg,
                 "per_query": {"visits": float(st[:, 0].mean()), "hops": float(st[:, 1].mean()),
                               "adjacency_entries": float(st[:, 2].mean())}})
    print(json.dumps(res), flush=True)
    g.free()
    return 0


def run_pq(args, torch, jasper_amd, datasets, dev, log):
    return run_directional(args, torch, jasper_amd, datasets, dev, log, use_pq=True)


def run_bruteforce(args, torch, jasper_amd, datasets, dev, log):
    """Exact k-NN of config 2's 10k queries over its 1M x 128 base."""
    base = torch.from_numpy(datasets.clustered(args.n, 128, 0)).to(dev)
    q = torch.from_numpy(datasets.clustered(args.nq, 128, 1)).to(dev)
    wall, ev, _ = _timed(torch, lambda: jasper_amd.bruteforce_knn(base, q, 10, "l2"), args.steps, args.warmup)
    flop = 2.0 * args.nq * args.n * 128
    tf = flop / (ev / 1000.0) / 1e12
    res = _line(args, "exact k-NN TFLOP/s (matrix cores), config 2", tf, "TFLOP/s", wall, "f16",
                {"workload": f"config 2 ground truth: {args.nq} queries x {args.n} x 128 fp16, L2, k=10",
                 "queries_per_s": args.nq / (wall / 1000.0)},
                {"bound": "mfma", "achieved": tf, "peak": 2500.0, "unit": "TFLOP/s", "frac": tf / 2500.0,
                 "traffic": None, "kernel": "bruteforce_knn (sample scan + bf_filter_kernel + bf_select_kernel)", "kernel_ms": ev,
                 "algorithmic_flop_per_launch": flop})
    print(json.dumps(res), flush=True)
    return 0


PEAK_MFMA_F16_TFLOPS = 2500.0


def run_rotate(args, torch, jasper_amd, datasets, dev, log):
    """Prerotation of 1M fp16 rows (the construct-time GEMM): d = 128 (config
    2's rows; HBM-bound, 64 flop/byte) or --rotate-dim 960 (config 4's rows;
    480 flop/byte, above the MI355X ridge of about 310: matrix-core bound)."""
    d = args.rotate_dim
    rows = datasets.sparse_abs(args.n, d, 0) if d == 960 else datasets.clustered(args.n, d, 0)
    x = torch.from_numpy(rows).to(dev)
    wall, ev, _ = _timed(torch, lambda: jasper_amd.rotate(x, 42), args.steps, args.warmup)
    nbytes = 4.0 * args.n * d + 2 * d * d
    flop = 2.0 * args.n * d * d
    gbs = nbytes / (ev / 1000.0) / 1e9
    tf = flop / (ev / 1000.0) / 1e12
    kernel = "rotate_tile_kernel" if d <= 192 else "rotate_gemm_kernel"
    if flop / nbytes < PEAK_MFMA_F16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        roof = {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                "traffic": None, "kernel": kernel, "kernel_ms": ev, "algorithmic_bytes_per_launch": nbytes}
        res = _line(args, f"prerotation GB/s, {args.n} x {d} fp16", gbs, "GB/s", wall, "f16",
                    {"workload": f"{args.n} x {d} fp16 rows times a {d} x {d} fp16 rotation, fp32 accumulation",
                     "tflops": tf}, roof)
    else:
        roof = {"bound": "mfma", "achieved": tf, "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": tf / PEAK_MFMA_F16_TFLOPS, "traffic": None, "kernel": kernel, "kernel_ms": ev,
                "algorithmic_flop_per_launch": flop}
        res = _line(args, f"prerotation TFLOP/s, {args.n} x {d} fp16", tf, "TFLOP/s", wall, "f16",
                    {"workload": f"{args.n} x {d} fp16 rows (config 4's generator) times a {d} x {d} fp16 rotation, "
                                 "fp32 accumulation", "hbm_gbs": gbs}, roof)
    log(f"rotate {args.n} x {d}: {ev:.3f} ms, {tf:.1f} TFLOP/s, {gbs:.0f} GB/s")
    print(json.dumps(res), flush=True)
    return 0


def run_rabitq(args, torch, jasper_amd, datasets, dev, log):
    """One-bit RaBitQ codes of 1M x 128 fp16 rows (fp32 matrix cores)."""
    x = torch.from_numpy(datasets.clustered(args.n, 128, 0)).to(dev)
    rot = torch.from_numpy(jasper_amd.rotation_matrix(128, 42)).to(dev)
    wall, ev, _ = _timed(torch, lambda: jasper_amd.rabitq_quantize(x, rotation=rot), args.steps, args.warmup)
    flop = 2.0 * args.n * 128 * 128
    tf = flop / (ev / 1000.0) / 1e12
    res = _line(args, "RaBitQ one-bit quantize vectors/s, 1M x 128 fp16", args.n / (ev / 1000.0), "vectors/s",
                wall, "f32",
                {"workload": f"{args.n} x 128 fp16 rows, rotation 128 x 128 fp32, zero centroid, L2",
                 "hbm_gbs": args.n * (256 + 24) / (ev / 1000.0) / 1e9},
                {"bound": "mfma", "achieved": tf, "peak": 157.3, "unit": "TFLOP/s", "frac": tf / 157.3,
                 "traffic": None, "kernel": "rabitq_kernel<8,true>", "kernel_ms": ev,
                 "algorithmic_flop_per_launch": flop})
    print(json.dumps(res), flush=True)
    return 0


def _sweep(torch, fn, queries, gt, bws, log, tag, **kw):
    nq = queries.size(0)
    out = []
    for bw in bws:
        run = lambda bw=bw: fn(queries, k=10, beam_width=bw, **kw)
        ids, _ = run()
        r = _recall(gt, ids.cpu().numpy())
        wall, _, _ = _timed(torch, run, 3, 1)
        out.append({"beam_width": bw, "recall_at_10": r, "qps": nq / (wall / 1000.0), **kw})
        log(f"{tag} bw={bw} recall={r:.4f} qps={nq / (wall / 1000.0):,.0f}")
    return out


def run_c5(args, torch, jasper_amd, datasets, dev, log):
    """Config 5: 100M x 128 clustered integer vectors (10,000 clusters)
    generated in HBM, R=64, alpha=1.2, prerotated, RaBitQ one-bit codes for
    the build's distance estimation (build_search="rabitq": the
    construction's search pops by the RaBitQ estimate), LSH k_ranks=16 (u8
    words), 32768 samples; 10k queries, k=10, directional search, QPS at
    recall@10 >= 0.9 (swept up to the API's beam-width limit, 1983). Beside
    it: the exact (reference) construction of the same rows, and the exact
    beam search on both graphs (what each graph allows without an
    estimator)."""
    n, nq, dim = args.c5_n, args.nq, 128
    t0 = time.perf_counter()
    base = datasets.clustered_device(n, dim, 0, dev)
    queries = datasets.clustered_device(nq, dim, 1, dev)
    torch.cuda.synchronize()
    log(f"c5 data {n} x {dim} generated in HBM in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    gt_ids, _ = jasper_amd.bruteforce_knn(base, queries, 10, "l2")
    gt = gt_ids.cpu().numpy()
    log(f"c5 ground truth {time.perf_counter() - t0:.1f}s")
    cfg = jasper_amd._resolve_directional_config(jasper_amd.DataType.FLOAT16, 64, jasper_amd.DistanceFunc.L2,
                                                  16, dim)
    stream = jasper_amd._stream_ptr(dev)
    budget = jasper_amd.parse_storage_size("10GB")
    exact_bws = (64, 128, 256, 384, 512)

    # config 5 as configured: RaBitQ build search, then the LSH artifacts
    t0 = time.perf_counter()
    handle = jasper_amd._agnostic("jasperx_construct_directional_ex")(
        cfg.encode(), jasper_amd._tensor_ptr(base), n, dim, 1.2, budget, False, True, 42, 1, stream)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    bst = jasper_amd.last_build_stats()
    log(f"c5 construct with the RaBitQ build search (prerotation + codes + Vamana) {build_s:.1f}s = "
        f"{n / build_s:,.0f} vec/s, batches={int(bst['batches'])} max_batch={int(bst['max_batch'])}")
    t0 = time.perf_counter()
    jasper_amd._op("build_lsh", cfg)(handle, 32768, 42)
    torch.cuda.synchronize()
    lsh_s = time.perf_counter() - t0
    log(f"c5 LSH artifacts {lsh_s:.1f}s")
    g = jasper_amd.Graph(handle, cfg, jasper_amd.DataType.FLOAT16, jasper_amd.DistanceFunc.L2, 64, dim,
                         is_directional=True, k_ranks=16, has_lsh=True, has_pq=False, prerotate=True,
                         prerotate_seed=42, has_rabitq=True)
    free, total = torch.cuda.mem_get_info()
    exact_rq = _sweep(torch, g.exact_search, queries, gt, exact_bws, log, "c5 rabitq-built graph, exact search")
    curve, chosen = [], None
    for unique, bws in ((False, [32, 64, 128, 256, 512, 1024]),
                        (True, [32, 64, 128, 256, 512, 768, 1024, 1536, 1983])):
        for c in _sweep(torch, g.directional_search, queries, gt, bws, log, f"c5 LSH unique={unique}",
                        unique=unique):
            curve.append(c)
            if c["recall_at_10"] >= 0.9 and (chosen is None or c["qps"] > chosen["qps"]):
                chosen = c
    rq_curve = _sweep(torch, g.rabitq_search, queries, gt, [64, 256, 1024], log, "c5 RaBitQ unique=True",
                      unique=True)
    if chosen is None:
        chosen = max(curve, key=lambda c: c["recall_at_10"])
    bw, unique = chosen["beam_width"], chosen["unique"]
    wall, ev, _ = _timed(torch, lambda: g.directional_search(queries, k=10, beam_width=bw, unique=unique),
                         args.steps, args.warmup)
    ids, _ = g.directional_search(queries, k=10, beam_width=bw, unique=unique)
    rec = _recall(gt, ids.cpu().numpy())
    st = g.directional_stats(queries, k=10, beam_width=bw, unique=unique).astype(np.int64)
    visits, hops, adj = st[:, 0].sum(), st[:, 1].sum(), st[:, 2].sum()
    alg = int(visits * 2 * dim + hops + adj * (4 + 16 + 2) + nq * (2 * dim + 80))
    ach = alg / (ev / 1000.0) / 1e9
    log(f"c5 LSH bw={bw} unique={unique}: recall {rec:.4f}, {nq / (wall / 1000.0):,.0f} QPS, kernel {ev:.3f} ms, "
        f"{ach:.0f} GB/s")
    g.free()

    # the exact (reference) construction of the same rows
    t0 = time.perf_counter()
    handle = jasper_amd._op("construct_directional", cfg)(
        jasper_amd._tensor_ptr(base), n, dim, 1.2, budget, False, True, 42, stream)
    torch.cuda.synchronize()
    exact_build_s = time.perf_counter() - t0
    log(f"c5 exact construct (prerotation + Vamana) {exact_build_s:.1f}s = {n / exact_build_s:,.0f} vec/s")
    ge = jasper_amd.Graph(handle, cfg, jasper_amd.DataType.FLOAT16, jasper_amd.DistanceFunc.L2, 64, dim,
                          is_directional=True, k_ranks=16, prerotate=True, prerotate_seed=42)
    exact_ex = _sweep(torch, ge.exact_search, queries, gt, exact_bws, log, "c5 exact-built graph, exact search")
    ge.free()
    res = _line(args, "config 5: build vectors/s (100M x 128 in HBM) and QPS @ recall@10>=0.9, directional LSH",
                nq / (wall / 1000.0), "queries/s", wall, "f16",
                {"workload": f"config 5: {n} x {dim} clustered integer fp16 (10,000 clusters, generated in HBM), "
                             "R=64 alpha=1.2, prerotate, RaBitQ build search, LSH k_ranks=16 u8 words, "
                             f"32768 samples, {nq} queries, k=10",
                 "build_vectors_per_s": n / build_s, "build_s": build_s, "lsh_s": lsh_s,
                 "build_max_batch": int(bst["max_batch"]),
                 "exact_build_vectors_per_s": n / exact_build_s, "exact_build_s": exact_build_s,
                 "beam_width": bw, "unique": unique, "recall_at_10": rec, "target_recall": 0.9,
                 "curve": curve, "curve_rabitq_search": rq_curve, "curve_exact_search_rabitq_built": exact_rq,
                 "curve_exact_search_exact_built": exact_ex, "hbm_used_gb": (total - free) / 1e9},
                {"bound": "hbm", "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": ach / PEAK_HBM_GBS,
                 "traffic": None, "kernel": "directional_kernel<L2,LSH>", "kernel_ms": ev,
                 "algorithmic_bytes_per_launch": alg,
                 "per_query": {"visits": float(st[:, 0].mean()), "hops": float(st[:, 1].mean()),
                               "adjacency_entries": float(st[:, 2].mean())}})
    print(json.dumps(res), flush=True)
    return 0


def run_c4(args, torch, jasper_amd, datasets, dev, log):
    """Config 4: 1M x 960 non-negative sparse vectors (|N(0,1)| * 0.05, 192
    dims zeroed per row) generated in HBM, L2, R=64, alpha=1.2, PQ with
    8-bit codebooks and one subspace per 8 dims (M = 120, --c4-m), prerotated
    (the Python default with build_pq); 1,000 queries, k=10, pq_search at
    bw=64. Also: the same graph's PQ retrained at M = 16 (the largest the
    reference's configs offer), and the exact beam search on the graph (what
    it allows without an estimator)."""
    n, nq, dim = args.n, min(args.nq, 1000), 960
    M = args.c4_m
    base = datasets.sparse_abs_device(n, dim, 0, dev)
    queries = datasets.sparse_abs_device(nq, dim, 1, dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base, n_neighbors=64, distance="l2", alpha=1.2, build_pq=True, k_ranks=16,
                               prerotate=True, pq_m=M)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    bst = jasper_amd.last_build_stats()
    log(f"c4 build (prerotation + Vamana + PQ M={M}) {build_s:.1f}s = {n / build_s:,.0f} vec/s")
    t0 = time.perf_counter()
    gt_ids, _ = jasper_amd.generate_groundtruth(base, queries, k=10, distance="l2")
    gt = gt_ids.numpy()
    log(f"c4 ground truth {time.perf_counter() - t0:.1f}s")

    def sweep(tag, bws):
        out = []
        for unique in (False, True):
            for bw in bws:
                run = lambda bw=bw, unique=unique: g.pq_search(queries, k=10, beam_width=bw, unique=unique)
                ids, _ = run()
                r = _recall(gt, ids.cpu().numpy())
                wall, ev, _ = _timed(torch, run, 3, 1)
                out.append({"unique": unique, "beam_width": bw, "recall_at_10": r, "qps": nq / (wall / 1000.0)})
                log(f"c4 {tag} unique={unique} bw={bw} recall={r:.4f} qps={nq / (wall / 1000.0):,.0f}")
        return out

    curve = sweep(f"M={M}", (32, 64, 128, 256))
    # the configured point: beam width 64, reference traversal
    bw = 64
    wall, ev, _ = _timed(torch, lambda: g.pq_search(queries, k=10, beam_width=bw), args.steps, args.warmup)
    ids, _ = g.pq_search(queries, k=10, beam_width=bw)
    rec = _recall(gt, ids.cpu().numpy())
    st = g.directional_stats(queries, k=10, beam_width=bw, pq=True).astype(np.int64)
    visits, hops, adj = st[:, 0].sum(), st[:, 1].sum(), st[:, 2].sum()
    # per hop: count byte, vector 2*dp; per edge: id 4, M code bytes, L2 norm 4
    alg = int(visits * 2 * dim + hops + adj * (4 + M + 4) + nq * (2 * dim + 80))
    ach = alg / (ev / 1000.0) / 1e9
    log(f"c4 M={M} bw={bw}: {wall:.3f} ms/step (events {ev:.3f} ms), {nq / (wall / 1000.0):,.0f} QPS, "
        f"recall {rec:.4f}, {alg / nq / 1e3:.1f} KB/query, {ach:.0f} GB/s")
    m16 = None
    if M != 16:
        t0 = time.perf_counter()
        jasper_amd._agnostic("jasperx_build_pq_m")(g.handle, 16, 40000, 12, 123)
        torch.cuda.synchronize()
        log(f"c4 PQ retrained at M=16 in {time.perf_counter() - t0:.1f}s")
        m16 = sweep("M=16", (64, 256))
    plain = _sweep(torch, g.exact_search, queries, gt, (32, 64, 128, 256), log, "c4 exact search on the graph")
    res = _line(args, "config 4: QPS @ bw=64 and build vectors/s, PQ-ADC directional search (1M x 960, L2)",
                nq / (wall / 1000.0), "queries/s", wall, "f16",
                {"workload": f"config 4: {n} x {dim} |N(0,1)|*0.05 with 192 zero dims (generated in HBM), L2, "
                             f"R=64 alpha=1.2, PQ M={M} dsub={dim // M}, prerotate, {nq} queries, k=10, bw=64",
                 "build_vectors_per_s": n / build_s, "build_s": build_s, "build_max_batch": int(bst["max_batch"]),
                 "beam_width": bw, "recall_at_10": rec, "curve": curve, "curve_pq_m16": m16,
                 "curve_exact_search": plain},
                {"bound": "hbm", "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": ach / PEAK_HBM_GBS,
                 "traffic": None, "kernel": f"directional_kernel<L2,PQ{' wide' if M > 16 else ''}>",
                 "kernel_ms": ev, "algorithmic_bytes_per_launch": alg,
                 "lut_centroid_bytes_per_query": M * 256 * (dim // M) * 4,
                 "per_query": {"visits": float(st[:, 0].mean()), "hops": float(st[:, 1].mean()),
                               "adjacency_entries": float(st[:, 2].mean())}})
    print(json.dumps(res), flush=True)
    g.free()
    return 0


def run_updates(args, torch, jasper_amd, datasets, dev, log):
    """Live updates on config 2: build 1M x 128, soft-delete 10% of the ids,
    consolidate, append 100k new vectors of the same mixture. Each operation
    is timed once on the GPU graph (they mutate it); recall@10 of the 10k
    queries at bw = 48 is measured against exact ground truth over the live
    vectors after each step, and viol counts deleted ids in the results (the
    reference's CI gate, scripts/ci/bench.py:132-134)."""
    n, nq, dim, bw = args.n, args.nq, 128, 48
    n_del, n_add = n // 10, n // 10
    base = torch.from_numpy(datasets.clustered(n, dim, 0)).to(dev)
    extra = torch.from_numpy(datasets.clustered(n_add, dim, 2)).to(dev)
    q = torch.from_numpy(datasets.clustered(nq, dim, 1)).to(dev)
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base, n_neighbors=64, distance="l2", alpha=1.2)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    rng = np.random.default_rng(7)
    dels = torch.from_numpy(np.sort(rng.choice(n, size=n_del, replace=False)).astype(np.int32))

    def live_recall(live_rows, live_ids):
        gt, _ = jasper_amd.bruteforce_knn(live_rows, q, 10, "l2")
        gt = live_ids[gt.long()].cpu().numpy()
        ids, _ = g.search(q, k=10, beam_width=bw)
        torch.cuda.synchronize()
        ids = ids.cpu().numpy()
        return _recall(gt, ids), ids

    def once(fn):
        torch.cuda.synchronize()
        t = time.perf_counter()
        out = fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) * 1000.0, out

    all_ids = torch.arange(n, device=dev)
    r0, _ = live_recall(base, all_ids)
    # self-recall of built vectors, for comparison with the appended ones
    out, _ = g.search(base[:nq].contiguous(), k=10, beam_width=64)
    out = out.cpu().numpy()
    base_self = float(np.mean([i in out[i] for i in range(nq)]))
    del_ms, _ = once(lambda: g.mark_deleted(dels))
    keep = torch.ones(n, dtype=torch.bool, device=dev)
    keep[dels.long().to(dev)] = False
    r1, ids1 = live_recall(base[keep].contiguous(), all_ids[keep])
    dead = set(dels.tolist())
    viol = int(sum(1 for x in ids1.ravel().tolist() if x in dead))
    cons_ms, _ = once(lambda: g.consolidate(1.2))
    r2, ids2 = live_recall(base[keep].contiguous(), all_ids[keep])
    viol += int(sum(1 for x in ids2.ravel().tolist() if x in dead))
    add_ms, new_ids = once(lambda: g.append(extra, 1.2))
    rows = torch.cat([base[keep], extra]).contiguous()
    labels = torch.cat([all_ids[keep], new_ids.to(dev).long()])
    r3, _ = live_recall(rows, labels)
    out, _ = g.search(extra[:nq], k=10, beam_width=64)
    out = out.cpu().numpy()
    nid = new_ids.numpy()
    self_recall = float(np.mean([nid[i] in out[i] for i in range(min(nq, n_add))]))
    g.free()
    # The reference's append gate (cmd/test_append.cu:66-121): construct on the
    # n rows, append the n_add new ones, search all appended rows themselves
    # (limit 2 * bw) and count those found in their own top 10. Beside it the
    # same rows searched in a graph built on all n + n_add rows at once: the
    # gap between the two is what the append costs, the rest is the data.
    def self_recall_of(graph, rows, want, bws=(64, 128)):
        res = {}
        for b in bws:
            o, _ = graph.search(rows, k=10, beam_width=b)
            o = o.cpu().numpy()
            res[b] = float(np.mean((o == want[:, None]).any(axis=1)))
        return res
    want = np.arange(n, n + n_add)
    ga = jasper_amd.Graph.build(base, n_neighbors=64, distance="l2", alpha=1.2)
    ga_ids = ga.append(extra, 1.2).numpy()
    assert np.array_equal(ga_ids, want)
    gate_append = self_recall_of(ga, extra, want)
    ga.free()
    gb = jasper_amd.Graph.build(torch.cat([base, extra]).contiguous(), n_neighbors=64, distance="l2", alpha=1.2)
    gate_built = self_recall_of(gb, extra, want)
    gb.free()
    log(f"reference append gate: appended rows' self-recall@10 at bw 64 / 128: {gate_append[64]:.4f} / "
        f"{gate_append[128]:.4f}; the same rows built in from the start: {gate_built[64]:.4f} / {gate_built[128]:.4f}")
    log(f"build {build_s:.2f}s; recall@10 bw={bw}: {r0:.4f} -> after deleting {n_del}: {r1:.4f} "
        f"(mark_deleted {del_ms:.1f} ms, viol={viol}) -> consolidate {cons_ms:.1f} ms: {r2:.4f} -> "
        f"append {n_add} in {add_ms:.1f} ms ({n_add / (add_ms / 1000.0):,.0f} vec/s): {r3:.4f}; "
        f"appended self-recall@10 {self_recall:.4f} (built vectors: {base_self:.4f})")
    res = _line(args, "live updates, config 2: append vectors/s (100k into 1M x 128)", n_add / (add_ms / 1000.0),
                "vectors/s", add_ms, "f32",
                {"workload": f"config 2 graph ({n} x 128, R=64); mark_deleted {n_del} random ids, consolidate "
                             f"(alpha 1.2), append {n_add} vectors of the same mixture (seed 2); recall@10 of "
                             f"{nq} queries at bw {bw} against exact ground truth over the live vectors",
                 "build_s": build_s, "mark_deleted_ms": del_ms, "consolidate_ms": cons_ms, "append_ms": add_ms,
                 "recall_built": r0, "recall_after_delete": r1, "recall_after_consolidate": r2,
                 "recall_after_append": r3, "viol": viol, "appended_self_recall_at_10": self_recall,
                 "built_self_recall_at_10": base_self,
                 "append_gate": {"protocol": f"build {n}, append {n_add}, search the {n_add} appended rows "
                                             "(k 10, limit 2 bw) as cmd/test_append.cu does",
                                 "self_recall_at_10_bw64": gate_append[64], "self_recall_at_10_bw128": gate_append[128],
                                 "same_rows_built_in_bw64": gate_built[64],
                                 "same_rows_built_in_bw128": gate_built[128]}},
                None)
    res["steps"], res["warmup"] = 1, 0
    print(json.dumps(res), flush=True)
    return 0


def run_scale(args, torch, jasper_amd, datasets, dev, log):
    """The partitioned build (construct_scale.cuh, cmd/create_scale_index.cu)
    on config 2 (1M x 128 clustered, R=64, L2, budget 10 GB): --scale-parts
    partitions built on their own, every pair merged. Timed once per
    partition count; recall@10 of the 10k queries at a few beam widths beside
    the plain build's, on the same data."""
    n, nq, dim = args.n, args.nq, 128
    base = torch.from_numpy(datasets.clustered(n, dim, 0)).to(dev)
    q = torch.from_numpy(datasets.clustered(nq, dim, 1)).to(dev)
    gt, _ = jasper_amd.bruteforce_knn(base, q, 10, "l2")
    gt = gt.cpu().numpy()
    bws = (32, 44, 64, 128)

    def recalls(g):
        out = {}
        for b in bws:
            ids, _ = g.search(q, k=10, beam_width=b)
            torch.cuda.synchronize()
            out[b] = _recall(gt, ids.cpu().numpy())
        return out

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base, n_neighbors=64, distance="l2", alpha=1.2)
    torch.cuda.synchronize()
    plain_s = time.perf_counter() - t0
    plain_r = recalls(g)
    g.free()
    log(f"plain build {plain_s:.2f}s, recall@10 {plain_r}")
    runs = []
    for P in [int(x) for x in args.scale_parts.split(",")]:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g = jasper_amd.Graph.build_scale(base, n_neighbors=64, distance="l2", alpha=1.2, n_parts=P,
                                         workspace_budget="10GB")
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        st = jasper_amd.last_scale_stats()
        r = recalls(g)
        g.free()
        runs.append({"n_parts": P, "build_s": wall, "partition_s": st["partition_ms"] / 1e3,
                     "merge_s": st["merge_ms"] / 1e3, "merges": int(st["merges"]),
                     "merge_batches": int(st["merge_batches"]), "part_batch": int(st["part_batch"]),
                     "merge_batch": int(st["merge_batch"]), "recall_at_10": {str(b): v for b, v in r.items()}})
        log(f"n_parts={P}: {wall:.2f}s (partitions {st['partition_ms'] / 1e3:.2f}s, {int(st['merges'])} merges "
            f"{st['merge_ms'] / 1e3:.2f}s), recall@10 {r}")
    head = runs[0]
    res = _line(args, f"partitioned build, config 2: vectors/s ({head['n_parts']} partitions)", n / head["build_s"],
                "vectors/s", head["build_s"] * 1000.0, "f32",
                {"workload": f"config 2 ({n} x 128 clustered, R=64, L2, alpha 1.2), budget 10 GB: partitions "
                             f"built on their own (batches min(budget batch, n / n_parts / 20)), every pair "
                             f"merged (batches of the budget batch); recall@10 of {nq} queries",
                 "plain_build_s": plain_s, "plain_recall_at_10": {str(b): v for b, v in plain_r.items()},
                 "runs": runs}, None)
    res["steps"], res["warmup"] = 1, 0
    print(json.dumps(res), flush=True)
    return 0


def run_diskann(args, torch, jasper_amd, datasets, dev, log):
    """The DiskANN build (construct_diskann.cuh, cmd/create_diskann_index.cu)
    on config 2 (1M x 128 clustered, L2, budget 10 GB): cross-polytope LSH
    shards with 2 copies, shards built at R_int = 32, merged to R = 64 (the
    reference's f16_r32_64_l2) and to R = 32; timed once each, recall@10 of
    the 10k queries beside the plain build's."""
    n, nq, dim = args.n, args.nq, 128
    base = torch.from_numpy(datasets.clustered(n, dim, 0)).to(dev)
    q = torch.from_numpy(datasets.clustered(nq, dim, 1)).to(dev)
    gt, _ = jasper_amd.bruteforce_knn(base, q, 10, "l2")
    gt = gt.cpu().numpy()
    bws = (32, 44, 64, 128)

    def recalls(g):
        out = {}
        for b in bws:
            ids, _ = g.search(q, k=10, beam_width=b)
            torch.cuda.synchronize()
            out[b] = _recall(gt, ids.cpu().numpy())
        return out

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base, n_neighbors=64, distance="l2", alpha=1.2)
    torch.cuda.synchronize()
    plain_s = time.perf_counter() - t0
    plain_r = recalls(g)
    g.free()
    log(f"plain build (R 64) {plain_s:.2f}s, recall@10 {plain_r}")
    runs = []
    for R_fin in (64, 32):
        for P in [int(x) for x in args.diskann_parts.split(",")]:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            g = jasper_amd.Graph.build_diskann(base, n_neighbors=R_fin, r_int=32, distance="l2", alpha=1.2,
                                               n_parts=P, n_dup=2, workspace_budget="10GB")
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            st = jasper_amd.last_diskann_stats()
            r = recalls(g)
            g.free()
            runs.append({"R_fin": R_fin, "n_parts": P, "build_s": wall, "assign_s": st["assign_ms"] / 1e3,
                         "shard_builds_s": st["build_ms"] / 1e3, "merges_s": st["merge_ms"] / 1e3,
                         "shards": int(st["shards"]), "max_shard": int(st["max_shard"]),
                         "recall_at_10": {str(b): v for b, v in r.items()}})
            log(f"R_fin={R_fin} n_parts={P}: {wall:.2f}s (assign {st['assign_ms']:.1f} ms, shard builds "
                f"{st['build_ms'] / 1e3:.2f}s, merges {st['merge_ms']:.1f} ms, largest shard "
                f"{int(st['max_shard'])}), recall@10 {r}")
    head = runs[0]
    res = _line(args, f"DiskANN build, config 2: vectors/s (R_int 32 -> R 64, {head['n_parts']} shards, 2 copies)",
                n / head["build_s"], "vectors/s", head["build_s"] * 1000.0, "f32",
                {"workload": f"config 2 ({n} x 128 clustered, L2, alpha 1.2), budget 10 GB: cross-polytope LSH "
                             f"shards (seed 42, 2 copies), shards built at R_int 32 (batches min(budget batch, "
                             f"n / n_parts / 20)), merged by stored distance; recall@10 of {nq} queries",
                 "plain_build_s": plain_s, "plain_recall_at_10": {str(b): v for b, v in plain_r.items()},
                 "runs": runs}, None)
    res["steps"], res["warmup"] = 1, 0
    print(json.dumps(res), flush=True)
    return 0


def run_c5plain(args, torch, jasper_amd, datasets, dev, log):
    """Config 5's 100M x 128 clustered integer rows without prerotation:
    the plain construction (the exact build search) and the plain beam
    search on that graph, QPS at the first swept beam width with recall@10
    >= 0.9. The rows are integers in [0, 218], so the graph keeps byte rows
    and both the build's searches and the queries read them. The roofline's
    algorithmic bytes come from the exact work counters of a 256-query
    sample (the counters' per-query seen bitmap is n / 8 bytes), scaled to
    the batch."""
    n, nq, dim = args.c5_n, args.nq, 128
    base = datasets.clustered_device(n, dim, 0, dev)
    queries = datasets.clustered_device(nq, dim, 1, dev)
    torch.cuda.synchronize()
    gt_ids, _ = jasper_amd.bruteforce_knn(base, queries, 10, "l2")
    gt = gt_ids.cpu().numpy()
    t0 = time.perf_counter()
    g = jasper_amd.Graph.build(base, n_neighbors=64, distance="l2", alpha=1.2)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    bst = jasper_amd.last_build_stats()
    fmt = g.row_format()
    log(f"c5 plain build {build_s:.1f}s = {n / build_s:,.0f} vec/s, batches={int(bst['batches'])}, rows {fmt}")
    curve = _sweep(torch, g.search, queries, gt, (64, 128, 256, 384, 512), log, "c5 plain graph search")
    chosen = next((c for c in curve if c["recall_at_10"] >= 0.9), curve[-1])
    bw = chosen["beam_width"]
    wall, ev, _ = _timed(torch, lambda: g.search(queries, k=10, beam_width=bw), args.steps, args.warmup)
    sample = queries[:256].contiguous()
    st = g.search_stats(sample, k=10, beam_width=bw).astype(np.int64)
    rows_b = query_row_bytes(fmt, sample.cpu().numpy(), dim)
    alg = algorithmic_bytes(st, dim, len(st), rows_b) * nq / len(st)
    gbs = alg / (ev / 1000.0) / 1e9
    res = _line(args, "QPS @ recall@10>=0.9, config 5 data (100M x 128) plain graph", nq / (wall / 1000.0),
                "queries/s", wall, search_dtype(fmt, queries.cpu().numpy()),
                {"workload": f"{n} x {dim} clustered integer fp16 (10,000 clusters), not prerotated, R=64 "
                             f"alpha=1.2, plain construction and beam search, {nq} queries, k=10",
                 "beam_width": bw, "recall_at_10": chosen["recall_at_10"], "build_s": build_s,
                 "build_vectors_per_s": n / build_s, "byte_rows": fmt["byte_rows"], "curve": curve},
                {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                 "traffic": None, "kernel": "beam_search_kernel<4,0,false,true>" if fmt["byte_rows"]
                 else "beam_search_kernel<4,0,false>", "kernel_ms": ev, "algorithmic_bytes_per_launch": alg,
                 "per_query": {"hops": float(st[:, 0].mean()), "adjacency_entries": float(st[:, 1].mean()),
                               "vectors_scored": float(st[:, 2].mean())},
                 "notes": "algorithmic bytes from a 256-query sample of the exact work counters"})
    print(json.dumps(res), flush=True)
    g.free()
    return 0


OTHER_PATHS = {"c4": run_c4, "c5": run_c5, "c5plain": run_c5plain, "directional": run_directional, "pq": run_pq, "bruteforce": run_bruteforce,
               "rotate": run_rotate, "rabitq": run_rabitq, "updates": run_updates, "scale": run_scale,
               "diskann": run_diskann}


if __name__ == "__main__":
    sys.exit(main())
