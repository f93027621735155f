#!/usr/bin/env python3
"""Benchmark of the PQ search hot path on one MI355X: per-query LUT build, fused ADC scan and top-k.

A step is one search of the whole query batch against the whole database (LUT build + fused scan + final
merge), with queries and results resident in HBM (the device entry point vk_search_device). The default workload
is the headline configuration: 1M vectors of d=128 from a 1000-component Gaussian mixture (sigma 0.3), PQ m=16
trained by 25 k-means iterations on the first 50k vectors, nq=1000 queries from the same mixture, k=10, fp32 LUTs.

Prints ONE JSON line on stdout (progress goes to stderr):
  value        queries/s over the timed steps (wall clock, device synchronised on both sides)
  roofline     the fused scan kernel's lookups/s (HIP events on its stream) against MI355X's lookup peak: 64 per
               CU-cycle, where the LDS returns 256 B/clk/CU (a 4-byte fp32 entry per lookup) and the VALU issues 64
               lane-ops/clk/CU (one add per lookup); checked live by a conflict-free LDS read microbenchmark, with
               the random-lookup floors beside it; plus its algorithmic HBM bytes against the 8 TB/s peak
  cpu_baseline the reference's CPU adc_search (compiled from its sources into oracle/_ref) or, if that library is
               absent, the oracle port, on a bounded sample of the same queries on this host's cores
  parity       the GPU results for the CPU sample compared with the CPU results (ids and distance bits)

--variant v9 runs the fp16-table search (FusedWarpF16): its parity is against the CPU restatement of the fp16
arithmetic, and `recall_delta` reports how much of the fp32 reference's top-k it returns.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config B|A|C32|C64|D|D1|E] [--queries-per-block Q]
                       [--ilp U] [--variant v8|v9|...] [--no-cpu] [--no-recall]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "queries/s @1M vecs m=16 k=10 nq=1000; % of LDS-lookup/HBM roofline"
A100_V8_QPS = 86216.0  # reference v8 at 1M x d128, PQ16, nq=1000, k=10 (results/final/scaling.csv:11)
HBM_PEAK_GBS = 8000.0   # MI355X published HBM3E bandwidth

# name -> (n, d, m, nq, k, data, train rows, iters, description)
CONFIGS = {
    "A": (100_000, 128, 16, 100, 10, "mixture", 50_000, 25, "pq-scan 100k x d128, m16, nq=100, k=10"),
    "B": (1_000_000, 128, 16, 1000, 10, "mixture", 50_000, 25, "pq-scan 1M x d128, m16 (16 B codes), nq=1000, k=10"),
    "C32": (1_000_000, 128, 32, 1000, 100, "mixture", 50_000, 25, "pq-scan 1M x d128, m32, nq=1000, k=100"),
    "C64": (1_000_000, 128, 64, 1000, 100, "mixture", 50_000, 25, "pq-scan 1M x d128, m64, nq=1000, k=100"),
    "D": (10_000_000, 128, 16, 1000, 10, "mixture", 50_000, 25, "pq-scan 10M x d128, m16, nq=1000, k=10"),
    "D1": (10_000_000, 128, 16, 1, 10, "mixture", 50_000, 25, "pq-scan 10M x d128, m16, nq=1, k=10 (latency)"),
    "E": (100_000_000, 128, 16, 1000, 10, "codes", 0, 0, "pq-scan 100M direct uniform codes, m16, nq=1000, k=10"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_workload(cfg):
    """Seeded synthetic data of the configuration: (centroids, codes, queries, base or None)."""
    from veckern_amd import host
    n, d, m, nq, k, data, train, iters, _ = CONFIGS[cfg]
    t0 = time.time()
    if data == "mixture":
        base = host.gaussian_mixture(d, 1000, 0.3, 1, 0, n)
        queries = host.gaussian_mixture(d, 1000, 0.3, 1, 1 << 40, nq)  # a disjoint row range of the same mixture
        centroids = host.pq_train(base[:min(train, n)], m, iters, seed=1)
        codes = host.pq_encode(centroids, base)
    else:  # codes drawn directly: uniform bytes, N(0, 1) codebooks and queries
        base = None
        codes = host.uniform_codes(0, n, m, 1)
        centroids = host.normal_values(1, host.STREAM_CODEBOOK, 0, m * 256 * (d // m)).reshape(m, 256, d // m)
        queries = host.normal_values(1, host.STREAM_QUERIES, 0, nq * d).reshape(nq, d)
    log(f"[bench] workload {cfg}: n={n} d={d} m={m} nq={nq} k={k} built in {time.time() - t0:.1f} s")
    return centroids, codes, queries, base


def microbench():
    """Measured rates: LDS random-lookup floors per table width, the conflict-free LDS read rate, HBM streaming."""
    import veckern_amd as vk
    vk.library()
    lib = ctypes.CDLL(os.path.join(ROOT, "veckern_amd", "lib", "libveckern_bench.so"))
    lib.vkb_lds_floor.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double)]
    lib.vkb_hbm_read.argtypes = [ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    lib.vkb_lds_peak.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    floors = {}
    for qg in (1, 2, 4):
        rate, ms = ctypes.c_double(), ctypes.c_double()
        if lib.vkb_lds_floor(qg, 2000, 3, ctypes.byref(rate), ctypes.byref(ms)) != 0:
            raise RuntimeError("LDS floor microbenchmark failed")
        floors[qg] = rate.value
    lds_peak = ctypes.c_double()
    if lib.vkb_lds_peak(4000, 3, ctypes.byref(lds_peak)) != 0:
        raise RuntimeError("LDS peak microbenchmark failed")
    gbs = ctypes.c_double()
    if lib.vkb_hbm_read(1600 << 20, 5, ctypes.byref(gbs)) != 0:
        raise RuntimeError("HBM read microbenchmark failed")
    return floors, lds_peak.value, gbs.value


def cpu_baseline(centroids, codes, queries, k, d, target_s=10.0):
    """Times the CPU search on a bounded sample of the queries; returns (record, results of the sample)."""
    from oracle import binding as orc
    nq = queries.shape[0]
    use_ref = orc.ref_available()
    if use_ref:
        rpq = orc.RefPQ(centroids, d)
        codes_cpu = rpq.remap_codes(codes)
        run = lambda q: rpq.adc_search(codes_cpu, q, k)
    else:
        run = lambda q: orc.adc_search(centroids, d, codes, q, k)
    cores = orc.max_threads()
    try:
        host_cores = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        host_cores = os.cpu_count() or 0
    probe = min(nq, max(1, cores))
    t0 = time.perf_counter()
    run(queries[:probe])
    per_query = (time.perf_counter() - t0) / probe
    sample = int(min(nq, max(probe, round(target_s / max(per_query, 1e-9)))))
    # When the whole batch takes well under that, passes over it are repeated until about 2 s of wall time (some
    # 30 s of CPU work on 16 threads), a steadier rate than one short pass; otherwise one pass over the sample.
    t0 = time.perf_counter()
    res = run(queries[:sample])
    passes = 1
    while sample == nq and time.perf_counter() - t0 < 2.0:
        run(queries)
        passes += 1
    elapsed = time.perf_counter() - t0
    rec = {
        "value": sample * passes / elapsed,
        "unit": "queries/s",
        "cores": cores,
        "cores_basis": f"OpenMP threads used (omp_get_max_threads); the host offers {host_cores} cores "
                       f"(sched_getaffinity, `nproc`)",
        "host_cores": host_cores,
        "kind": "reference" if use_ref else "port",
        "sample": f"first {sample} of the {nq} queries against all {codes.shape[0]} codes, k={k}, "
                  + (f"{passes} passes, " if passes > 1 else "")
                  + f"{elapsed:.2f} s wall on {cores} OpenMP threads "
                  + ("(reference src/cpu/cpu_ref.cpp adc_search, -O3 -fopenmp)" if use_ref
                     else "(oracle port of cpu_ref.cpp adc_search, -O3 -fopenmp)"),
    }
    return rec, res


def bench_ivf(args, centroids, codes, queries, base):
    """IVF index on the configuration's data: coarse centroids by a few seeded Lloyd rounds (GPU assignment), then
    timed searches (HBM-resident queries and results; host buffers reported beside) and recall against the
    exhaustive PQ search and the exact ground truth."""
    import veckern_amd as vk
    from veckern_amd import host
    n, d, m, nq, k, data, _, _, desc = CONFIGS[args.config]
    if base is None:
        raise SystemExit("--ivf-lists needs base vectors (a mixture configuration)")
    nlist, nprobe = args.ivf_lists, args.nprobe
    t0 = time.time()
    rng = np.random.default_rng(1)
    coarse = base[np.sort(rng.choice(n, size=nlist, replace=False))].copy()
    for _ in range(2):  # Lloyd rounds: assignment on the GPU, means on the host
        ids = vk.ivf_assign(coarse, base)
        order = np.argsort(ids, kind="stable")
        counts = np.bincount(ids, minlength=nlist)
        starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
        sums = np.add.reduceat(base[order].astype(np.float64), starts[counts > 0], axis=0)
        coarse[counts > 0] = (sums / counts[counts > 0, None]).astype(np.float32)
    list_ids = vk.ivf_assign(coarse, base)
    log(f"[bench] IVF: {nlist} lists built in {time.time() - t0:.1f} s; largest list {np.bincount(list_ids).max()}")
    ix = vk.IVFIndex(coarse, centroids, codes, list_ids)
    # vectors each query's probed lists hold (coarse distances as float64 on the host: only the sizes are used)
    sizes = np.bincount(list_ids, minlength=nlist)
    cd = ((queries.astype(np.float64)[:, None, :] - coarse.astype(np.float64)[None]) ** 2).sum(-1)
    scanned = float(np.mean(sizes[np.argsort(cd, axis=1)[:, :nprobe]].sum(1)))
    # Timed steps with queries and results resident in HBM (the headline's convention), then the same searches
    # through host buffers (pageable copies in and out) for the PCIe-inclusive rate.
    dq = vk.DeviceArray.from_host(np.ascontiguousarray(queries, dtype=np.float32))
    dout = vk.DeviceArray(nq * k * vk.NEIGHBOR_DTYPE.itemsize)
    for _ in range(args.warmup):
        ix.search_device(dq.address, nq, nprobe, k, dout.address)
    totals = vk.Timings()
    t0 = time.perf_counter()  # each search_device call returns with its stream synchronised
    for _ in range(args.steps):
        t = ix.search_device(dq.address, nq, nprobe, k, dout.address)
        totals.lut_ms += t.lut_ms
        totals.scan_ms += t.scan_ms
        totals.select_ms += t.select_ms
    elapsed = time.perf_counter() - t0
    qps = nq * args.steps / elapsed
    res = dout.download(np.empty((nq, k), dtype=vk.NEIGHBOR_DTYPE))
    ix.search(queries, nprobe, k)  # untimed: the first host-buffer search allocates the page-locked staging
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dist, ids_out, t = ix.search(queries, nprobe, k)
        totals.transfer_ms += t.transfer_ms
    qps_host = nq * args.steps / (time.perf_counter() - t0)
    assert (res["id"] == ids_out).all() and (res["dist"].view(np.uint32) == dist.view(np.uint32)).all(), \
        "device-resident and host-buffer IVF searches differ"
    dq.free()
    dout.free()
    shape = ix.last_launch()
    with vk.PQSearcher(centroids, codes, d) as s:
        s.set_tuning(vk.Tuning(queries_per_block=4))
        _, ex_ids, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
    overlap = float(np.mean([len(set(ids_out[q]) & set(ex_ids[q])) / k for q in range(nq)]))
    ev = min(100, nq)
    gt = host.exact_knn(base, queries[:ev], k)
    out = np.empty((ev, k), dtype=vk.NEIGHBOR_DTYPE)
    out["dist"], out["id"] = dist[:ev], ids_out[:ev]
    rec = host.recall_at_k(out, gt["id"], k)
    ex = np.empty((ev, k), dtype=vk.NEIGHBOR_DTYPE)
    ex["id"] = ex_ids[:ev]
    rec_ex = host.recall_at_k(ex, gt["id"], k)
    step_ms = elapsed * 1e3 / args.steps
    log(f"[bench] IVF nprobe={nprobe}: {step_ms:.3f} ms/step, {qps:,.0f} queries/s (HBM-resident; "
        f"{qps_host:,.0f} with host buffers); per step probe + tables + plan "
        f"{totals.lut_ms / args.steps:.3f} + scan {totals.scan_ms / args.steps:.3f} + merge "
        f"{totals.select_ms / args.steps:.3f} ms (host buffers add {totals.transfer_ms / args.steps:.3f} ms of "
        f"copies); top-{k} overlap "
        f"with the exhaustive search {overlap:.4f}; recall@{k} {rec:.4f} (exhaustive {rec_ex:.4f}); "
        f"{scanned:,.0f} vectors scanned per query ({scanned / n * 100:.2f} %)")
    record = {
        "metric": f"queries/s, IVF-PQ ({nlist} lists, nprobe {nprobe})",
        "value": qps, "unit": "queries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": step_ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: the configuration's seeded mixture; coarse centroids from 2 Lloyd rounds",
        "config": {"workload": desc + f", IVF {nlist} lists, nprobe {nprobe}", "n": n, "d": d, "m": m, "nq": nq,
                   "k": k, "queries_per_block": shape.queries_per_block, "blocks": shape.blocks_x},
        "stage_ms": {"probe": totals.lut_ms / args.steps, "scan": totals.scan_ms / args.steps,
                     "merge": totals.select_ms / args.steps, "transfer": totals.transfer_ms / args.steps},
        "qps_host_buffers": qps_host, "topk_overlap_with_exhaustive": overlap, "recall_at_k": rec, "recall_at_k_exhaustive": rec_ex,
        "vectors_scanned_per_query": scanned,
    }
    ix.close()
    print(json.dumps(record), flush=True)


def load_traffic(cfg, f16):
    """Counter record of the search kernel for this configuration (profiles/traffic.json, from rocprofv3 --pmc runs):
    HBM bytes per launch and the binding pipe, if recorded."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(cfg + ("/v9" if f16 else ""))
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # 100 untimed steps let the GPU's clocks settle: at the headline, 10 warm-up steps left the timed 200 about 1 %
    # slower, and 5 before 50 timed steps about 5 % slower, than 100 before either.
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="B", choices=sorted(CONFIGS))
    ap.add_argument("--variant", default="v8")
    ap.add_argument("--queries-per-block", type=int, default=None,
                    help="Q (default 8 for the fp16-table variant v9, whose 16-byte reads hold 8 queries' entries; "
                         "2 for config A, whose 100k-vector slabs give a block too little to scan for 4 queries' "
                         "tables; 4 otherwise)")
    ap.add_argument("--ilp", type=int, default=4)
    ap.add_argument("--blocks-per-query", type=int, default=0)
    ap.add_argument("--threads", type=int, default=0,
                    help="v8/v9 block size: 512 or 1024 (0: the library chooses)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and its parity check")
    ap.add_argument("--no-recall", action="store_true", help="skip the exact ground truth and recall")
    ap.add_argument("--ivf-lists", type=int, default=0, metavar="NLIST",
                    help="instead of the exhaustive search, time the IVF index (NLIST coarse lists) on the same data")
    ap.add_argument("--nprobe", type=int, default=32, help="lists probed per query with --ivf-lists")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run one plain device copy of BYTES (for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.calibrate_copy:
        import veckern_amd as vk
        vk.library()
        lib = ctypes.CDLL(os.path.join(ROOT, "veckern_amd", "lib", "libveckern_bench.so"))
        lib.vkb_copy.argtypes = [ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
        gbs = ctypes.c_double()
        if lib.vkb_copy(args.calibrate_copy, 1, ctypes.byref(gbs)) != 0:
            raise RuntimeError("copy kernel failed")
        print(json.dumps({"copy_bytes": args.calibrate_copy, "dispatches": 2, "gbs": gbs.value}), flush=True)
        return

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (the search path is built and "
              f"measured on a single MI355X; multi-GPU sharding is a design note, not a code path)", file=sys.stderr)
        sys.exit(2)

    import veckern_amd as vk
    variant = next(v for v in vk.ScanVariant if vk.variant_name(v).startswith(args.variant))
    n, d, m, nq, k, data, _, _, desc = CONFIGS[args.config]
    centroids, codes, queries, base = make_workload(args.config)
    if args.ivf_lists:
        return bench_ivf(args, centroids, codes, queries, base)

    floors, lds_peak, hbm_gbs = microbench()
    info = vk.device_info()
    # 64 lookups per CU-cycle: 256 B/clk/CU of LDS reads at 4 bytes per fp32 entry, and 64 VALU lanes per CU-cycle
    # at one add (fp32) or one v_fma_mix_f32 (fp16 entries) per lookup.
    peak = 64.0 * info.sm_count * info.clock_khz * 1e3
    log(f"[bench] LDS random-lookup floor: " + ", ".join(f"QG{q} {r / 1e12:.2f} Tlookup/s" for q, r in floors.items())
        + f"; conflict-free LDS reads {lds_peak / 1e12:.2f} T entries/s (peak {peak / 1e12:.2f}); "
        f"HBM read {hbm_gbs:.0f} GB/s")

    t_setup = time.perf_counter()
    s = vk.PQSearcher(centroids, codes, d)
    setup_s = time.perf_counter() - t_setup
    # Queries per block: fp16 tables put 8 queries in one 16-byte table read; 100k runs faster at 2 (launch- and
    # latency-bound: more, smaller slabs); 1M at m=32 (k=100) at 4 with one 1024-thread block per CU (1.86 ms against
    # 1.92 at Q=2); m=64 at 2, the most its tables allow.
    # 10M (nq=1000) at 8: the search is VALU-bound there and eight queries share each code byte's address op (5.30
    # against 5.40 ms at Q=4); at 1M eight queries per block cost more in per-block tables and merges than they save.
    if args.queries_per_block is None:
        args.queries_per_block = (8 if variant == vk.ScanVariant.FusedWarpF16 or args.config == "D"
                                  else (2 if args.config == "A" else 4))
    s.set_tuning(vk.Tuning(scan_threads=args.threads or 256, queries_per_block=args.queries_per_block,
                           vectors_per_step=args.ilp, blocks_per_query=args.blocks_per_query))
    dq = vk.DeviceArray.from_host(queries)
    dout = vk.DeviceArray(nq * k * 8)
    t_first = time.perf_counter()
    s.search_device(dq.address, nq, k, variant, dout.address)  # builds the sorted code layout (slot order on the GPU)
    first_s = time.perf_counter() - t_first
    for _ in range(max(args.warmup - 1, 0)):
        s.search_device(dq.address, nq, k, variant, dout.address)
    shape = s.last_launch()

    totals = vk.Timings()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        t = s.search_device(dq.address, nq, k, variant, dout.address)
        totals.lut_ms += t.lut_ms
        totals.scan_ms += t.scan_ms
        totals.select_ms += t.select_ms
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    qps = nq * args.steps / elapsed
    scan_ms = totals.scan_ms / args.steps
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step, {qps:,.0f} queries/s; per step LUT "
        f"{totals.lut_ms / args.steps:.3f} + scan {scan_ms:.3f} + select {totals.select_ms / args.steps:.3f} ms")

    out = np.empty((nq, k), dtype=vk.NEIGHBOR_DTYPE)
    dout.download(out)

    # Host-buffer path (queries in and results out over PCIe), reported beside the device-resident value: the
    # median total (transfers + search) of several warmed calls, as the reference times its repetitions
    # (bench_main.cpp:199-217).
    host_totals = []
    for _ in range(6):
        _, _, th = s.search(queries, k, variant)
        host_totals.append(th.total_ms())
    host_ms = float(np.median(host_totals[1:]))
    host_qps = nq / (host_ms * 1e-3)

    lookups = float(n) * m * nq
    achieved = lookups / (scan_ms * 1e-3)
    q_eff = shape.queries_per_block
    hbm_bytes = float(n) * m * math.ceil(nq / q_eff)
    f16 = variant == vk.ScanVariant.FusedWarpF16
    # The binding pipe, from the counters of this kernel (profiles/traffic.json): "valu" where the VALU issues more
    # wave64 instructions per CU-cycle than the LDS is busy (1M and 10M at m=16: 0.91-0.93 against 77-90 %; fp16
    # tables), "lds" where bank conflicts keep the LDS busier (m=32 and m=64 at k=100, 100M uniform codes: 87-97 %).
    counters = load_traffic(args.config, f16) or {}
    roofline = {
        "bound": counters.get("bound", "valu"),
        "bound_basis": ({"valu_instr_per_cu_cycle": counters["valu_per_cu_cycle"], "lds_busy": counters["lds_busy"]}
                        if "lds_busy" in counters else None),
        "achieved": achieved / 1e12,
        "peak": peak / 1e12,
        "unit": "Tlookup/s",
        "frac": achieved / peak,
        "traffic": counters.get("bytes_per_launch"),
        "traffic_detail": counters or None,
        "kernel": "fused_wave_kernel_t (scan + per-wave top-k)",
        "kernel_ms": scan_ms,
        "algorithmic": f"n*m*nq = {lookups:.3e} LDS lookups per launch (one {2 if f16 else 4}-byte table read + "
                       f"one fp32 add each)",
        "peak_basis": (f"64 lookups per CU-cycle x {info.sm_count} CUs x {info.clock_khz / 1e6:.2f} GHz: the LDS "
                       f"returns 256 B/clk/CU (one 4-byte fp32 entry per lookup) and the VALU 64 lane-ops/clk/CU "
                       f"(one add, or one v_fma_mix_f32 for fp16 entries, per lookup)"),
        "peak_measured": lds_peak / 1e12,
        "peak_measured_basis": "conflict-free ds_read_b128 microbenchmark, 4-byte entries per second",
        "random_lookup_floor_by_width": {f"b{32 * q}_Q{q}": floors[q] / 1e12 for q in floors},
        "hbm": {"achieved_gbs": hbm_bytes / (scan_ms * 1e-3) / 1e9, "peak_gbs": HBM_PEAK_GBS,
                "frac": hbm_bytes / (scan_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "measured_read_gbs": hbm_gbs,
                "algorithmic_bytes": hbm_bytes,
                "note": "n*m code bytes per slab of Q queries, ceil(nq/Q) slabs per launch"},
    }

    record = {
        "metric": METRIC,
        "value": qps,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        # The reference's A100 figure includes its PCIe transfers, so the comparable rate is the host-buffer one;
        # the lower of it and the device-resident rate is used.
        "vs_baseline": min(host_qps, qps) / A100_V8_QPS if args.config == "B" else None,
        "vs_baseline_basis": ("min(qps_host_buffers, value) / the reference's A100 v8 86,216 queries/s, which "
                              "includes its PCIe transfers (results/final/scaling.csv:11)")
                             if args.config == "B" else None,
        "dtype": "f16 tables, f32 sums" if f16 else "f32",
        "data": ("synthetic: seeded 1000-component Gaussian mixture (sigma 0.3), PQ trained by seeded k-means"
                 if data == "mixture" else "synthetic: seeded uniform codes, N(0,1) codebooks and queries"),
        "config": {"workload": desc, "n": n, "d": d, "m": m, "nq": nq, "k": k, "variant": vk.variant_name(variant),
                   "queries_per_block": shape.queries_per_block, "vectors_per_step": shape.vectors_per_step,
                   "threads": shape.threads, "blocks": shape.blocks_x, "blocks_per_cu": shape.blocks_per_sm},
        "roofline": roofline,
        "stage_ms": {"lut": totals.lut_ms / args.steps, "scan": scan_ms, "select": totals.select_ms / args.steps},
        "searcher_setup_s": {"create": setup_s, "first_search": first_s,
                             "note": "PQSearcher creation (device copies of codes and codebook) and the first "
                                     "search, which builds the slot order and sorted code layout on the GPU"},
        "qps_host_buffers": host_qps,
        "qps_host_buffers_basis": f"median total (H2D queries + search + D2H results) of 5 warmed calls: "
                                  f"{host_ms:.3f} ms",
    }

    if args.config == "E":
        # The 100M workload's stated target is 80 % of HBM peak in algorithmic code bytes (n*m per slab of Q
        # queries). Fewer queries per block stream more code bytes per lookup: when this run's Q is above 2, a few
        # steps at Q=2 are timed as well and reported beside it.
        hbm_frac = roofline["hbm"]["frac"]
        record["hbm_target_met"] = bool(hbm_frac >= 0.80)
        at_q2 = None
        if q_eff > 2 and variant == vk.ScanVariant.FusedWarp:
            s.set_tuning(vk.Tuning(queries_per_block=2, vectors_per_step=args.ilp,
                                   blocks_per_query=args.blocks_per_query))
            s.search_device(dq.address, nq, k, variant, dout.address)
            q2_ms = sum(s.search_device(dq.address, nq, k, variant, dout.address).scan_ms for _ in range(3)) / 3
            q2_bytes = float(n) * m * math.ceil(nq / s.last_launch().queries_per_block)
            at_q2 = {"queries_per_block": s.last_launch().queries_per_block, "kernel_ms": q2_ms,
                     "achieved_gbs": q2_bytes / (q2_ms * 1e-3) / 1e9,
                     "frac": q2_bytes / (q2_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "queries_per_s": nq / (q2_ms * 1e-3)}
            record["hbm_target_at_q2"] = at_q2
            record["hbm_target_met_at_q2"] = bool(at_q2["frac"] >= 0.80)
            log(f"[bench] at Q=2: {q2_ms:.2f} ms per search, {at_q2['frac'] * 100:.1f} % of the HBM peak")
        record["hbm_target"] = {
            "target_frac": 0.80, "achieved_frac": hbm_frac,
            "reason": None if hbm_frac >= 0.80 else
            (f"at Q={q_eff} each code byte serves {q_eff} queries, so the fastest search reads codes at "
             f"{hbm_frac * 100:.1f} % of the HBM peak while its lookups run at {roofline['frac'] * 100:.1f} % of the "
             f"lookup peak" + ("" if at_q2 is None else
                               f"; at Q=2 the same search streams codes at {at_q2['frac'] * 100:.1f} % of the HBM peak "
                               f"({at_q2['kernel_ms']:.1f} ms per search against {scan_ms:.1f} ms)")),
        }
        log(f"[bench] HBM target (80 % of {HBM_PEAK_GBS / 1e3:.0f} TB/s) met: {record['hbm_target_met']} "
            f"({hbm_frac * 100:.1f} %)")

    if not args.no_recall and base is not None:
        from veckern_amd import host
        ev = min(100, nq)
        gt = host.exact_knn(base, queries[:ev], k)
        record["recall_at_k"] = host.recall_at_k(out[:ev], gt["id"], k)
        log(f"[bench] recall@{k} over {ev} queries: {record['recall_at_k']:.4f}")

    if not args.no_cpu:
        rec, res = cpu_baseline(centroids, codes, queries, k, d)
        record["cpu_baseline"] = rec
        sample = res.shape[0]
        against = rec["kind"]
        if f16:
            # fp16 tables are checked against their own restatement; the fp32 reference gives the recall delta
            from oracle import binding as orc
            overlap = float(np.mean([len(set(res["id"][q]) & set(out["id"][q])) / k for q in range(sample)]))
            record["recall_delta"] = {"queries": sample, "topk_overlap_with_fp32_reference": overlap,
                                      "note": "fraction of the fp32 CPU reference's top-k ids that the fp16-table "
                                              "search also returns"}
            log(f"[bench] fp16 tables: top-{k} overlap with the fp32 reference {overlap:.4f}")
            res = orc.adc_search_f16(centroids, d, codes, queries[:sample], k)
            against = "oracle fp16-table restatement"
        same_ids = bool((res["id"] == out[:sample]["id"]).all())
        same_bits = bool((res["dist"].view(np.uint32) == out[:sample]["dist"].view(np.uint32)).all())
        record["parity"] = {"queries": sample, "ids_identical": same_ids, "dist_bits_identical": same_bits,
                            "against": against}
        log(f"[bench] CPU {rec['kind']}: {rec['value']:.1f} queries/s on {rec['cores']} threads; parity ids "
            f"{same_ids} dist bits {same_bits}")
    else:
        record["cpu_baseline"] = None

    s.close()
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
