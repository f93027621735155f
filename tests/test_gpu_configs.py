"""Parity at the benchmark's full sizes: every workload bench.py measures, built by bench.make_workload, searched on
the GPU through the C ABI and compared with the reference's own CPU adc_search (cpu_ref.cpp:38-54, compiled from its
sources into oracle/_ref; the oracle port when that library is absent). The bar is the one of every parity test:
ids identical and distance bits identical.

Workloads (d = 128 throughout):
  A    100k vectors, m16, nq=100, k=10, Q=2            all queries
  B    1M, m16, nq=1000, k=10, Q=4 (the headline)      all queries; the launch shape is asserted
  C32  1M, m32, nq=1000, k=100, Q=2 and Q=4           all queries
  C64  1M, m64, nq=1000, k=100                         all queries
  D    10M, m16, nq=1000, k=10                         the GPU searches all 1000, the first 100 are compared
  D1   10M, m16, nq=1, k=10                            the single-query search (one slab over every block)
  E    100M uniform codes, m16, nq=1000, k=10          the GPU searches all 1000, the first 16 are compared
fp16 tables (ScanVariant.FusedWarpF16) at B (all queries) and D (first 100) are compared with the oracle's
restatement of the fp16-table arithmetic.

Large launches exercise what the small parity cases cannot: hundreds of slabs, per-slab completion counters over
many slabs, the block-merged (one list per block) partial lists when more than 8 blocks share a slab (A, D1), and
id / tile arithmetic at 10M and 100M vectors.
"""
import gc

import numpy as np
import pytest

import veckern_amd as vk
from bench import CONFIGS, make_workload
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def cpu_search(centroids, codes, queries, k, d):
    """The reference's adc_search (oracle/_ref) on the given queries, or the oracle port without it."""
    if orc.ref_available():
        rpq = orc.RefPQ(centroids, d)
        try:
            return rpq.adc_search(rpq.remap_codes(codes), queries, k)
        finally:
            rpq.close()
    return orc.adc_search(centroids, d, codes, queries, k)


def assert_identical(dist, ids, exp, label):
    assert ids.shape == exp.shape, label
    bad = np.argwhere((ids != exp["id"]) | (dist.view(np.uint32) != exp["dist"].view(np.uint32)))
    if bad.size:
        q, j = bad[0]
        raise AssertionError(f"{label}: {len(bad)} mismatches; first at query {q} rank {j}: got ({dist[q, j]!r}, "
                             f"{ids[q, j]}) expected ({exp['dist'][q, j]!r}, {exp['id'][q, j]})")
    assert (np.diff(dist, axis=1) >= 0).all(), label


def search_device(s, queries, k, variant):
    """One search with queries and results in HBM (the benchmark's timed entry point)."""
    nq = queries.shape[0]
    dq = vk.DeviceArray.from_host(np.ascontiguousarray(queries, dtype=np.float32))
    dout = vk.DeviceArray(nq * k * vk.NEIGHBOR_DTYPE.itemsize)
    try:
        s.search_device(dq.address, nq, k, variant, dout.address)
        out = dout.download(np.empty((nq, k), dtype=vk.NEIGHBOR_DTYPE))
    finally:
        dq.free()
        dout.free()
    return out["dist"], out["id"]


class Workload:
    def __init__(self, cfg):
        print(f"\n    [configs] building workload {cfg}", flush=True)
        n, d, m, nq, k, *_ = CONFIGS[cfg]
        self.cfg, self.n, self.d, self.m, self.nq, self.k = cfg, n, d, m, nq, k
        self.centroids, self.codes, self.queries, base = make_workload(cfg)
        del base  # only the codes are searched
        gc.collect()


def run_config(cfg, q, compared, variant=vk.ScanVariant.FusedWarp, check_device=True):
    w = Workload(cfg)
    print(f"    [configs] {cfg}: GPU search (Q={q}, {vk.variant_name(variant)})", flush=True)
    with vk.PQSearcher(w.centroids, w.codes, w.d) as s:
        s.set_tuning(vk.Tuning(queries_per_block=q))
        dist, ids, _ = s.search(w.queries, w.k, variant)
        shape = s.last_launch()
        if check_device:
            dd, di = search_device(s, w.queries, w.k, variant)
            assert (di == ids).all() and (dd.view(np.uint32) == dist.view(np.uint32)).all(), \
                f"{cfg}: device-resident and host-buffer searches differ"
    print(f"    [configs] {cfg}: CPU reference on {compared} queries", flush=True)
    sample = w.queries[:compared]
    if variant == vk.ScanVariant.FusedWarpF16:
        exp = orc.adc_search_f16(w.centroids, w.d, w.codes, sample, w.k)
    else:
        exp = cpu_search(w.centroids, w.codes, sample, w.k, w.d)
    assert_identical(dist[:compared], ids[:compared], exp, f"{cfg} {vk.variant_name(variant)} Q={q}")
    w.dist, w.ids = dist, ids
    return w, shape


def test_config_a_all_queries():
    _, shape = run_config("A", 2, 100)
    assert shape.queries_per_block == 2


def test_config_b_headline_all_queries_and_launch_shape():
    w, shape = run_config("B", 4, 1000)
    info = vk.device_info()
    # One 1024-thread block per CU (16 waves sharing one granule counter): 250 slabs of 4 queries, one block each
    # while the slabs are no more than the CUs.
    assert shape.threads == 1024 and shape.queries_per_block == 4 and shape.vectors_per_step == 4
    assert shape.blocks_per_sm == 1
    assert shape.blocks_x == 250 * max(1, info.sm_count // 250), (shape.blocks_x, info.sm_count)
    # The 512-thread instances (two blocks per CU, each slab split between two blocks) return the same bits.
    print("    [configs] B: GPU search with 512-thread blocks", flush=True)
    with vk.PQSearcher(w.centroids, w.codes, w.d) as s:
        s.set_tuning(vk.Tuning(scan_threads=512, queries_per_block=4))
        dist, ids, _ = s.search(w.queries, w.k, vk.ScanVariant.FusedWarp)
        narrow = s.last_launch()
    assert narrow.threads == 512
    resident = narrow.blocks_per_sm * info.sm_count
    assert narrow.blocks_x == 250 * (resident // 250), (narrow.blocks_x, resident)
    assert (ids == w.ids).all() and (dist.view(np.uint32) == w.dist.view(np.uint32)).all()


@pytest.mark.parametrize("cfg,q", [("C32", 2), ("C32", 4), ("C64", 2)])
def test_config_c_k100_all_queries(cfg, q):
    _, shape = run_config(cfg, q, 1000)
    assert shape.queries_per_block == q


@pytest.mark.parametrize("q", [4, 8])
def test_config_d_10m(q):
    # Q=8, the benchmark's default at 10M: two 4-query tables sharing each address, code words staged per tile.
    _, shape = run_config("D", q, 100)
    assert shape.queries_per_block == q and shape.threads == 1024


def test_config_d1_single_query():
    w, shape = run_config("D1", 4, 1)
    # one slab spread over every CU: the block-merged partial lists and the many-list final merge
    assert shape.queries_per_block == 1 and shape.blocks_x >= 64


def test_config_e_100m_direct_codes():
    run_config("E", 4, 16)


@pytest.mark.parametrize("cfg,compared", [("B", 1000), ("D", 100)])
def test_fp16_tables_at_b_and_d(cfg, compared):
    _, shape = run_config(cfg, 8, compared, variant=vk.ScanVariant.FusedWarpF16, check_device=False)
    assert shape.queries_per_block == 8
