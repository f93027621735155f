"""GPU parity of every ScanVariant and of distances(), through the C ABI (cases of the reference's
tests/test_gpu.cpp:62-202, at a bit-exact bar instead of its 1e-3 tolerance and 99% id agreement).
"""
import numpy as np
import pytest

import veckern_amd as vk
from oracle import binding as orc
from tests import datagen

pytestmark = pytest.mark.gpu

N, D, M, NQ = 50_003, 64, 16, 37
SCAN = [vk.ScanVariant.GlobalLut, vk.ScanVariant.SharedLut, vk.ScanVariant.SharedLutVec, vk.ScanVariant.Interleaved]
# v4 (Fused) is rejected before launch in this build: its run-time-indexed per-thread list faulted the GPU with a
# memory-aperture violation whose cause is not established, so it is not run here (see test_v4_is_rejected).
FUSED = [vk.ScanVariant.FusedReg, vk.ScanVariant.FusedVec, vk.ScanVariant.FusedVecMQ, vk.ScanVariant.FusedWarp]


@pytest.fixture(scope="module")
def fx():
    centroids, codes, queries = datagen.pq_fixture(N, D, M, NQ, seed=11)
    s = vk.PQSearcher(centroids, codes, D)
    yield centroids, codes, queries, s
    s.close()


_cache = {}


def expected(fx, k):
    if k not in _cache:
        centroids, codes, queries, _ = fx
        _cache[k] = orc.adc_search(centroids, D, codes, queries, k)
    return _cache[k]


def check(fx, k, v, tuning=vk.Tuning(), queries=None, exp=None):
    _, _, q, s = fx
    s.set_tuning(tuning)
    q = q if queries is None else queries
    exp = expected(fx, k) if exp is None else exp
    d, i, _ = s.search(q, k, v)
    bad = (i != exp["id"]) | (d.view(np.uint32) != exp["dist"].view(np.uint32))
    assert not bad.any(), f"{vk.variant_name(v)} k={k} {tuning}: {int(bad.sum())} mismatches"
    assert (np.diff(d, axis=1) >= 0).all()


def test_every_scan_variant_reproduces_cpu_distances(fx):
    centroids, codes, queries, s = fx
    exp = orc.adc_scan(orc.compute_lut(centroids, D, M, queries), codes)
    for v in SCAN:
        got, t = s.distances(queries, v)
        assert (got.view(np.uint32) == exp.view(np.uint32)).all(), vk.variant_name(v)
        assert t.scan_ms > 0


def test_distances_rejects_fused_variants(fx):
    _, _, queries, s = fx
    for v in FUSED + [vk.ScanVariant.Fused]:
        with pytest.raises(vk.VkError):
            s.distances(queries[:1], v)


def test_search_all_variants_k10(fx):
    for v in SCAN + FUSED:
        check(fx, 10, v)


@pytest.mark.parametrize("k", [1, 16, 33, 100])
def test_every_k_template(fx, k):
    check(fx, k, vk.ScanVariant.SharedLut)
    for v in FUSED:
        check(fx, k, v)


@pytest.mark.parametrize("q", [1, 2, 4, 8])
def test_v7_every_queries_per_block(fx, q):
    for k in (1, 8, 10, 32):
        check(fx, k, vk.ScanVariant.FusedVecMQ, vk.Tuning(queries_per_block=q))


def test_tuning_overrides(fx):
    for threads in (64, 96, 128, 512, 1024):
        check(fx, 10, vk.ScanVariant.SharedLutVec, vk.Tuning(scan_threads=threads))
        check(fx, 10, vk.ScanVariant.Interleaved, vk.Tuning(scan_threads=threads))
    for bpq in (1, 3, 16):
        for v in (vk.ScanVariant.FusedReg, vk.ScanVariant.FusedVec, vk.ScanVariant.FusedVecMQ):
            check(fx, 10, v, vk.Tuning(blocks_per_query=bpq))
    for ilp in (2, 4):
        for bpq in (0, 7):
            for k in (1, 10, 33):
                for v in (vk.ScanVariant.FusedVec, vk.ScanVariant.FusedVecMQ, vk.ScanVariant.FusedWarp):
                    check(fx, k, v, vk.Tuning(vectors_per_step=ilp, blocks_per_query=bpq))


def test_launch_shape_reports_the_wave_model(fx):
    _, _, queries, s = fx
    s.set_tuning(vk.Tuning())
    s.search(queries, 10, vk.ScanVariant.FusedVecMQ)
    shape = s.last_launch()
    assert shape.queries_per_block == 2 and shape.grid_y == 19  # ceil(37 / 2)
    assert shape.blocks_per_sm > 0 and shape.waves > 0


def test_m8_codes_rejected_by_word_variants_and_accepted_by_v5():
    centroids, codes, queries = datagen.pq_fixture(N, D, 8, NQ, seed=12)
    with vk.PQSearcher(centroids, codes, D) as s:
        for v in (vk.ScanVariant.SharedLutVec, vk.ScanVariant.FusedVec, vk.ScanVariant.FusedVecMQ,
                  vk.ScanVariant.FusedWarp):
            with pytest.raises(vk.VkError):
                s.search(queries, 10, v)
        exp = orc.adc_search(centroids, D, codes, queries, 10)
        for v in (vk.ScanVariant.GlobalLut, vk.ScanVariant.Interleaved, vk.ScanVariant.FusedReg):
            d, i, _ = s.search(queries, 10, v)
            assert (i == exp["id"]).all() and (d.view(np.uint32) == exp["dist"].view(np.uint32)).all()


def test_invalid_tuning_and_k_are_rejected(fx):
    _, _, queries, s = fx
    for bad in (vk.Tuning(100, 0, 2, 1), vk.Tuning(256, -1, 2, 1), vk.Tuning(256, 0, 3, 1), vk.Tuning(256, 0, 2, 3)):
        with pytest.raises(vk.VkError):
            s.set_tuning(bad)
    with pytest.raises(vk.VkError):
        s.search(queries[:1], 129, vk.ScanVariant.FusedReg)


def test_v4_is_rejected_before_launch(fx):
    _, _, queries, s = fx
    with pytest.raises(vk.VkLogicError, match="v4_fused is not launched"):
        s.search(queries[:1], 10, vk.ScanVariant.Fused)


@pytest.mark.skip(reason="v4_fused faulted the GPU (memory-aperture violation with its list in scratch, reached "
                         "through generic pointers by a non-inlined insert); the cause is not established, so no v4 "
                         "kernel is run")
def test_v4_parity():
    pass


def test_tie_heavy_data_every_variant():
    centroids, codes, queries = datagen.tie_fixture(9_001, 64, 16, 11, seed=21)
    with vk.PQSearcher(centroids, codes, 64) as s:
        for k in (10, 64):
            exp = orc.adc_search(centroids, 64, codes, queries, k)
            for v in SCAN + FUSED:
                d, i, _ = s.search(queries, k, v)
                assert (i == exp["id"]).all() and (d.view(np.uint32) == exp["dist"].view(np.uint32)).all(), \
                    f"{vk.variant_name(v)} k={k}"


@pytest.mark.parametrize("n", [12_288, 12_292])
def test_unfused_selection_on_aligned_rows(n):
    # rows of n distances with n % 4 == 0: the select kernel reads them in 1024-distance rounds of 16-byte loads
    # (n = 12,288: whole rounds only; 12,292: a 4-distance tail), k = 10 and 100, ties included
    centroids, codes, queries = datagen.tie_fixture(n, D, M, 21, seed=23)
    exp = {k: orc.adc_search(centroids, D, codes, queries, k) for k in (10, 100)}
    with vk.PQSearcher(centroids, codes, D) as s:
        for v in SCAN:
            for k in (10, 100):
                d, i, _ = s.search(queries, k, v)
                bad = (i != exp[k]["id"]) | (d.view(np.uint32) != exp[k]["dist"].view(np.uint32))
                assert not bad.any(), f"{vk.variant_name(v)} n={n} k={k}: {int(bad.sum())} mismatches"
