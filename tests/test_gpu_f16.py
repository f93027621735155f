"""GPU parity of the fp16-table search (ScanVariant.FusedWarpF16) through the C ABI.

The bar is bit-exact against the oracle's restatement of the same arithmetic (oracle/vk_oracle.c,
vko_adc_search_f16): fp32 LUT entries, a per-query power-of-two scale, round-to-nearest-even binary16, fp32 sums
in sub-space order, top-k by (dist, id), distances scaled back. Cases cover every Q (1, 2, 4, 8 queries per
16-byte read), ILP, both final-merge paths, m = 16/32/64 and a run-time m, tie-heavy data, data whose tables
would overflow binary16 without the scale, tiny-valued data with binary16 subnormal entries, and the distance to
the fp32 path (recall delta).
"""
import numpy as np
import pytest

import veckern_amd as vk
from tests import datagen
from oracle import binding as orc

pytestmark = pytest.mark.gpu

F16 = vk.ScanVariant.FusedWarpF16
N, D, M, NQ = 50_003, 64, 16, 37


@pytest.fixture(scope="module")
def fixture():
    return datagen.pq_fixture(N, D, M, NQ, seed=11)


@pytest.fixture(scope="module")
def searcher(fixture):
    centroids, codes, _ = fixture
    s = vk.PQSearcher(centroids, codes, D)
    yield s
    s.close()


_expected_cache = {}


def expected(fixture, k):
    if k not in _expected_cache:
        centroids, codes, queries = fixture
        _expected_cache[k] = orc.adc_search_f16(centroids, D, codes, queries, k)
    return _expected_cache[k]


def assert_same(got_d, got_i, exp, label=""):
    assert got_i.shape == exp.shape, label
    bad = np.argwhere((got_i != exp["id"]) | (got_d.view(np.uint32) != exp["dist"].view(np.uint32)))
    if bad.size:
        q, j = bad[0]
        raise AssertionError(f"{label}: {len(bad)} mismatches; first at query {q} rank {j}: "
                             f"got ({got_d[q, j]!r}, {got_i[q, j]}) expected ({exp['dist'][q, j]!r}, {exp['id'][q, j]})")


@pytest.mark.parametrize("k", [1, 10, 33, 64, 100, 128])
def test_f16_every_k(fixture, searcher, k):
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning(queries_per_block=8))
    d, i, t = searcher.search(queries, k, F16)
    assert_same(d, i, expected(fixture, k), f"v9 k={k}")
    assert t.scan_ms > 0 and t.lut_ms == 0 and t.select_ms == 0


@pytest.mark.parametrize("q", [1, 2, 4, 8])
@pytest.mark.parametrize("ilp", [1, 2, 4])
def test_f16_every_q_and_ilp(fixture, searcher, q, ilp):
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning(queries_per_block=q, vectors_per_step=ilp))
    for k in (10, 100):
        d, i, _ = searcher.search(queries, k, F16)
        assert_same(d, i, expected(fixture, k), f"v9 Q={q} ILP={ilp} k={k}")
    shape = searcher.last_launch()
    assert shape.queries_per_block == q and shape.vectors_per_step == ilp


@pytest.mark.parametrize("bpq", [1, 3, 16])
def test_f16_both_final_merge_paths(fixture, searcher, bpq):
    # few blocks per slab: one partial list per wave; many: the block merges its wave lists first
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning(blocks_per_query=bpq, queries_per_block=8))
    for k in (1, 10, 128):
        d, i, _ = searcher.search(queries, k, F16)
        assert_same(d, i, expected(fixture, k), f"v9 bpq={bpq} k={k}")


@pytest.mark.parametrize("family", ["random", "tie"])
@pytest.mark.parametrize("m", [16, 32, 64])
def test_f16_other_m_and_tie_heavy_data(family, m):
    gen = datagen.random_fixture if family == "random" else datagen.tie_fixture
    n, d, nq = 20_011, 128, 13
    centroids, codes, queries = gen(n, d, m, nq, seed=7 + m)
    with vk.PQSearcher(centroids, codes, d) as s:
        for q in (1, 4, 8):
            s.set_tuning(vk.Tuning(queries_per_block=q))
            for k in (10, 100):
                got_d, got_i, _ = s.search(queries, k, F16)
                exp = orc.adc_search_f16(centroids, d, codes, queries, k)
                assert_same(got_d, got_i, exp, f"{family} m={m} Q={q} k={k}")


def test_f16_generic_m_path():
    n, d, m, nq = 9_001, 96, 48, 9
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=4)
    with vk.PQSearcher(centroids, codes, d) as s:
        for q in (1, 2, 4):
            s.set_tuning(vk.Tuning(queries_per_block=q))
            got_d, got_i, _ = s.search(queries, 10, F16)
            assert_same(got_d, got_i, orc.adc_search_f16(centroids, d, codes, queries, 10), f"m=48 Q={q}")


@pytest.mark.parametrize("scale", [300.0, 1e-3])
def test_f16_scaled_data(scale):
    # x300: fp32 entries up to ~1e6 would overflow binary16 (65504) without the per-query power of two;
    # x1e-3: entries near 1e-6 would sit in binary16's subnormal range without it
    n, d, m, nq = 20_011, 64, 16, 11
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=21)
    centroids, queries = (centroids * scale).astype(np.float32), (queries * scale).astype(np.float32)
    with vk.PQSearcher(centroids, codes, d) as s:
        for q in (1, 8):
            s.set_tuning(vk.Tuning(queries_per_block=q))
            got_d, got_i, _ = s.search(queries, 10, F16)
            exp = orc.adc_search_f16(centroids, d, codes, queries, 10)
            assert np.isfinite(exp["dist"]).all()
            assert_same(got_d, got_i, exp, f"x{scale} Q={q}")


def test_f16_subnormal_table_entries():
    # queries that nearly coincide with one centroid per sub-space next to far-away centroids: a dynamic range of
    # ~1e12 inside one table puts the small entries in binary16's subnormal range (and some at zero)
    n, d, m, nq = 12_007, 64, 16, 6
    rng = np.random.default_rng(17)
    centroids = rng.standard_normal((m, 256, d // m)).astype(np.float32) * 100
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    pick = rng.integers(0, 256, size=(nq, m))
    queries = np.concatenate([centroids[s][pick[:, s]] for s in range(m)], axis=1)
    queries = (queries + rng.standard_normal(queries.shape).astype(np.float32) * 1e-4).astype(np.float32)
    with vk.PQSearcher(centroids, codes, d) as s:
        for q in (1, 8):
            s.set_tuning(vk.Tuning(queries_per_block=q))
            got_d, got_i, _ = s.search(queries, 16, F16)
            assert_same(got_d, got_i, orc.adc_search_f16(centroids, d, codes, queries, 16), f"subnormal Q={q}")


def test_f16_tiny_database_and_nq_one():
    n, d, m, nq = 70, 32, 16, 5
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=10)
    with vk.PQSearcher(centroids, codes, d) as s:
        for k in (1, 64, 70):
            got_d, got_i, _ = s.search(queries, k, F16)
            assert_same(got_d, got_i, orc.adc_search_f16(centroids, d, codes, queries, k), f"n=70 k={k}")
        got_d, got_i, _ = s.search(queries[:1], 10, F16)
        assert_same(got_d, got_i, orc.adc_search_f16(centroids, d, codes, queries[:1], 10), "nq=1")


@pytest.mark.parametrize("family", ["random", "tie"])
def test_f16_single_query_over_many_blocks(family):
    # one query spread over ~37 blocks: the last block bounds the k-th best by the k-th smallest head of the blocks'
    # lists and merges only the pairs at or below it (tie-heavy data: pairs equal to the bound must survive);
    # repeated searches check that the slab state starts fresh
    gen = datagen.random_fixture if family == "random" else datagen.tie_fixture
    n, d, m, nq = 300_007, 32, 16, 2
    centroids, codes, queries = gen(n, d, m, nq, seed=41)
    with vk.PQSearcher(centroids, codes, d) as s:
        for k in (1, 10, 64, 100, 10):
            got_d, got_i, _ = s.search(queries[:1], k, F16)
            assert s.last_launch().blocks_x > 8
            assert_same(got_d, got_i, orc.adc_search_f16(centroids, d, codes, queries[:1], k), f"{family} k={k}")


def test_f16_stays_close_to_the_fp32_path(fixture, searcher):
    # the recall delta: the fp16 tables change ranks only where fp32 distances are within table rounding
    centroids, codes, queries = fixture
    searcher.set_tuning(vk.Tuning(queries_per_block=8))
    d16, i16, _ = searcher.search(queries, 10, F16)
    d32, i32, _ = searcher.search(queries, 10, vk.ScanVariant.FusedWarp)
    overlap = np.mean([len(set(i16[q]) & set(i32[q])) / 10 for q in range(NQ)])
    assert overlap >= 0.9, overlap
    assert np.allclose(d16, d32, rtol=2e-3)


def test_f16_rejects_what_v8_rejects(searcher, fixture):
    _, _, queries = fixture
    for k in (0, 129):
        with pytest.raises(vk.VkError):
            searcher.search(queries[:1], k, F16)
    with pytest.raises(vk.VkError):
        searcher.distances(queries[:1], F16)
