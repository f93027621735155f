"""GPU parity of the search path through the C ABI: every result must equal the oracle's exactly.

The bar is bit-exact: distances are summed in the same order as the CPU reference (cpu_ref.cpp:46-49) and the
LUT is rounded like it (no FMA), so `dist` arrays must be identical and ids identical under the (dist, id) order
(ties included). Cases follow the reference's tests/test_gpu.cpp: n not a multiple of 64 or of any block size,
a prime query count, every K template, every queries-per-block and ILP setting, tuning overrides.
"""
import numpy as np
import pytest

import veckern_amd as vk
from tests import datagen
from oracle import binding as orc

pytestmark = pytest.mark.gpu

N, D, M, NQ = 50_003, 64, 16, 37  # the reference fixture's shape (test_gpu.cpp:17)


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
        _expected_cache[k] = orc.adc_search(centroids, D, codes, queries, k)
    return _expected_cache[k]


def assert_same(got_d, got_i, exp, label=""):
    assert got_i.shape == exp.shape, label
    bad = np.argwhere((got_i != exp["id"]) | (got_d.view(np.uint32) != exp["dist"].view(np.uint32)))
    if bad.size:
        q, j = bad[0]
        raise AssertionError(f"{label}: {len(bad)} mismatches; first at query {q} rank {j}: "
                             f"got ({got_d[q, j]!r}, {got_i[q, j]}) expected ({exp['dist'][q, j]!r}, {exp['id'][q, j]})")


def test_device_info_is_sane():
    info = vk.device_info()
    print(f"\n    {info.name} {info.arch}: {info.sm_count} CUs, {info.peak_bandwidth_gbs:.0f} GB/s, "
          f"{info.max_smem_per_block} B LDS/block, {info.clock_khz / 1e6:.2f} GHz")
    assert info.sm_count > 0 and info.peak_bandwidth_gbs > 0 and info.max_smem_per_block >= 65536
    assert info.warp_size == 64


@pytest.mark.parametrize("k", [1, 8, 10, 16, 33, 64, 100, 128])
def test_fused_warp_every_k(fixture, searcher, k):
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning())
    d, i, t = searcher.search(queries, k, vk.ScanVariant.FusedWarp)
    assert_same(d, i, expected(fixture, k), f"v8 k={k}")
    # One launch builds the tables, scans and merges: its whole time is scan_ms.
    assert t.scan_ms > 0 and t.lut_ms == 0 and t.select_ms == 0


@pytest.mark.parametrize("q", [1, 2, 4, 8])
@pytest.mark.parametrize("ilp", [1, 2, 4])
def test_fused_warp_every_q_and_ilp(fixture, searcher, q, ilp):
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning(queries_per_block=q, vectors_per_step=ilp))
    for k in (1, 10, 32, 128):
        d, i, _ = searcher.search(queries, k, vk.ScanVariant.FusedWarp)
        assert_same(d, i, expected(fixture, k), f"v8 Q={q} ILP={ilp} k={k}")
        shape = searcher.last_launch()
        assert shape.queries_per_block == q and shape.vectors_per_step == ilp


@pytest.mark.parametrize("bpq", [1, 3, 7, 16])
def test_fused_warp_blocks_per_query(fixture, searcher, bpq):
    _, _, queries = fixture
    for q in (2, 4):
        searcher.set_tuning(vk.Tuning(blocks_per_query=bpq, queries_per_block=q))
        for k in (1, 10, 33, 128):
            d, i, _ = searcher.search(queries, k, vk.ScanVariant.FusedWarp)
            assert_same(d, i, expected(fixture, k), f"v8 bpq={bpq} Q={q} k={k}")


def test_single_query_spreads_over_the_device(fixture, searcher):
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning(queries_per_block=1))
    d, i, _ = searcher.search(queries[:1], 10, vk.ScanVariant.FusedWarp)
    assert_same(d, i, expected(fixture, 10)[:1], "v8 nq=1")
    s = searcher.last_launch()
    # spread over ceil(n / (16 vectors x 512 threads)) blocks (the reference's rule), at most one per CU
    expected_blocks = min(vk.device_info().sm_count, -(-N // 8192))
    assert s.blocks_x == expected_blocks and s.blocks_x > 1


@pytest.mark.parametrize("family", ["random", "tie"])
def test_long_lists_merge_whole(family):
    # One query over ~20 blocks: each block merges its 8 wave lists, and the last block's 8 waves split the blocks'
    # lists; lists longer than 32 go in whole through the bitonic list merge, shorter ones as 64-pair chunks.
    # k on both sides of 32 and of 64 (one and two list registers); tie-heavy data exercises the id order.
    gen = datagen.random_fixture if family == "random" else datagen.tie_fixture
    n, d, m, nq = 200_003, 32, 16, 3
    centroids, codes, queries = gen(n, d, m, nq, seed=23)
    with vk.PQSearcher(centroids, codes, d) as s:
        s.set_tuning(vk.Tuning(queries_per_block=1))
        for k in (32, 33, 64, 65, 100, 128):
            got_d, got_i, _ = s.search(queries[:1], k, vk.ScanVariant.FusedWarp)
            assert s.last_launch().blocks_x > 8
            assert_same(got_d, got_i, orc.adc_search(centroids, d, codes, queries[:1], k), f"{family} nq=1 k={k}")
            # the three queries in one slab over 3 blocks: a wave of the last block merges each query's 24 lists
            s.set_tuning(vk.Tuning(queries_per_block=4, blocks_per_query=3))
            got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
            assert_same(got_d, got_i, orc.adc_search(centroids, d, codes, queries, k), f"{family} Q=4 k={k}")
            s.set_tuning(vk.Tuning(queries_per_block=1))


@pytest.mark.parametrize("family", ["random", "tie"])
def test_single_query_final_merge_paths(family):
    # One query over many blocks with one-register lists (k <= 64): the last block bounds the k-th best by the k-th
    # smallest list head of each wave's 64 lists and merges only the pairs at or below it. Cases: k=10 over 100
    # lists (a few dozen survivors, one sort); k=33 over 100 lists and k=64 over 30 (no wave has 64 heads, so every
    # real pair survives: more than 64, streamed from LDS); k=64 over 40 (2560 pairs overflow the 16 KB of LDS: the
    # merge of every list). Tie-heavy data checks that pairs equal to the bound and the id order survive the filter.
    gen = datagen.random_fixture if family == "random" else datagen.tie_fixture
    n, d, m, nq = 400_009, 32, 16, 2
    centroids, codes, queries = gen(n, d, m, nq, seed=31)
    with vk.PQSearcher(centroids, codes, d) as s:
        for k, bpq in ((10, 100), (33, 100), (64, 30), (64, 40), (1, 256)):
            s.set_tuning(vk.Tuning(queries_per_block=1, blocks_per_query=bpq))
            got_d, got_i, _ = s.search(queries[:1], k, vk.ScanVariant.FusedWarp)
            assert s.last_launch().blocks_x == bpq
            assert_same(got_d, got_i, orc.adc_search(centroids, d, codes, queries[:1], k), f"{family} k={k} bpq={bpq}")


@pytest.mark.parametrize("variant", [vk.ScanVariant.FusedWarp, vk.ScanVariant.FusedWarpF16])
def test_final_merge_bound_equal_to_the_kth_best(variant):
    # The k best vectors each head a different block's list, so the bound (the k-th smallest head) is the k-th best
    # itself and exactly k pairs survive the filter: the pair equal to the bound must be kept. The 16 planted
    # vectors have first code bytes 16 apart and distances 0.05^2 .. 0.8^2, far below the random vectors' (~60).
    # With 64 and 100 blocks they fall in 16 different blocks of the layout the first search builds for its one-query
    # (4-byte) table reads (checked on the CPU against slot_order.hpp for this data); the default block count is kept
    # as an ordinary parity case.
    rng = np.random.default_rng(17)
    n, d, m = 300_007, 32, 16
    centroids = rng.standard_normal((m, 256, d // m)).astype(np.float32)
    query = rng.standard_normal((1, d)).astype(np.float32)
    codes = rng.integers(0, 255, size=(n, m), dtype=np.uint8)  # 255 is kept for the planted vectors
    planted = rng.choice(n, 16, replace=False)
    sub = query[0].reshape(m, d // m)
    centroids[1:, 255] = sub[1:]
    for j, v in enumerate(planted):
        centroids[0, 16 * j] = sub[0] + np.array([0.05 * (j + 1), 0.0], dtype=np.float32)
        codes[v, 0] = 16 * j
        codes[v, 1:] = 255
    oracle_search = orc.adc_search_f16 if variant == vk.ScanVariant.FusedWarpF16 else orc.adc_search
    with vk.PQSearcher(centroids, codes, d) as s:
        for bpq in (0, 64, 100):
            s.set_tuning(vk.Tuning(queries_per_block=1, blocks_per_query=bpq))
            for k in (10, 16):
                exp = oracle_search(centroids, d, codes, query, k)
                assert set(exp["id"][0]) == set(planted[:k])
                got_d, got_i, _ = s.search(query, k, variant)
                assert s.last_launch().blocks_x > 16
                assert_same(got_d, got_i, exp, f"bpq={bpq} k={k}")


def test_bulk_and_one_by_one_admission_agree():
    # Blocks that scan few vectors of a slab use the instance admitting candidates in bulk; above 2^18 vectors per
    # block and slab the one admitting them one by one (the headline's). 300k vectors with one block per slab take
    # the second, the default spread (~8k vectors per block) the first; both must equal the oracle.
    n, d, m, nq = 300_007, 64, 16, 9
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=41)
    with vk.PQSearcher(centroids, codes, d) as s:
        for k in (1, 10, 64):
            exp = orc.adc_search(centroids, d, codes, queries, k)
            for q in (2, 4, 8):
                slabs = -(-nq // q)
                for bpq in (1, 0):
                    s.set_tuning(vk.Tuning(queries_per_block=q, blocks_per_query=bpq))
                    got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
                    assert_same(got_d, got_i, exp, f"k={k} Q={q} bpq={bpq}")
                    blocks = s.last_launch().blocks_x
                    assert (blocks == slabs) if bpq == 1 else (blocks > 4 * slabs)


@pytest.mark.parametrize("family", ["random", "tie"])
@pytest.mark.parametrize("m", [16, 32, 64])
def test_fused_warp_other_m_and_tie_heavy_data(family, m):
    gen = datagen.random_fixture if family == "random" else datagen.tie_fixture
    n, d, nq = 20_011, 128, 13
    centroids, codes, queries = gen(n, d, m, nq, seed=5 + m)
    with vk.PQSearcher(centroids, codes, d) as s:
        for q in (1, 2, 4, 8):
            s.set_tuning(vk.Tuning(queries_per_block=q))
            for k in (10, 100):
                got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
                exp = orc.adc_search(centroids, d, codes, queries, k)
                assert_same(got_d, got_i, exp, f"{family} m={m} Q={q} k={k}")


def test_admission_bursts_from_falling_distances():
    # The scan visits vectors sorted by their first code bytes. Here sub-space 0 dominates every distance and falls
    # as its code rises, so along the scan nearly every tile beats the lists' thresholds: tiles admit a few lanes,
    # many lanes, or all 64, the lists' admission queues fill and overflow mid-granule, and whole tiles merge at once.
    # A small second query mixes in the usual sparse admissions. Both must equal the oracle at every list length.
    rng = np.random.default_rng(23)
    n, d, m, nq = 60_013, 32, 16, 11
    dsub = d // m
    centroids = rng.standard_normal((m, 256, dsub)).astype(np.float32)
    centroids[0, :, 0] = np.arange(256, dtype=np.float32)
    centroids[0, :, 1] = 0.0
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    queries[: nq - 1, 0] = 1000.0  # (1000 - c)^2 falls with the sub-space-0 code c, in steps of ~1500
    queries[:, 1] = 0.0  # the other sub-spaces add ~30 of noise, distinct values within a step
    with vk.PQSearcher(centroids, codes, d) as s:
        for k in (1, 10, 64, 100, 128):
            exp = orc.adc_search(centroids, d, codes, queries, k)
            for q in (1, 2, 4, 8):
                s.set_tuning(vk.Tuning(queries_per_block=q))
                got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
                assert_same(got_d, got_i, exp, f"falling k={k} Q={q}")


def test_generic_m_path():
    # m = 48 is not one of the compile-time specialisations; the kernel reads m at run time.
    n, d, m, nq = 9_001, 96, 48, 9
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=3)
    with vk.PQSearcher(centroids, codes, d) as s:
        for q in (1, 2):
            s.set_tuning(vk.Tuning(queries_per_block=q))
            got_d, got_i, _ = s.search(queries, 10, vk.ScanVariant.FusedWarp)
            assert_same(got_d, got_i, orc.adc_search(centroids, d, codes, queries, 10), f"m=48 Q={q}")


def test_tiny_database_and_k_equal_n():
    n, d, m, nq = 70, 32, 16, 5
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=9)
    with vk.PQSearcher(centroids, codes, d) as s:
        for k in (1, 64, 70):
            got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
            assert_same(got_d, got_i, orc.adc_search(centroids, d, codes, queries, k), f"n=70 k={k}")


@pytest.mark.parametrize("n", [1, 255, 256, 257, 768, 769, 4_160])
def test_layout_block_boundaries(n):
    # The sorted layout deals and spreads only full 256-slot blocks; a partial last block keeps its slots at the end,
    # and padding slots up to the next 256 are never read as vectors. Sizes around those boundaries, every k kind.
    d, m, nq = 32, 16, 3
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=n)
    with vk.PQSearcher(centroids, codes, d) as s:
        for k in sorted({1, min(10, n), n if n <= 128 else 128}):
            got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarp)
            assert_same(got_d, got_i, orc.adc_search(centroids, d, codes, queries, k), f"v8 n={n} k={k}")
            got_d, got_i, _ = s.search(queries, k, vk.ScanVariant.FusedWarpF16)
            assert_same(got_d, got_i, orc.adc_search_f16(centroids, d, codes, queries, k), f"v9 n={n} k={k}")


def test_device_resident_entry_point(fixture, searcher):
    _, _, queries = fixture
    searcher.set_tuning(vk.Tuning(queries_per_block=4))
    k = 10
    dq = vk.DeviceArray.from_host(queries)
    dout = vk.DeviceArray(NQ * k * 8)
    t = searcher.search_device(dq.address, NQ, k, vk.ScanVariant.FusedWarp, dout.address)
    out = np.empty((NQ, k), dtype=vk.NEIGHBOR_DTYPE)
    dout.download(out)
    assert_same(out["dist"], out["id"], expected(fixture, k), "device entry")
    assert t.transfer_ms == 0 and t.scan_ms > 0


def test_invalid_k_is_rejected(searcher, fixture):
    _, _, queries = fixture
    for k in (0, 129):
        with pytest.raises(vk.VkError):
            searcher.search(queries[:1], k, vk.ScanVariant.FusedWarp)


def test_batches_beyond_one_launch():
    # more queries than one launch takes (65,535): two batches through the same searcher, per-slab counters and
    # partial-list buffers reused; every result must still be exact
    n, d, m, nq = 1_201, 32, 16, 65_535 + 4_000
    centroids, codes, queries = datagen.random_fixture(n, d, m, nq, seed=31)
    with vk.PQSearcher(centroids, codes, d) as s:
        s.set_tuning(vk.Tuning(queries_per_block=4))
        got_d, got_i, _ = s.search(queries, 10, vk.ScanVariant.FusedWarp)
    exp = orc.adc_search(centroids, d, codes, queries, 10)
    assert_same(got_d, got_i, exp, "two batches")
