"""GPU inverted-file search (vk_ivf_*) against the oracle's restatement (vko_ivf_search), bit-exact: coarse probe
by exact distances (ties to the lower list id), then the exhaustive search's ADC distances and (dist, id) order
over the probed lists only. Covers nprobe = 1 .. nlist (all lists = the exhaustive search), every K template,
empty and tiny lists, a query whose lists span many blocks, blocks that finish many queries, tie-heavy data and a
run-time m.
"""
import numpy as np
import pytest

import veckern_amd as vk
from tests import datagen
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def ivf_case(seed, n, d, m, nq, nlist, family="random", empty_lists=0):
    gen = datagen.random_fixture if family == "random" else datagen.tie_fixture
    centroids, codes, queries = gen(n, d, m, nq, seed=seed)
    rng = np.random.default_rng(seed + 7)
    coarse = rng.standard_normal((nlist, d)).astype(np.float32)
    list_ids = rng.integers(0, nlist - empty_lists, size=n).astype(np.int32)  # the last lists stay empty
    return coarse, centroids, codes, list_ids, queries


def assert_same(got_d, got_i, exp, label=""):
    bad = np.argwhere((got_i != exp["id"]) | (got_d.view(np.uint32) != exp["dist"].view(np.uint32)))
    if bad.size:
        q, j = bad[0]
        raise AssertionError(f"{label}: {len(bad)} mismatches; first at query {q} rank {j}: got "
                             f"({got_d[q, j]!r}, {got_i[q, j]}) expected ({exp['dist'][q, j]!r}, {exp['id'][q, j]})")


@pytest.fixture(scope="module")
def index_case():
    case = ivf_case(90, 60_013, 64, 16, 37, 64, empty_lists=3)
    coarse, cent, codes, list_ids, queries = case
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        yield case, ix


@pytest.mark.parametrize("nprobe", [1, 4, 16, 64])
@pytest.mark.parametrize("k", [1, 10, 100])
def test_ivf_matches_oracle(index_case, nprobe, k):
    (coarse, cent, codes, list_ids, queries), ix = index_case
    ix.set_tuning(vk.Tuning(queries_per_block=4))
    d, i, t = ix.search(queries, nprobe, k)
    assert_same(d, i, orc.ivf_search(coarse, cent, 64, codes, list_ids, queries, nprobe, k), f"nprobe={nprobe} k={k}")
    assert t.scan_ms > 0 and t.lut_ms > 0 and t.select_ms > 0


def test_ivf_all_lists_is_the_exhaustive_search(index_case):
    (coarse, cent, codes, list_ids, queries), ix = index_case
    d, i, _ = ix.search(queries, 64, 10)
    assert_same(d, i, orc.adc_search(cent, 64, codes, queries, 10), "nprobe=nlist")


@pytest.mark.parametrize("q", [1, 2, 4])
def test_ivf_takes_one_query_per_slab_whatever_the_tuning(index_case, q):
    (coarse, cent, codes, list_ids, queries), ix = index_case
    ix.set_tuning(vk.Tuning(queries_per_block=q))
    d, i, _ = ix.search(queries, 8, 33)
    assert_same(d, i, orc.ivf_search(coarse, cent, 64, codes, list_ids, queries, 8, 33), f"Q={q}")
    assert ix.last_launch().queries_per_block == 1


def test_ivf_blocks_finish_many_queries():
    # ~100 vectors per list (one granule each), 3000 queries x 2 probes: each block's range holds the runs of
    # several queries, so lists are written and restarted inside a block; k = 100 exercises the long lists
    coarse, cent, codes, list_ids, queries = ivf_case(96, 20_000, 32, 16, 3_000, 200)
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        for k in (10, 100):
            d, i, _ = ix.search(queries, 2, k)
            assert_same(d, i, orc.ivf_search(coarse, cent, 32, codes, list_ids, queries, 2, k), f"k={k}")
            assert ix.last_launch().blocks_x < 3_000 * 2


def test_ivf_plan_with_many_slabs():
    # 3000 queries x 32 probes = 96,000 slabs (the plan's prefix over queries runs in one block, its slab offsets in
    # one thread per slab), against 3000 x 2.
    coarse, cent, codes, list_ids, queries = ivf_case(97, 20_000, 32, 16, 3_000, 200)
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        for nprobe in (32, 2):
            d, i, _ = ix.search(queries, nprobe, 10)
            assert_same(d, i, orc.ivf_search(coarse, cent, 32, codes, list_ids, queries, nprobe, 10), f"nprobe={nprobe}")


def test_ivf_single_query_spreads_lists_over_many_blocks(index_case):
    (coarse, cent, codes, list_ids, queries), ix = index_case
    ix.set_tuning(vk.Tuning(queries_per_block=4))
    d, i, _ = ix.search(queries[:1], 3, 10)
    assert_same(d, i, orc.ivf_search(coarse, cent, 64, codes, list_ids, queries[:1], 3, 10), "nq=1")


@pytest.mark.parametrize("family", ["random", "tie"])
@pytest.mark.parametrize("m", [32, 64])
def test_ivf_other_m_and_ties(family, m):
    coarse, cent, codes, list_ids, queries = ivf_case(91 + m, 20_011, 128, m, 13, 20, family)
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        for nprobe, k in ((2, 10), (7, 128)):
            d, i, _ = ix.search(queries, nprobe, k)
            assert_same(d, i, orc.ivf_search(coarse, cent, 128, codes, list_ids, queries, nprobe, k),
                        f"{family} m={m} nprobe={nprobe} k={k}")


def test_ivf_generic_m_and_tiny_lists():
    coarse, cent, codes, list_ids, queries = ivf_case(95, 3_001, 96, 48, 9, 500)  # ~6 vectors per list
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        for nprobe in (1, 5, 128):
            d, i, _ = ix.search(queries, nprobe, 10)
            assert_same(d, i, orc.ivf_search(coarse, cent, 96, codes, list_ids, queries, nprobe, 10),
                        f"m=48 nprobe={nprobe}")


def test_ivf_rejects_bad_arguments(index_case):
    (coarse, cent, codes, list_ids, queries), ix = index_case
    for nprobe, k in ((0, 10), (65, 10), (4, 0), (4, 129)):
        with pytest.raises(vk.VkError):
            ix.search(queries, nprobe, k)
    bad = list_ids.copy()
    bad[5] = 64
    with pytest.raises(vk.VkError):
        vk.IVFIndex(coarse, cent, codes, bad)


def test_ivf_assign_is_the_nearest_coarse_centroid():
    rng = np.random.default_rng(97)
    coarse = rng.standard_normal((300, 64)).astype(np.float32)
    coarse[150] = coarse[20]  # a duplicated centroid: the lower index wins
    x = rng.standard_normal((10_007, 64)).astype(np.float32)
    x[:50] = coarse[20]       # exact hits on the duplicated centroid
    got = vk.ivf_assign(coarse, x)
    cand = np.zeros((x.shape[0], 300), dtype=vk.NEIGHBOR_DTYPE)
    cand["id"] = np.arange(300)
    exp = orc.rerank_exact(coarse, x, cand, 1)["id"][:, 0]
    assert (got == exp).all() and (got[:50] == 20).all()


@pytest.mark.parametrize("nlist,d,n", [(1, 8, 33), (70, 100, 4_099), (129, 130, 31)])
def test_ivf_assign_on_ragged_tiles(nlist, d, n):
    """Centroid counts and dimensions that are not whole 64-wide tiles or slices, fewer vectors than one 32-row
    tile, duplicated centroids in different tiles (the lower index wins) and a vector of NaNs (list 0)."""
    rng = np.random.default_rng(nlist * 1000 + d)
    coarse = rng.standard_normal((nlist, d)).astype(np.float32)
    if nlist > 65:
        coarse[nlist - 1] = coarse[3]
    x = rng.standard_normal((n, d)).astype(np.float32)
    if nlist > 65:
        x[: min(n, 7)] = coarse[3]
    x[n // 2] = np.nan
    got = vk.ivf_assign(coarse, x)
    cand = np.zeros((n, nlist), dtype=vk.NEIGHBOR_DTYPE)
    cand["id"] = np.arange(nlist)
    exp = orc.rerank_exact(coarse, x, cand, 1)["id"][:, 0]
    keep = np.arange(n) != n // 2
    assert (got[keep] == exp[keep]).all()
    assert got[n // 2] == 0
    if nlist > 65:
        assert (got[: min(n, 7)] == 3).all()


def test_ivf_device_resident_search_matches_host_buffers(index_case):
    (coarse, cent, codes, list_ids, queries), ix = index_case
    nq, k = queries.shape[0], 10
    dq = vk.DeviceArray.from_host(np.ascontiguousarray(queries, dtype=np.float32))
    dout = vk.DeviceArray(nq * k * vk.NEIGHBOR_DTYPE.itemsize)
    try:
        t = ix.search_device(dq.address, nq, 16, k, dout.address)
        got = dout.download(np.empty((nq, k), dtype=vk.NEIGHBOR_DTYPE))
    finally:
        dq.free()
        dout.free()
    assert t.transfer_ms == 0 and t.scan_ms > 0
    assert_same(got["dist"], got["id"], orc.ivf_search(coarse, cent, 64, codes, list_ids, queries, 16, k), "device")


def test_ivf_probe_ties_go_to_the_lower_list():
    # duplicated coarse centroids and queries sitting exactly on them: equal probe distances, the lower list id
    # must be probed first (the reference's (dist, id) order); also d not a multiple of the probe's 32-wide slices
    coarse, cent, codes, list_ids, queries = ivf_case(98, 8_003, 48, 16, 70, 40)
    coarse[7] = coarse[3]
    coarse[31] = coarse[3]
    queries[:10] = coarse[3]
    queries[10:20] = coarse[12]
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        for nprobe in (1, 2, 3):
            d, i, _ = ix.search(queries, nprobe, 10)
            assert_same(d, i, orc.ivf_search(coarse, cent, 48, codes, list_ids, queries, nprobe, 10),
                        f"probe ties nprobe={nprobe}")


def test_ivf_probe_over_many_lists():
    # 2,048 coarse centroids: the probe's distance rows are whole 1024-wide rounds of the row select
    coarse, cent, codes, list_ids, queries = ivf_case(99, 30_011, 32, 16, 45, 2048)
    with vk.IVFIndex(coarse, cent, codes, list_ids) as ix:
        for nprobe, k in ((1, 10), (40, 100)):
            d, i, _ = ix.search(queries, nprobe, k)
            assert_same(d, i, orc.ivf_search(coarse, cent, 32, codes, list_ids, queries, nprobe, k),
                        f"nlist=2048 nprobe={nprobe} k={k}")
