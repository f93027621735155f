"""GPU exact re-ranking (vk_rerank / vk_rerank_device, the reference's rerank_exact, cpu_ref.cpp:66-77) against
the oracle's restatement, bit-exact: distances summed in dimension order without FMA, ids under the (dist, id)
order. Covers r below, at and above one wave (64), every K template, -1 padding, duplicated ids, d not a
multiple of 4, the device entry point, the search -> re-rank pipeline, and out-of-range ids (an error).
"""
import numpy as np
import pytest

import veckern_amd as vk
from tests import datagen
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def case(seed, n, d, nq, r, family="normal"):
    rng = np.random.default_rng(seed)
    if family == "ties":
        base = rng.integers(0, 3, size=(n, d)).astype(np.float32)
        queries = rng.integers(0, 3, size=(nq, d)).astype(np.float32)
    else:
        base = rng.standard_normal((n, d)).astype(np.float32)
        queries = rng.standard_normal((nq, d)).astype(np.float32)
    cand = np.zeros((nq, r), dtype=vk.NEIGHBOR_DTYPE)
    cand["id"] = rng.integers(-1, n, size=(nq, r))
    if r >= 6:
        cand["id"][:, :3] = cand["id"][:, 3:6]
    return base, queries, cand


def assert_same(got_d, got_i, exp, label=""):
    bad = np.argwhere((got_i != exp["id"]) | (got_d.view(np.uint32) != exp["dist"].view(np.uint32)))
    if bad.size:
        q, j = bad[0]
        raise AssertionError(f"{label}: {len(bad)} mismatches; first at query {q} rank {j}: got "
                             f"({got_d[q, j]!r}, {got_i[q, j]}) expected ({exp['dist'][q, j]!r}, {exp['id'][q, j]})")


@pytest.mark.parametrize("r", [1, 10, 64, 100, 129, 1000])
@pytest.mark.parametrize("k", [1, 10, 64, 100, 128])
def test_rerank_matches_oracle(r, k):
    base, queries, cand = case(50 + r, 20_000, 128, 37, r)
    with vk.Reranker(base) as rr:
        d, i, t = rr.rerank(queries, cand, k)
    assert_same(d, i, orc.rerank_exact(base, queries, cand, k), f"r={r} k={k}")
    assert t.scan_ms > 0 and t.transfer_ms > 0


@pytest.mark.parametrize("d", [96, 37, 1])
@pytest.mark.parametrize("family", ["normal", "ties"])
def test_rerank_other_dims_and_ties(d, family):
    base, queries, cand = case(60 + d, 5_000, d, 21, 200, family)
    with vk.Reranker(base) as rr:
        for k in (10, 128):
            got_d, got_i, _ = rr.rerank(queries, cand, k)
            assert_same(got_d, got_i, orc.rerank_exact(base, queries, cand, k), f"d={d} {family} k={k}")


def test_rerank_all_padding_and_empty_batch():
    base, queries, cand = case(70, 1_000, 64, 5, 40)
    cand["id"][:] = -1
    with vk.Reranker(base) as rr:
        d, i, _ = rr.rerank(queries, cand, 10)
        assert (i == -1).all() and np.isinf(d).all()
        d, i, _ = rr.rerank(queries[:0], cand[:0], 10)
        assert d.shape == (0, 10)


def test_rerank_device_entry_point():
    base, queries, cand = case(71, 8_000, 128, 19, 100)
    k = 10
    dq, dc = vk.DeviceArray.from_host(queries), vk.DeviceArray.from_host(cand)
    dout = vk.DeviceArray(19 * k * 8)
    with vk.Reranker(base) as rr:
        t = rr.rerank_device(dq.address, 19, dc.address, 100, k, dout.address)
    out = np.empty((19, k), dtype=vk.NEIGHBOR_DTYPE)
    dout.download(out)
    assert_same(out["dist"], out["id"], orc.rerank_exact(base, queries, cand, k), "device")
    assert t.transfer_ms == 0 and t.scan_ms > 0


def test_search_then_rerank_pipeline():
    # the reference's --rerank R flow: PQ search for R candidates, exact re-rank to k
    n, d, m, nq = 30_011, 64, 16, 23
    centroids, codes, queries = datagen.pq_fixture(n, d, m, nq, seed=12)
    base = datagen.mixture(n + nq, d, 50, 0.3, seed=12)[:n]  # the vectors pq_fixture encoded
    with vk.PQSearcher(centroids, codes, d) as s, vk.Reranker(base) as rr:
        cd, ci, _ = s.search(queries, 100, vk.ScanVariant.FusedWarp)
        cand = np.zeros((nq, 100), dtype=vk.NEIGHBOR_DTYPE)
        cand["dist"], cand["id"] = cd, ci
        got_d, got_i, _ = rr.rerank(queries, cand, 10)
    assert_same(got_d, got_i, orc.rerank_exact(base, queries, cand, 10), "pipeline")


def test_out_of_range_ids_are_an_error_and_never_read():
    base, queries, cand = case(72, 1_000, 32, 4, 30)
    cand["id"][2, 5] = 1_000  # == n
    with vk.Reranker(base) as rr:
        with pytest.raises(vk.VkInvalidArgument):
            rr.rerank(queries, cand, 10)
        for k in (0, 129):
            with pytest.raises(vk.VkError):
                rr.rerank(queries, cand, k)
        # the re-ranker stays usable after an error
        cand["id"][2, 5] = 3
        got_d, got_i, _ = rr.rerank(queries, cand, 10)
        assert_same(got_d, got_i, orc.rerank_exact(base, queries, cand, 10), "after error")
