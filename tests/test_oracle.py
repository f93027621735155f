"""Pins the oracle (oracle/vk_oracle.c) before it is trusted as the GPU path's checker.

Each oracle function is checked four ways:
  1. against golden fixtures written from the reference's own compiled CPU code (tests/golden/*.npz);
  2. against that code live (oracle/_ref/libvkref.so), bit for bit, on more seeds and shapes, when it is built;
  3. against independent computations: numpy float32 element-wise arithmetic for the LUT and the scan, a full
     lexicographic sort for top-k, Python sets for recall, and the reference's invariants (ADC equals the exact
     distance to the decoded vector; staged LUT + scan + select equals the fused search);
  4. planted mistakes (a dropped term, a swapped pair, an off-by-one id) must fail those same comparisons.
"""
import glob
import os

import numpy as np
import pytest

from oracle import binding as b

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["clustered_m8.npz", "clustered_m16.npz", "ties_m16.npz", "tiny_diffs.npz"]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def load(name):
    return np.load(os.path.join(GOLDEN, name))


# ---------------------------------------------------------------- 1. golden fixtures from the reference

@pytest.mark.parametrize("name", FIXTURES)
def test_lut_and_scan_match_golden(name):
    z = load(name)
    d = int(z["d"])
    lut = b.compute_lut(z["centroids"], d, z["codes"].shape[1], z["queries"])
    assert (bits(lut) == bits(z["lut"])).all()
    dists = b.adc_scan(lut, z["codes"])
    assert (bits(dists) == bits(z["dists"])).all()


@pytest.mark.parametrize("name", FIXTURES)
def test_search_and_select_match_golden(name):
    z = load(name)
    d = int(z["d"])
    for key in z.files:
        if not key.startswith("search_k") or not key.endswith("_id"):
            continue
        k = int(key[len("search_k"):-3])
        got = b.adc_search(z["centroids"], d, z["codes"], z["queries"], k)
        assert (got["id"] == z[f"search_k{k}_id"]).all() and (bits(got["dist"]) == bits(z[f"search_k{k}_dist"])).all()
        sel = b.select_topk(z["dists"], k)
        assert (sel["id"] == z[f"select_k{k}_id"]).all() and (bits(sel["dist"]) == bits(z[f"select_k{k}_dist"])).all()


def test_topk_known_answer():
    # reference tests/test_cpu.cpp:33-46: the tie on 1.0 is broken by id; missing results pad as {inf, -1}
    z = load("topk_kat.npz")
    top3 = b.topk_run(z["values"], z["ids"], 3)
    assert list(top3["id"]) == [1, 3, 4] == list(z["top3_id"])
    pad = b.topk_run(np.array([2.0], np.float32), np.array([9], np.int32), 4)
    assert list(pad["id"]) == list(z["pad_id"]) == [9, -1, -1, -1]
    assert np.isinf(pad["dist"][1:]).all() and (bits(pad["dist"]) == bits(z["pad_dist"])).all()


def test_recall_known_answer():
    z = load("recall_kat.npz")
    found = np.zeros(z["found_id"].shape, dtype=b.NEIGHBOR)
    found["id"] = z["found_id"]
    for k in (1, 2, 3, 4):
        assert b.recall_at_k(found, z["truth"], k) == float(z[f"recall_k{k}"])


def test_every_golden_file_is_checked():
    names = {os.path.basename(p) for p in glob.glob(os.path.join(GOLDEN, "*.npz"))}
    assert names == set(FIXTURES) | {"topk_kat.npz", "recall_kat.npz"}


# ---------------------------------------------------------------- 2. the reference's compiled CPU code, live

needs_ref = pytest.mark.skipif(not b.ref_available(), reason="oracle/_ref not built (reference checkout absent)")


def random_case(seed, n, d, m, nq, family):
    rng = np.random.default_rng(seed)
    if family == "ties":
        cent = rng.integers(0, 3, size=(m, 256, d // m)).astype(np.float32)
        queries = rng.integers(0, 3, size=(nq, d)).astype(np.float32)
    else:
        cent = rng.standard_normal((m, 256, d // m)).astype(np.float32)
        queries = rng.standard_normal((nq, d)).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    return cent, codes, queries


@needs_ref
@pytest.mark.parametrize("seed,n,d,m,nq", [(1, 3000, 32, 4, 6), (2, 2500, 64, 8, 5), (3, 4000, 128, 16, 4),
                                           (4, 1000, 128, 32, 3), (5, 700, 128, 64, 2)])
@pytest.mark.parametrize("family", ["normal", "ties"])
def test_oracle_equals_reference_live(seed, n, d, m, nq, family):
    cent, codes, queries = random_case(seed, n, d, m, nq, family)
    rpq = b.RefPQ(cent, d)
    codes_ref = rpq.remap_codes(codes)
    lut_ref = rpq.compute_lut(queries)
    lut = b.compute_lut(cent, d, m, queries)
    for s in range(m):
        assert (bits(lut[:, s, rpq.perm[s]]) == bits(lut_ref[:, s, :])).all()
    for k in (1, 10, 64, 128, n + 5):  # k > n pads with {inf, -1}
        exp = rpq.adc_search(codes_ref, queries, k)
        got = b.adc_search(cent, d, codes, queries, k)
        assert (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()


@needs_ref
def test_topk_equals_reference_on_random_streams():
    rng = np.random.default_rng(9)
    for trial in range(50):
        count = int(rng.integers(0, 400))
        vals = rng.integers(0, 20, size=count).astype(np.float32)  # many ties
        ids = rng.permutation(count).astype(np.int32)
        k = int(rng.integers(1, 64))
        a, r = b.topk_run(vals, ids, k), b.topk_run(vals, ids, k, use_ref=True)
        assert (a["id"] == r["id"]).all() and (bits(a["dist"]) == bits(r["dist"])).all()


@needs_ref
def test_recall_equals_reference_on_random_rows():
    rng = np.random.default_rng(10)
    for trial in range(30):
        nq, stride = int(rng.integers(1, 20)), int(rng.integers(1, 12))
        found = np.zeros((nq, stride), dtype=b.NEIGHBOR)
        found["id"] = rng.integers(-1, 8, size=(nq, stride))
        truth = rng.integers(-1, 8, size=(nq, stride)).astype(np.int32)
        for k in range(0, stride + 1):
            exp = b.ref().vkref_recall_at_k(found.ctypes.data, stride, truth.ctypes.data, stride, nq, k)
            assert b.recall_at_k(found, truth, k) == exp


# ---------------------------------------------------------------- 3. independent computations

def numpy_lut(cent, queries):
    """Element-wise float32 numpy: diff, square, add, in sub-dimension order (no fused multiply-add)."""
    m, ksub, dsub = cent.shape
    q = queries.reshape(queries.shape[0], m, 1, dsub)
    acc = np.zeros((queries.shape[0], m, ksub), dtype=np.float32)
    for j in range(dsub):
        diff = (q[:, :, :, j] - cent[None, :, :, j]).astype(np.float32)
        acc = (acc + (diff * diff).astype(np.float32)).astype(np.float32)
    return acc


def numpy_scan(lut, codes):
    acc = np.zeros((lut.shape[0], codes.shape[0]), dtype=np.float32)
    for s in range(codes.shape[1]):
        acc = (acc + lut[:, s, codes[:, s]]).astype(np.float32)
    return acc


def sorted_topk(dists, k):
    nq, n = dists.shape
    out = np.zeros((nq, k), dtype=b.NEIGHBOR)
    out["dist"], out["id"] = np.inf, -1
    for q in range(nq):
        order = np.lexsort((np.arange(n), dists[q]))[:k]
        out[q, :len(order)]["dist"] = dists[q, order]
        out[q, :len(order)]["id"] = order
    return out


@pytest.mark.parametrize("family", ["normal", "ties"])
def test_lut_and_scan_equal_numpy_float32(family):
    cent, codes, queries = random_case(21, 5000, 64, 16, 4, family)
    lut = b.compute_lut(cent, 64, 16, queries)
    assert (bits(lut) == bits(numpy_lut(cent, queries))).all()
    assert (bits(b.adc_scan(lut, codes)) == bits(numpy_scan(lut, codes))).all()


@pytest.mark.parametrize("k", [1, 7, 64, 300])
def test_select_equals_full_sort(k):
    cent, codes, queries = random_case(22, 3000, 32, 8, 5, "ties")
    dists = b.adc_scan(b.compute_lut(cent, 32, 8, queries), codes)
    got, exp = b.select_topk(dists, k), sorted_topk(dists, k)
    assert (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()


def test_staged_equals_fused():
    # reference tests/test_cpu.cpp:84-94
    cent, codes, queries = random_case(23, 4000, 64, 16, 6, "normal")
    staged = b.select_topk(b.adc_scan(b.compute_lut(cent, 64, 16, queries), codes), 10)
    fused = b.adc_search(cent, 64, codes, queries, 10)
    assert (staged["id"] == fused["id"]).all() and (bits(staged["dist"]) == bits(fused["dist"])).all()


def test_adc_equals_distance_to_decoded_vector():
    # reference tests/test_cpu.cpp:58-67
    cent, codes, queries = random_case(24, 2000, 64, 16, 5, "normal")
    dists = b.adc_scan(b.compute_lut(cent, 64, 16, queries), codes)
    decoded = np.concatenate([cent[s][codes[:, s]] for s in range(16)], axis=1).astype(np.float64)
    exact = ((queries.astype(np.float64)[:, None, :] - decoded[None, :, :]) ** 2).sum(-1)
    assert np.allclose(dists, exact, rtol=1e-5, atol=1e-3)


def test_recall_equals_set_formula():
    rng = np.random.default_rng(25)
    found = np.zeros((40, 10), dtype=b.NEIGHBOR)
    found["id"] = rng.integers(-1, 30, size=(40, 10))
    truth = rng.integers(-1, 30, size=(40, 12)).astype(np.int32)
    for k in (1, 5, 10):
        exp = np.mean([sum(i in set(truth[q, :k]) for i in found["id"][q, :k]) / k for q in range(40)])
        assert abs(b.recall_at_k(found, truth, k) - exp) < 1e-12
    assert b.recall_at_k(found, truth, 11) == -1.0  # k beyond a stride is an error (the reference throws)


# ---------------------------------------------------------------- 4. planted mistakes are caught

def test_planted_mistakes_fail_the_checks():
    z = load("clustered_m16.npz")
    d = int(z["d"])
    lut = b.compute_lut(z["centroids"], d, 16, z["queries"])
    # a dropped sub-space term
    dropped = np.zeros((lut.shape[0], z["codes"].shape[0]), dtype=np.float32)
    for s in range(15):
        dropped = (dropped + lut[:, s, z["codes"][:, s]]).astype(np.float32)
    assert not (bits(dropped) == bits(z["dists"])).all()
    # transposed sub-vector (wrong centroid index order)
    assert not (bits(b.compute_lut(z["centroids"][:, ::-1].copy(), d, 16, z["queries"])) == bits(z["lut"])).all()
    # an FMA-style rounding of the LUT (one rounding for diff*diff + acc) differs somewhere
    c64, q64 = z["centroids"].astype(np.float64), z["queries"].astype(np.float64)
    m, _, dsub = z["centroids"].shape
    acc = np.zeros(lut.shape, dtype=np.float32)
    for j in range(dsub):
        diff = (z["queries"].reshape(-1, m, 1, dsub)[..., j] - z["centroids"][None, :, :, j]).astype(np.float32)
        acc = (acc.astype(np.float64) + diff.astype(np.float64) ** 2).astype(np.float32)
    assert not (bits(acc) == bits(z["lut"])).all()
    # ties broken the wrong way (by descending id) change the selected ids
    t = load("ties_m16.npz")
    wrong = sorted_topk(-t["dists"], 16)
    assert not (wrong["id"] == t["select_k16_id"]).all()
    # an off-by-one id
    good = b.adc_search(z["centroids"], d, z["codes"], z["queries"], 10)
    assert not ((good["id"] + 1) == z["search_k10_id"]).all()
    del c64, q64
