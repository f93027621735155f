"""The product's CPU code in libveckern_cpu against the reference's CPU path.

  - ProductQuantizer::train must return the reference's codebook bit for bit for the same (x, n, iters, seed): the
    same std::mt19937_64 stream, std::shuffle initialisation, float mean update and empty-cluster re-seeding
    (reference src/cpu/pq.cpp:31-69). Pinned by golden codebooks written from the reference's own compiled code
    (tests/golden/train_kmeans.npz) and, when oracle/_ref is built, by that code live on more shapes and seeds.
  - The CPU search path (veckern/cpu_ref.hpp: compute_lut, adc_scan, select_topk, adc_search; the bench driver's
    "cpu_reference" row) must give the reference's results bit for bit: pinned by the golden fixtures (LUT, ADC
    matrix, top-k for several k, ties, subnormal LUT entries) and by the reference's cpu_ref.cpp live.
"""
import os

import numpy as np
import pytest

from oracle import binding as b
from tests import datagen
from veckern_amd import host

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["clustered_m8.npz", "clustered_m16.npz", "ties_m16.npz", "tiny_diffs.npz"]
needs_ref = pytest.mark.skipif(not b.ref_available(), reason="oracle/_ref not built (reference checkout absent)")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same(got, exp):
    return (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()


def ref_train(x, m, iters, seed):
    n, d = x.shape
    lib = b.ref()
    h = lib.vkref_pq_create(d, m)
    assert h
    try:
        assert lib.vkref_pq_train(h, np.ascontiguousarray(x).ctypes.data, n, iters, seed) == 0
        cent = np.empty((m, 256, d // m), dtype=np.float32)
        lib.vkref_pq_centroids(h, cent.ctypes.data)
    finally:
        lib.vkref_pq_destroy(h)
    return cent


# ---------------------------------------------------------------- training

def test_train_matches_reference_golden_codebooks():
    z = np.load(os.path.join(GOLDEN, "train_kmeans.npz"))
    for j in range(int(z["cases"])):
        x, m, iters, seed = z[f"x{j}"], int(z[f"m{j}"]), int(z[f"iters{j}"]), int(z[f"seed{j}"])
        got = host.pq_train(x, m, iters, seed=seed)
        assert (bits(got) == bits(z[f"centroids{j}"])).all(), f"case {j}: m={m} iters={iters} seed={seed}"


def test_train_reseed_case_really_has_empty_clusters():
    # the golden case with 40 distinct rows: at most 40 clusters can be non-empty after an assignment, so at least
    # 216 re-seeds happen per iteration and the result depends on the random stream's draws in cluster order
    z = np.load(os.path.join(GOLDEN, "train_kmeans.npz"))
    x = z["x1"]
    assert len(np.unique(x, axis=0)) == 40 and int(z["iters1"]) >= 1


@needs_ref
@pytest.mark.parametrize("n,d,m,iters,seed", [(300, 16, 4, 1, 1), (1000, 32, 8, 5, 7), (2000, 64, 16, 4, 123),
                                              (257, 8, 1, 3, 2), (5000, 128, 16, 2, 1)])
def test_train_equals_reference_live(n, d, m, iters, seed):
    x = datagen.mixture(n, d, 30, 0.3, seed)
    assert (bits(host.pq_train(x, m, iters, seed=seed)) == bits(ref_train(x, m, iters, seed))).all()


@needs_ref
def test_train_with_repeated_rows_equals_reference_live():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((25, 16)).astype(np.float32)[rng.integers(0, 25, size=1000)]
    for seed in (1, 2, 99):
        assert (bits(host.pq_train(x, 4, 3, seed=seed)) == bits(ref_train(x, 4, 3, seed))).all()


def test_train_seed_changes_the_codebook():
    x = datagen.mixture(600, 16, 20, 0.3, 5)
    assert not (host.pq_train(x, 4, 2, seed=1) == host.pq_train(x, 4, 2, seed=2)).all()


# ---------------------------------------------------------------- the CPU search path

@pytest.mark.parametrize("name", FIXTURES)
def test_cpu_search_matches_reference_golden(name):
    z = np.load(os.path.join(GOLDEN, name))
    d = int(z["d"])
    lut = host.compute_lut(z["centroids"], z["queries"])
    assert (bits(lut) == bits(z["lut"])).all()
    dists = host.adc_scan(lut, z["codes"])
    assert (bits(dists) == bits(z["dists"])).all()
    for key in z.files:
        if not (key.startswith("search_k") and key.endswith("_id")):
            continue
        k = int(key[len("search_k"):-3])
        exp = {"id": z[f"search_k{k}_id"], "dist": z[f"search_k{k}_dist"]}
        assert same(host.adc_search(z["centroids"], z["codes"], z["queries"], k), exp), f"{name} search k={k}"
        exp = {"id": z[f"select_k{k}_id"], "dist": z[f"select_k{k}_dist"]}
        assert same(host.select_topk(z["dists"], k), exp), f"{name} select k={k}"
        assert d == z["queries"].shape[1]


@needs_ref
@pytest.mark.parametrize("family", ["pq", "random", "ties"])
@pytest.mark.parametrize("k", [1, 10, 100])
def test_cpu_search_equals_reference_live(family, k):
    n, d, m, nq = 5_003, 64, 16, 23
    maker = {"pq": datagen.pq_fixture, "random": datagen.random_fixture, "ties": datagen.tie_fixture}[family]
    centroids, codes, queries = maker(n, d, m, nq, seed=31)
    rpq = b.RefPQ(centroids, d)
    try:
        exp = rpq.adc_search(rpq.remap_codes(codes), queries, k)
    finally:
        rpq.close()
    assert same(host.adc_search(centroids, codes, queries, k), exp)


@needs_ref
def test_cpu_search_pads_like_the_reference_when_k_exceeds_n():
    centroids, codes, queries = datagen.random_fixture(37, 32, 8, 5, seed=2)
    rpq = b.RefPQ(centroids, 32)
    try:
        exp = rpq.adc_search(rpq.remap_codes(codes), queries, 45)
    finally:
        rpq.close()
    got = host.adc_search(centroids, codes, queries, 45)
    assert same(got, exp)
    assert (got["id"][:, 37:] == -1).all() and np.isinf(got["dist"][:, 37:]).all()


def test_cpu_search_staged_equals_fused():
    # reference tests/test_cpu.cpp:84-94: LUT + scan + select gives the fused search's results
    centroids, codes, queries = datagen.pq_fixture(3_001, 32, 8, 9, seed=4)
    staged = host.select_topk(host.adc_scan(host.compute_lut(centroids, queries), codes), 17)
    assert same(staged, host.adc_search(centroids, codes, queries, 17))


def test_cpu_search_equals_the_oracle():
    centroids, codes, queries = datagen.tie_fixture(4_099, 64, 16, 13, seed=8)
    for k in (1, 64, 128):
        assert same(host.adc_search(centroids, codes, queries, k), b.adc_search(centroids, 64, codes, queries, k))
