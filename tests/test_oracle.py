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
    # train_kmeans.npz pins the product's PQ trainer (tests/test_cpu_path.py); the oracle has no trainer
    names = {os.path.basename(p) for p in glob.glob(os.path.join(GOLDEN, "*.npz"))}
    assert names == set(FIXTURES) | {"topk_kat.npz", "recall_kat.npz", "train_kmeans.npz"}


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


# ---------------------------------------------------------------- 5. the fp16-table search (FusedWarpF16)

def _same_f32(got, exp):
    """Bit equality, with any NaN matching any NaN (payloads are not specified by the format)."""
    gn, en = np.isnan(got), np.isnan(exp)
    return (gn == en).all() and (bits(got)[~gn] == bits(exp)[~en]).all()


def test_f16_to_f32_matches_numpy_for_every_binary16_value():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    assert _same_f32(b.f16_bits_to_f32(h), h.view(np.float16).astype(np.float32))


def test_f32_to_f16_matches_numpy_round_to_nearest_even():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(vals)
    # every binary16 value converts back to itself
    assert (b.f32_to_f16_bits(vals[finite]) == h[finite]).all()
    # every midpoint between neighbouring finite values (exact in f32), and one f32 ulp either side of it
    pos = np.sort(vals[finite & (vals >= 0)]).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    probe = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
                            np.float32([65504, 65519.996, 65520, 65536, 1e9, 2.0**-24, 2.0**-25, 3 * 2.0**-26,
                                        2.0**-26, 1e-30, 0.0])])
    probe = np.concatenate([probe, -probe])
    with np.errstate(over="ignore"):
        exp = probe.astype(np.float16).view(np.uint16)
    assert (b.f32_to_f16_bits(probe) == exp).all()
    # random bit patterns over the whole f32 range
    rnd = np.random.default_rng(31).integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        exp = rnd.astype(np.float16)
    got = b.f32_to_f16_bits(rnd).view(np.float16)
    assert _same_f32(got.astype(np.float32), exp.astype(np.float32))


def test_table_shift_closed_forms():
    f = lambda *v: b.table_shift(np.float32(v))
    assert f(0.0, 0.0) == 0
    assert f(1.0) == -14 and f(1.5, 0.25) == -14
    assert f(2.0**14) == 0 and f(3.0, 65504.0) == 1
    assert f(2.0**-149) == -149 - 14 and f(2.0**-127, 0.0) == -127 - 14
    assert f(np.inf, 1.0) == 0 and f(np.nan, 1.0) == 0


def numpy_search_f16(cent, d, codes, queries, k):
    """numpy restatement of the fp16-table search: float32 LUT, np.frexp for the exponent, np.ldexp scaling,
    numpy's float16 rounding, a float32 scan in sub-space order, (dist, id) sort, exact scaling back."""
    lut = numpy_lut(cent, queries)
    out = np.zeros((queries.shape[0], k), dtype=b.NEIGHBOR)
    for q in range(queries.shape[0]):
        mx = lut[q].max()
        shift = 0 if (mx == 0 or not np.isfinite(mx)) else int(np.frexp(mx)[1]) - 1 - 14
        with np.errstate(over="ignore"):
            t = np.ldexp(lut[q], -shift).astype(np.float32).astype(np.float16).astype(np.float32)
        acc = np.zeros(codes.shape[0], dtype=np.float32)
        for s in range(codes.shape[1]):
            acc = (acc + t[s, codes[:, s]]).astype(np.float32)
        order = np.lexsort((np.arange(codes.shape[0]), acc))[:k]
        out[q]["dist"] = np.ldexp(acc[order], shift).astype(np.float32)
        out[q]["id"] = order
    return out


@pytest.mark.parametrize("scale", [1.0, 300.0, 1e-6])
def test_search_f16_equals_numpy_restatement(scale):
    cent, codes, queries = random_case(32, 3000, 32, 8, 5, "normal")
    cent, queries = (cent * scale).astype(np.float32), (queries * scale).astype(np.float32)
    got = b.adc_search_f16(cent, 32, codes, queries, 17)
    exp = numpy_search_f16(cent, 32, codes, queries, 17)
    assert (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()


def test_search_f16_equals_fp32_search_when_tables_are_exact():
    # small-integer data: every LUT entry is an integer below 2^11, so scaling by a power of two and rounding to
    # binary16 are exact, every sum is exact, and the fp16 search must return the fp32 search's bits
    cent, codes, queries = random_case(33, 4000, 64, 16, 6, "ties")
    f16 = b.adc_search_f16(cent, 64, codes, queries, 25)
    f32 = b.adc_search(cent, 64, codes, queries, 25)
    assert (f16["id"] == f32["id"]).all() and (bits(f16["dist"]) == bits(f32["dist"])).all()


def test_planted_fp16_mistakes_fail_the_checks():
    # rounding by truncation instead of to nearest even
    x = np.float32([1.0 + 2.0**-11 + 2.0**-20, 3.0 + 3 * 2.0**-11])
    trunc = (x.view(np.uint32) >> 13 & 0x3ff) | ((x.view(np.uint32) >> 23) - 112) << 10
    assert not (b.f32_to_f16_bits(x) == trunc.astype(np.uint16)).all()
    # no per-query scaling: large-valued tables overflow binary16 and the results change
    cent, codes, queries = random_case(34, 2000, 32, 8, 3, "normal")
    cent, queries = (cent * 300).astype(np.float32), (queries * 300).astype(np.float32)
    lut = b.compute_lut(cent, 32, 8, queries)
    with np.errstate(over="ignore"):
        unscaled = lut.astype(np.float16).astype(np.float32)
    assert np.isinf(unscaled).any()
    good = b.adc_search_f16(cent, 32, codes, queries, 10)
    assert np.isfinite(good["dist"]).all()


# ---------------------------------------------------------------- 6. exact re-ranking (rerank_exact)

def rerank_case(seed, n=3000, d=48, nq=7, r=150, family="normal"):
    rng = np.random.default_rng(seed)
    if family == "ties":
        base = rng.integers(0, 3, size=(n, d)).astype(np.float32)
        queries = rng.integers(0, 3, size=(nq, d)).astype(np.float32)
    else:
        base = rng.standard_normal((n, d)).astype(np.float32)
        queries = rng.standard_normal((nq, d)).astype(np.float32)
    cand = np.zeros((nq, r), dtype=b.NEIGHBOR)
    cand["id"] = rng.integers(-1, n, size=(nq, r))
    cand["dist"] = rng.standard_normal((nq, r)).astype(np.float32)  # ignored by the re-rank
    cand["id"][:, :3] = cand["id"][:, 3:6]  # duplicated ids are pushed twice, as the reference does
    return base, queries, cand


@needs_ref
@pytest.mark.parametrize("k", [1, 10, 100, 160])
@pytest.mark.parametrize("family", ["normal", "ties"])
def test_rerank_equals_reference_live(k, family):
    base, queries, cand = rerank_case(41, family=family)
    got = b.rerank_exact(base, queries, cand, k)
    exp = b.rerank_exact(base, queries, cand, k, use_ref=True)
    assert (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()


@pytest.mark.parametrize("k", [1, 10, 160])
def test_rerank_equals_numpy_brute_force(k):
    base, queries, cand = rerank_case(42)
    got = b.rerank_exact(base, queries, cand, k)
    for q in range(queries.shape[0]):
        ids = cand["id"][q][cand["id"][q] >= 0]
        # l2sq's order: float32 diff, square, add, in dimension order
        acc = np.zeros(ids.size, dtype=np.float32)
        for j in range(base.shape[1]):
            diff = (queries[q, j] - base[ids, j]).astype(np.float32)
            acc = (acc + (diff * diff).astype(np.float32)).astype(np.float32)
        order = np.lexsort((ids, acc))[:k]
        exp_d = np.full(k, np.inf, dtype=np.float32)
        exp_i = np.full(k, -1, dtype=np.int32)
        exp_d[:order.size], exp_i[:order.size] = acc[order], ids[order]
        assert (got["id"][q] == exp_i).all() and (bits(got["dist"][q]) == bits(exp_d)).all()


def test_rerank_of_the_exact_candidates_is_the_exact_knn():
    # invariant: re-ranking all n ids gives the exhaustive exact k-NN (exact_knn, cpu_ref.cpp:56-64)
    base, queries, _ = rerank_case(43, n=500)
    allc = np.zeros((queries.shape[0], 500), dtype=b.NEIGHBOR)
    allc["id"] = np.arange(500)
    got = b.rerank_exact(base, queries, allc, 20)
    d64 = ((queries.astype(np.float64)[:, None, :] - base.astype(np.float64)[None]) ** 2).sum(-1)
    for q in range(queries.shape[0]):
        assert set(got["id"][q]) == set(np.argsort(d64[q], kind="stable")[:20]) or \
            np.allclose(np.sort(d64[q])[:20], got["dist"][q], rtol=1e-5)


# ---------------------------------------------------------------- 7. PQ encoding (nearest centroid)

def numpy_encode(cent, x):
    """float32 l2sq in dimension order for all 256 centroids, first minimum (np.argmin returns the first)."""
    m, _, dsub = cent.shape
    codes = np.empty((x.shape[0], m), dtype=np.uint8)
    for s in range(m):
        sub = x[:, s * dsub:(s + 1) * dsub]
        acc = np.zeros((x.shape[0], 256), dtype=np.float32)
        for j in range(dsub):
            diff = (sub[:, j:j + 1] - cent[s][None, :, j]).astype(np.float32)
            acc = (acc + (diff * diff).astype(np.float32)).astype(np.float32)
        codes[:, s] = np.argmin(acc, axis=1)
    return codes


@pytest.mark.parametrize("family", ["normal", "ties"])
def test_pq_encode_equals_numpy_first_minimum(family):
    cent, _, x = random_case(51, 10, 64, 16, 3000, family)
    if family == "ties":
        cent[:, 17] = cent[:, 3]  # duplicated centroids: the lower index must win
    assert (b.pq_encode(cent, x) == numpy_encode(cent, x)).all()


@needs_ref
def test_pq_encode_equals_reference_live():
    # tie-free codebook, so the reference's own (permuted) centroid order cannot change the winner
    cent, _, x = random_case(52, 10, 128, 16, 4000, "normal")
    rpq = b.RefPQ(cent, 128)
    assert (b.pq_encode(cent, x) == rpq.encode(x)).all()
    rpq.close()


def test_pq_encode_of_the_centroids_is_the_identity():
    cent, _, _ = random_case(53, 10, 32, 8, 1, "normal")
    x = np.ascontiguousarray(cent.transpose(1, 0, 2).reshape(256, 32))  # row c = centroid c of every sub-space
    assert (b.pq_encode(cent, x) == np.arange(256, dtype=np.uint8)[:, None]).all()


# ---------------------------------------------------------------- 8. IVF search (inverted lists)

def ivf_case(seed, n=4000, d=64, m=16, nq=6, nlist=40, family="normal"):
    cent, codes, queries = random_case(seed, n, d, m, nq, family)
    rng = np.random.default_rng(seed + 1)
    coarse = rng.standard_normal((nlist, d)).astype(np.float32)
    list_ids = rng.integers(0, nlist, size=n).astype(np.int32)
    return coarse, cent, codes, list_ids, queries


@pytest.mark.parametrize("family", ["normal", "ties"])
def test_ivf_probing_every_list_is_the_exhaustive_search(family):
    coarse, cent, codes, list_ids, queries = ivf_case(61, family=family)
    got = b.ivf_search(coarse, cent, 64, codes, list_ids, queries, 40, 25)
    exp = b.adc_search(cent, 64, codes, queries, 25)
    assert (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()


@pytest.mark.parametrize("nprobe", [1, 3, 17])
def test_ivf_equals_numpy_restatement(nprobe):
    coarse, cent, codes, list_ids, queries = ivf_case(62)
    got = b.ivf_search(coarse, cent, 64, codes, list_ids, queries, nprobe, 12)
    lut = numpy_lut(cent, queries)
    dists = numpy_scan(lut, codes)
    for q in range(queries.shape[0]):
        cd = np.zeros(coarse.shape[0], dtype=np.float32)
        for j in range(64):  # l2sq in dimension order
            diff = (queries[q, j] - coarse[:, j]).astype(np.float32)
            cd = (cd + (diff * diff).astype(np.float32)).astype(np.float32)
        probed = np.lexsort((np.arange(coarse.shape[0]), cd))[:nprobe]
        keep = np.nonzero(np.isin(list_ids, probed))[0]
        order = keep[np.lexsort((keep, dists[q, keep]))][:12]
        exp_d = np.full(12, np.inf, dtype=np.float32)
        exp_i = np.full(12, -1, dtype=np.int32)
        exp_d[:order.size], exp_i[:order.size] = dists[q, order], order
        assert (got["id"][q] == exp_i).all() and (bits(got["dist"][q]) == bits(exp_d)).all()


def test_ivf_one_list_is_the_exhaustive_search():
    coarse, cent, codes, list_ids, queries = ivf_case(63, nlist=1)
    list_ids[:] = 0
    got = b.ivf_search(coarse, cent, 64, codes, list_ids, queries, 1, 10)
    exp = b.adc_search(cent, 64, codes, queries, 10)
    assert (got["id"] == exp["id"]).all() and (bits(got["dist"]) == bits(exp["dist"])).all()
