#!/usr/bin/env python3
"""Writes the golden fixtures in this directory from the reference's own CPU code.

The reference's src/cpu/{cpu_ref,pq,io}.cpp are compiled where they lie into oracle/_ref/libvkref.so by
oracle/Makefile (`make -C oracle ref`, needs the reference checkout). This script runs them on small seeded
inputs and stores inputs and outputs as .npz fixtures (numpy, no pickles). tests/test_oracle.py checks the
oracle against these files, so the oracle stays pinned wherever the reference library cannot be built.

Fixtures:
  clustered_m8.npz   reference synthetic_clustered data, reference-trained PQ (m=8): LUT, ADC matrix, top-k
  clustered_m16.npz  the same with m=16, several k including k > 64
  ties_m16.npz       small-integer codebook and queries: many equal distances, order decided by id
  tiny_diffs.npz     centroids within 1e-20 of the query: squared differences underflow to subnormals / zero
  topk_kat.npz       the reference's TopK known-answer case and padding (tests/test_cpu.cpp:33-46)
  recall_kat.npz     recall_at_k on hand-made rows with padding ids and repeated ids
  train_kmeans.npz   ProductQuantizer::train codebooks: clustered data; rows repeated so that most clusters go
                     empty and are re-seeded; zero iterations (the shuffled initial points alone)

`python make_golden.py NAME ...` writes only the named fixtures.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import binding as b  # noqa: E402


def ref_clustered(n, d, clusters, seed):
    out = np.empty((n, d), dtype=np.float32)
    b.ref().vkref_synthetic_clustered(n, d, clusters, seed, out.ctypes.data)
    return out


def ref_train(x, m, iters, seed=1):
    n, d = x.shape
    lib = b.ref()
    h = lib.vkref_pq_create(d, m)
    assert h and lib.vkref_pq_train(h, np.ascontiguousarray(x).ctypes.data, n, iters, seed) == 0
    cent = np.empty((m, 256, d // m), dtype=np.float32)
    lib.vkref_pq_centroids(h, cent.ctypes.data)
    codes = np.empty((n, m), dtype=np.uint8)
    lib.vkref_pq_encode(h, np.ascontiguousarray(x).ctypes.data, n, codes.ctypes.data)
    lib.vkref_pq_destroy(h)
    return cent, codes


def outputs(cent, d, codes, queries, ks):
    rpq = b.RefPQ(cent, d)
    codes_ref = rpq.remap_codes(codes)
    lut_ref = rpq.compute_lut(queries)
    # the reference LUT is indexed by its own centroid order; store it in the given codebook's order
    lut = np.empty_like(lut_ref)
    for s in range(rpq.m):
        lut[:, s, :] = lut_ref[:, s, rpq.inverse[s]]
    nq, n, m = queries.shape[0], codes.shape[0], codes.shape[1]
    dists = np.empty((nq, n), dtype=np.float32)
    b.ref().vkref_adc_scan(np.ascontiguousarray(lut).ctypes.data, nq, np.ascontiguousarray(codes).ctypes.data, n, m,
                           dists.ctypes.data)
    out = {"lut": lut, "dists": dists}
    for k in ks:
        res = rpq.adc_search(codes_ref, queries, k)
        out[f"search_k{k}_dist"] = res["dist"]
        out[f"search_k{k}_id"] = res["id"]
        sel = np.empty((nq, k), dtype=b.NEIGHBOR)
        b.ref().vkref_select_topk(dists.ctypes.data, nq, n, k, sel.ctypes.data)
        out[f"select_k{k}_dist"] = sel["dist"]
        out[f"select_k{k}_id"] = sel["id"]
    return out


def save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.1f} KiB)")


def write_train_fixture():
    rng = np.random.default_rng(17)
    cases = []
    cases.append((ref_clustered(700, 16, 10, 3), 4, 3, 5))
    distinct = rng.standard_normal((40, 8)).astype(np.float32)
    cases.append((distinct[rng.integers(0, 40, size=300)], 2, 2, 9))  # 40 distinct rows: >= 216 empty clusters
    cases.append((ref_clustered(400, 32, 7, 4), 8, 0, 1))
    arrays = {}
    for j, (x, m, iters, seed) in enumerate(cases):
        cent, _ = ref_train(x, m, iters, seed)
        arrays.update({f"x{j}": x, f"m{j}": np.int64(m), f"iters{j}": np.int64(iters), f"seed{j}": np.int64(seed),
                       f"centroids{j}": cent})
    save("train_kmeans.npz", cases=np.int64(len(cases)), **arrays)


def main():
    if not b.ref_available():
        sys.exit("oracle/_ref/libvkref.so is not built (make -C oracle ref, with the reference checkout present)")
    only = set(sys.argv[1:])
    if only:
        if "train_kmeans.npz" in only:
            write_train_fixture()
        return

    write_train_fixture()
    for m, n, d, nq, ks, name in [(8, 2000, 32, 5, (1, 10, 100), "clustered_m8.npz"),
                                  (16, 2003, 64, 5, (10, 33, 128), "clustered_m16.npz")]:
        base = ref_clustered(n, d, 20, 7)
        queries = ref_clustered(nq, d, 20, 8)
        cent, codes = ref_train(base, m, 10)
        save(name, centroids=cent, codes=codes, queries=queries, d=np.int64(d),
             **outputs(cent, d, codes, queries, ks))

    rng = np.random.default_rng(5)
    m, d, n, nq = 16, 32, 1500, 4
    cent = rng.integers(0, 3, size=(m, 256, d // m)).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    queries = rng.integers(0, 3, size=(nq, d)).astype(np.float32)
    save("ties_m16.npz", centroids=cent, codes=codes, queries=queries, d=np.int64(d),
         **outputs(cent, d, codes, queries, (16, 64)))

    m, d, n, nq = 16, 32, 600, 3
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    cent = np.repeat(queries[0].reshape(m, 1, d // m), 256, axis=1).copy()
    cent += (rng.integers(0, 5, size=cent.shape) * 1e-20).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    save("tiny_diffs.npz", centroids=cent, codes=codes, queries=queries, d=np.int64(d),
         **outputs(cent, d, codes, queries, (10,)))

    kat_d = np.array([5, 1, 4, 1, 3], dtype=np.float32)
    kat_i = np.arange(5, dtype=np.int32)
    top3 = b.topk_run(kat_d, kat_i, 3, use_ref=True)
    pad = b.topk_run(np.array([2.0], dtype=np.float32), np.array([9], dtype=np.int32), 4, use_ref=True)
    save("topk_kat.npz", values=kat_d, ids=kat_i, top3_dist=top3["dist"], top3_id=top3["id"],
         pad_dist=pad["dist"], pad_id=pad["id"])

    found = np.zeros((3, 4), dtype=b.NEIGHBOR)
    found["id"] = [[1, 2, 3, 4], [5, -1, -1, 7], [8, 8, 9, 10]]
    truth = np.array([[4, 3, 2, 99], [7, 5, -1, 0], [8, 11, 12, 13]], dtype=np.int32)
    recalls = {}
    for k in (1, 2, 3, 4):
        r = b.ref().vkref_recall_at_k(found.ctypes.data, 4, truth.ctypes.data, 4, 3, k)
        recalls[f"recall_k{k}"] = np.float64(r)
    save("recall_kat.npz", found_id=found["id"], truth=truth, **recalls)


if __name__ == "__main__":
    main()
