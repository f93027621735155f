"""ctypes binding of the oracle (oracle/lib/libvk_oracle.so) and, when built, of the reference's own CPU library
(oracle/_ref/libvkref.so). Test infrastructure: these are the checkers the GPU path is compared against.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_LIB = os.path.join(ROOT, "oracle", "lib", "libvk_oracle.so")
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libvkref.so")

NEIGHBOR = np.dtype([("dist", np.float32), ("id", np.int32)])
_P = ctypes.c_void_p
_S = ctypes.c_size_t

_oracle = None
_ref = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"{ORACLE_LIB} missing: run `make -C oracle`")
        lib = ctypes.CDLL(ORACLE_LIB)
        lib.vko_less.argtypes = [ctypes.c_float, ctypes.c_int32, ctypes.c_float, ctypes.c_int32]
        lib.vko_l2sq.restype = ctypes.c_float
        lib.vko_l2sq.argtypes = [_P, _P, _S]
        lib.vko_compute_lut.argtypes = [_P, _S, _S, _P, _S, _P]
        lib.vko_adc_scan.argtypes = [_P, _S, _P, _S, _S, _P]
        lib.vko_select_topk.argtypes = [_P, _S, _S, _S, _P]
        lib.vko_adc_search.argtypes = [_P, _S, _S, _P, _S, _P, _S, _S, _P]
        lib.vko_recall_at_k.restype = ctypes.c_double
        lib.vko_recall_at_k.argtypes = [_P, _S, _P, _S, _S, _S]
        lib.vko_max_threads.restype = ctypes.c_int
        lib.vko_topk_run.argtypes = [_P, _P, _S, _S, _P]
        lib.vko_f32_to_f16_array.argtypes = [_P, _S, _P]
        lib.vko_f16_to_f32_array.argtypes = [_P, _S, _P]
        lib.vko_table_shift.restype = ctypes.c_int
        lib.vko_table_shift.argtypes = [_P, _S]
        lib.vko_adc_search_f16.argtypes = [_P, _S, _S, _P, _S, _P, _S, _S, _P]
        lib.vko_rerank_exact.argtypes = [_P, _S, _P, _S, _P, _S, _S, _P]
        lib.vko_pq_encode.argtypes = [_P, _S, _S, _P, _S, _P]
        lib.vko_ivf_search.argtypes = [_P, _S, _P, _S, _S, _P, _P, _S, _P, _S, _S, _S, _P]
        _oracle = lib
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(REF_LIB)
        lib.vkref_pq_create.restype = _P
        lib.vkref_pq_create.argtypes = [_S, _S]
        lib.vkref_pq_destroy.argtypes = [_P]
        lib.vkref_pq_train.argtypes = [_P, _P, _S, _S, ctypes.c_uint64]
        lib.vkref_pq_encode.argtypes = [_P, _P, _S, _P]
        lib.vkref_pq_decode.argtypes = [_P, _P, _S, _P]
        lib.vkref_pq_centroids.argtypes = [_P, _P]
        lib.vkref_compute_lut.argtypes = [_P, _P, _S, _P]
        lib.vkref_adc_scan.argtypes = [_P, _S, _P, _S, _S, _P]
        lib.vkref_select_topk.argtypes = [_P, _S, _S, _S, _P]
        lib.vkref_adc_search.argtypes = [_P, _P, _S, _P, _S, _S, _P]
        lib.vkref_exact_knn.argtypes = [_P, _S, _P, _S, _S, _S, _P]
        lib.vkref_rerank_exact.argtypes = [_P, _S, _P, _S, _P, _S, _S, _P]
        lib.vkref_recall_at_k.restype = ctypes.c_double
        lib.vkref_recall_at_k.argtypes = [_P, _S, _P, _S, _S, _S]
        lib.vkref_topk_run.argtypes = [_P, _P, _S, _S, _P]
        lib.vkref_synthetic_clustered.argtypes = [_S, _S, _S, ctypes.c_uint64, _P]
        _ref = lib
    return _ref


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- oracle wrappers

def compute_lut(centroids: np.ndarray, d: int, m: int, queries: np.ndarray) -> np.ndarray:
    q = _c(queries, np.float32).reshape(-1, d)
    c = _c(centroids, np.float32)
    lut = np.empty((q.shape[0], m, 256), dtype=np.float32)
    oracle().vko_compute_lut(c.ctypes.data, d, m, q.ctypes.data, q.shape[0], lut.ctypes.data)
    return lut


def adc_scan(lut: np.ndarray, codes: np.ndarray) -> np.ndarray:
    lut = _c(lut, np.float32)
    codes = _c(codes, np.uint8)
    n, m = codes.shape
    nq = lut.size // (m * 256)
    out = np.empty((nq, n), dtype=np.float32)
    oracle().vko_adc_scan(lut.ctypes.data, nq, codes.ctypes.data, n, m, out.ctypes.data)
    return out


def select_topk(dists: np.ndarray, k: int) -> np.ndarray:
    dists = _c(dists, np.float32)
    nq, n = dists.shape
    out = np.empty((nq, k), dtype=NEIGHBOR)
    oracle().vko_select_topk(dists.ctypes.data, nq, n, k, out.ctypes.data)
    return out


def adc_search(centroids: np.ndarray, d: int, codes: np.ndarray, queries: np.ndarray, k: int) -> np.ndarray:
    codes = _c(codes, np.uint8)
    n, m = codes.shape
    q = _c(queries, np.float32).reshape(-1, d)
    c = _c(centroids, np.float32)
    out = np.empty((q.shape[0], k), dtype=NEIGHBOR)
    rc = oracle().vko_adc_search(c.ctypes.data, d, m, codes.ctypes.data, n, q.ctypes.data, q.shape[0], k,
                                 out.ctypes.data)
    if rc != 0:
        raise ValueError("vko_adc_search rejected its input")
    return out


def adc_search_f16(centroids: np.ndarray, d: int, codes: np.ndarray, queries: np.ndarray, k: int) -> np.ndarray:
    """The fp16-table search (ScanVariant.FusedWarpF16) restated on the CPU."""
    codes = _c(codes, np.uint8)
    n, m = codes.shape
    q = _c(queries, np.float32).reshape(-1, d)
    c = _c(centroids, np.float32)
    out = np.empty((q.shape[0], k), dtype=NEIGHBOR)
    rc = oracle().vko_adc_search_f16(c.ctypes.data, d, m, codes.ctypes.data, n, q.ctypes.data, q.shape[0], k,
                                     out.ctypes.data)
    if rc != 0:
        raise ValueError("vko_adc_search_f16 rejected its input")
    return out


def ivf_search(coarse: np.ndarray, centroids: np.ndarray, d: int, codes: np.ndarray, list_ids: np.ndarray,
               queries: np.ndarray, nprobe: int, k: int) -> np.ndarray:
    """IVF search: the exhaustive search restricted to each query's nprobe nearest lists."""
    co = _c(coarse, np.float32).reshape(-1, d)
    c = _c(centroids, np.float32)
    codes = _c(codes, np.uint8)
    n, m = codes.shape
    li = _c(list_ids, np.int32)
    q = _c(queries, np.float32).reshape(-1, d)
    out = np.empty((q.shape[0], k), dtype=NEIGHBOR)
    if oracle().vko_ivf_search(co.ctypes.data, co.shape[0], c.ctypes.data, d, m, codes.ctypes.data, li.ctypes.data,
                               n, q.ctypes.data, q.shape[0], nprobe, k, out.ctypes.data) != 0:
        raise ValueError("vko_ivf_search rejected its input")
    return out


def pq_encode(centroids: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Nearest centroid per sub-space (the reference's ProductQuantizer::encode) of the rows of x."""
    c = _c(centroids, np.float32)
    m = c.shape[0]
    x = _c(x, np.float32)
    n, d = x.shape
    codes = np.empty((n, m), dtype=np.uint8)
    oracle().vko_pq_encode(c.ctypes.data, d, m, x.ctypes.data, n, codes.ctypes.data)
    return codes


def rerank_exact(base: np.ndarray, queries: np.ndarray, candidates: np.ndarray, k: int,
                 use_ref: bool = False) -> np.ndarray:
    """Exact re-ranking of nq x r candidates (NEIGHBOR records; ids < 0 skipped) against base rows."""
    base = _c(base, np.float32)
    d = base.shape[1]
    q = _c(queries, np.float32).reshape(-1, d)
    cand = _c(candidates, NEIGHBOR).reshape(q.shape[0], -1)
    out = np.empty((q.shape[0], k), dtype=NEIGHBOR)
    if use_ref:
        ref().vkref_rerank_exact(base.ctypes.data, d, q.ctypes.data, q.shape[0], cand.ctypes.data, cand.shape[1], k,
                                 out.ctypes.data)
    elif oracle().vko_rerank_exact(base.ctypes.data, d, q.ctypes.data, q.shape[0], cand.ctypes.data,
                                   cand.shape[1], k, out.ctypes.data) != 0:
        raise MemoryError("vko_rerank_exact failed")
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    oracle().vko_f32_to_f16_array(x.ctypes.data, x.size, out.ctypes.data)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    oracle().vko_f16_to_f32_array(h.ctypes.data, h.size, out.ctypes.data)
    return out


def table_shift(table: np.ndarray) -> int:
    t = _c(table, np.float32)
    return oracle().vko_table_shift(t.ctypes.data, t.size)


def recall_at_k(found: np.ndarray, truth: np.ndarray, k: int) -> float:
    found = _c(found, NEIGHBOR)
    truth = _c(truth, np.int32)
    return oracle().vko_recall_at_k(found.ctypes.data, found.shape[1], truth.ctypes.data, truth.shape[1],
                                    found.shape[0], k)


def topk_run(dists, ids, k: int, use_ref: bool = False) -> np.ndarray:
    d = _c(dists, np.float32)
    i = _c(ids, np.int32)
    out = np.empty(k, dtype=NEIGHBOR)
    fn = ref().vkref_topk_run if use_ref else oracle().vko_topk_run
    fn(d.ctypes.data, i.ctypes.data, d.size, k, out.ctypes.data)
    return out


# ---------------------------------------------------------------- the reference's own CPU library (oracle/_ref)

class RefPQ:
    """A reference ProductQuantizer (oracle/_ref) holding a given codebook.

    The reference class has no codebook setter, so it is trained for 0 iterations on 256 points whose s-th
    sub-vectors are the 256 given centroids of sub-space s: its initialisation then copies exactly those points,
    in a shuffled order per sub-space (pq.cpp:41-45). `perm[s][c]` is the given centroid the reference stores at
    index c; `remap_codes` translates codes written against the given codebook into the reference's indices.
    """

    def __init__(self, centroids: np.ndarray, d: int):
        cent = _c(centroids, np.float32)
        m = cent.shape[0]
        dsub = d // m
        cent = cent.reshape(m, 256, dsub)
        points = np.ascontiguousarray(cent.transpose(1, 0, 2).reshape(256, d))
        lib = ref()
        self._h = lib.vkref_pq_create(d, m)
        if not self._h:
            raise ValueError("reference ProductQuantizer rejected (d, m)")
        if lib.vkref_pq_train(self._h, points.ctypes.data, 256, 0, 1) != 0:
            raise ValueError("reference training failed")
        got = np.empty((m, 256, dsub), dtype=np.float32)
        lib.vkref_pq_centroids(self._h, got.ctypes.data)
        self.d, self.m = d, m
        self.perm = np.empty((m, 256), dtype=np.int64)
        self.inverse = np.empty((m, 256), dtype=np.uint8)
        for s in range(m):
            # Match stored and given centroids by value. Equal vectors give equal LUT entries, so with repeated
            # centroids any index holding the same vector is a valid match, in either direction.
            given_of, ref_of = {}, {}
            for c in range(256):
                given_of.setdefault(cent[s, c].tobytes(), c)
                ref_of.setdefault(got[s, c].tobytes(), c)
            self.perm[s] = [given_of[got[s, r].tobytes()] for r in range(256)]
            self.inverse[s] = [ref_of[cent[s, c].tobytes()] for c in range(256)]
        self.centroids = got

    def remap_codes(self, codes: np.ndarray) -> np.ndarray:
        codes = _c(codes, np.uint8)
        out = np.empty_like(codes)
        for s in range(self.m):
            out[:, s] = self.inverse[s][codes[:, s]]
        return out

    def encode(self, x: np.ndarray) -> np.ndarray:
        """The reference's ProductQuantizer::encode, translated back to indices of the given codebook."""
        x = _c(x, np.float32)
        codes = np.empty((x.shape[0], self.m), dtype=np.uint8)
        ref().vkref_pq_encode(self._h, x.ctypes.data, x.shape[0], codes.ctypes.data)
        for s in range(self.m):
            codes[:, s] = self.perm[s][codes[:, s]]
        return codes

    def adc_search(self, codes_ref: np.ndarray, queries: np.ndarray, k: int) -> np.ndarray:
        """The reference's adc_search (cpu_ref.cpp:38-54); codes must already be remapped."""
        codes_ref = _c(codes_ref, np.uint8)
        q = _c(queries, np.float32).reshape(-1, self.d)
        out = np.empty((q.shape[0], k), dtype=NEIGHBOR)
        ref().vkref_adc_search(self._h, codes_ref.ctypes.data, codes_ref.shape[0], q.ctypes.data, q.shape[0], k,
                               out.ctypes.data)
        return out

    def compute_lut(self, queries: np.ndarray) -> np.ndarray:
        q = _c(queries, np.float32).reshape(-1, self.d)
        lut = np.empty((q.shape[0], self.m, 256), dtype=np.float32)
        ref().vkref_compute_lut(self._h, q.ctypes.data, q.shape[0], lut.ctypes.data)
        return lut

    def close(self):
        if self._h:
            ref().vkref_pq_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def max_threads() -> int:
    return oracle().vko_max_threads()
