"""Host-side tools of veckern_amd (lib/libveckern_cpu.so, include/veckern/host.h): seeded synthetic data, the PQ
codec, recall evaluation, and the CPU search path (veckern/cpu_ref.hpp) that the benchmark driver times beside the
GPU. They build the GPU search's inputs, score its outputs and give its CPU counterpart.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import NEIGHBOR_DTYPE, _HERE

LIB_PATH = os.path.join(_HERE, "lib", "libveckern_cpu.so")
_P, _S = ctypes.c_void_p, ctypes.c_size_t
_lib = None

# Stream numbers of the N(0, 1) value streams used for directly generated inputs (distinct from the streams the
# C++ generators use internally).
STREAM_CODEBOOK = 30
STREAM_QUERIES = 31


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `make -C veckern_amd cpu`")
        lib = ctypes.CDLL(LIB_PATH)
        lib.vkh_last_error.restype = ctypes.c_char_p
        lib.vkh_max_threads.restype = ctypes.c_int
        lib.vkh_philox4x32_10.argtypes = [_P, _P, _P]
        lib.vkh_philox4x32_10.restype = None
        lib.vkh_gaussian_mixture.argtypes = [_S, _S, ctypes.c_float, ctypes.c_uint64, _S, _S, _P]
        lib.vkh_synthetic_source.argtypes = [_S, _S, ctypes.c_uint64, _S, _S, _S, _P]
        lib.vkh_synthetic_clustered.argtypes = [_S, _S, _S, ctypes.c_uint64, _P]
        lib.vkh_uniform_codes.argtypes = [_S, _S, _S, ctypes.c_uint64, _P]
        lib.vkh_normal_values.argtypes = [ctypes.c_uint64, ctypes.c_uint32, _S, _S, _P]
        lib.vkh_pq_train.argtypes = [_P, _S, _S, _S, _S, ctypes.c_uint64, _P]
        lib.vkh_pq_encode.argtypes = [_P, _S, _S, _P, _S, _P]
        lib.vkh_pq_decode.argtypes = [_P, _S, _S, _P, _S, _P]
        lib.vkh_compute_lut.argtypes = [_P, _S, _S, _P, _S, _P]
        lib.vkh_adc_scan.argtypes = [_P, _S, _P, _S, _S, _P]
        lib.vkh_select_topk.argtypes = [_P, _S, _S, _S, _P]
        lib.vkh_adc_search.argtypes = [_P, _S, _S, _P, _S, _P, _S, _S, _P]
        lib.vkh_exact_knn.argtypes = [_P, _S, _P, _S, _S, _S, _P]
        lib.vkh_rerank_exact.argtypes = [_P, _S, _P, _S, _P, _S, _S, _P]
        lib.vkh_recall_at_k.restype = ctypes.c_double
        lib.vkh_recall_at_k.argtypes = [_P, _S, _P, _S, _S, _S]
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(library().vkh_last_error().decode())


def max_threads() -> int:
    return library().vkh_max_threads()


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, dtype=np.uint32)
    library().vkh_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
    return out


def gaussian_mixture(d: int, components: int, sigma: float, seed: int, first: int, count: int) -> np.ndarray:
    out = np.empty((count, d), dtype=np.float32)
    _check(library().vkh_gaussian_mixture(d, components, sigma, seed, first, count, out.ctypes.data))
    return out


def synthetic_source(d: int, clusters: int, seed: int, latent_dim: int, first: int, count: int) -> np.ndarray:
    out = np.empty((count, d), dtype=np.float32)
    _check(library().vkh_synthetic_source(d, clusters, seed, latent_dim, first, count, out.ctypes.data))
    return out


def synthetic_clustered(n: int, d: int, clusters: int, seed: int) -> np.ndarray:
    out = np.empty((n, d), dtype=np.float32)
    _check(library().vkh_synthetic_clustered(n, d, clusters, seed, out.ctypes.data))
    return out


def uniform_codes(first: int, n: int, m: int, seed: int) -> np.ndarray:
    out = np.empty((n, m), dtype=np.uint8)
    _check(library().vkh_uniform_codes(first, n, m, seed, out.ctypes.data))
    return out


def normal_values(seed: int, stream: int, first: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    _check(library().vkh_normal_values(seed, stream, first, count, out.ctypes.data))
    return out


def pq_train(x: np.ndarray, m: int, iters: int, seed: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    cent = np.empty((m, 256, d // m), dtype=np.float32)
    _check(library().vkh_pq_train(x.ctypes.data, n, d, m, iters, seed, cent.ctypes.data))
    return cent


def pq_encode(centroids: np.ndarray, x: np.ndarray) -> np.ndarray:
    cent = np.ascontiguousarray(centroids, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    m = cent.shape[0]
    codes = np.empty((n, m), dtype=np.uint8)
    _check(library().vkh_pq_encode(cent.ctypes.data, d, m, x.ctypes.data, n, codes.ctypes.data))
    return codes


def pq_decode(centroids: np.ndarray, codes: np.ndarray, d: int) -> np.ndarray:
    cent = np.ascontiguousarray(centroids, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    n, m = codes.shape
    x = np.empty((n, d), dtype=np.float32)
    _check(library().vkh_pq_decode(cent.ctypes.data, d, m, codes.ctypes.data, n, x.ctypes.data))
    return x


def compute_lut(centroids: np.ndarray, queries: np.ndarray) -> np.ndarray:
    """The CPU path's tables: (nq, m, 256) squared sub-distances."""
    cent = np.ascontiguousarray(centroids, dtype=np.float32)
    m = cent.shape[0]
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq, d = q.shape
    lut = np.empty((nq, m, 256), dtype=np.float32)
    _check(library().vkh_compute_lut(cent.ctypes.data, d, m, q.ctypes.data, nq, lut.ctypes.data))
    return lut


def adc_scan(lut: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """The CPU path's ADC distances: (nq, n)."""
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    n, m = codes.shape
    nq = lut.size // (m * 256)
    out = np.empty((nq, n), dtype=np.float32)
    _check(library().vkh_adc_scan(lut.ctypes.data, nq, codes.ctypes.data, n, m, out.ctypes.data))
    return out


def select_topk(dists: np.ndarray, k: int) -> np.ndarray:
    dists = np.ascontiguousarray(dists, dtype=np.float32)
    nq, n = dists.shape
    out = np.empty((nq, k), dtype=NEIGHBOR_DTYPE)
    _check(library().vkh_select_topk(dists.ctypes.data, nq, n, k, out.ctypes.data))
    return out


def adc_search(centroids: np.ndarray, codes: np.ndarray, queries: np.ndarray, k: int) -> np.ndarray:
    """The CPU search path (LUT, scan and top-k per query on all host threads): (nq, k) neighbours."""
    cent = np.ascontiguousarray(centroids, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    n, m = codes.shape
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq, d = q.shape
    out = np.empty((nq, k), dtype=NEIGHBOR_DTYPE)
    _check(library().vkh_adc_search(cent.ctypes.data, d, m, codes.ctypes.data, n, q.ctypes.data, nq, k,
                                    out.ctypes.data))
    return out


def exact_knn(base: np.ndarray, queries: np.ndarray, k: int) -> np.ndarray:
    base = np.ascontiguousarray(base, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    out = np.empty((q.shape[0], k), dtype=NEIGHBOR_DTYPE)
    _check(library().vkh_exact_knn(base.ctypes.data, base.shape[0], q.ctypes.data, q.shape[0], base.shape[1], k,
                                   out.ctypes.data))
    return out


def rerank_exact(base: np.ndarray, queries: np.ndarray, candidates: np.ndarray, k: int) -> np.ndarray:
    base = np.ascontiguousarray(base, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    cand = np.ascontiguousarray(candidates, dtype=NEIGHBOR_DTYPE)
    out = np.empty((q.shape[0], k), dtype=NEIGHBOR_DTYPE)
    _check(library().vkh_rerank_exact(base.ctypes.data, base.shape[1], q.ctypes.data, q.shape[0], cand.ctypes.data,
                                      cand.shape[1], k, out.ctypes.data))
    return out


def recall_at_k(found: np.ndarray, truth_ids: np.ndarray, k: int) -> float:
    """found: (nq, >=k) neighbours; truth_ids: (nq, >=k) int32."""
    f = np.ascontiguousarray(found, dtype=NEIGHBOR_DTYPE)
    t = np.ascontiguousarray(truth_ids, dtype=np.int32)
    r = library().vkh_recall_at_k(f.ctypes.data, f.shape[1], t.ctypes.data, t.shape[1], f.shape[0], k)
    if r < 0:
        raise RuntimeError(library().vkh_last_error().decode())
    return r


# ---- vector files (the TEXMEX formats of SIFT1M/GIST1M; reference src/cpu/io.cpp:12-52, C++ in host/io.cpp).
# Each row is a little-endian int32 dimension followed by that many values: float32 (.fvecs), uint8 (.bvecs) or
# int32 (.ivecs). The readers memory-map the file, check that every row carries the same dimension, and return at
# most max_n rows (0 = all); .bvecs rows come back as float32 like the C++ reader's.

def _read_vecs(path: str, value: np.dtype, max_n: int) -> np.ndarray:
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    if raw.size < 4:
        raise ValueError(f"{path}: empty or truncated vector file")
    d = int(raw[:4].view("<i4")[0])
    row = 4 + d * np.dtype(value).itemsize
    if d <= 0 or raw.size % row:
        raise ValueError(f"{path}: size {raw.size} is not a whole number of rows of dimension {d}")
    n = raw.size // row if max_n == 0 else min(max_n, raw.size // row)
    rows = raw[: n * row].reshape(n, row)
    if (rows[:, :4].copy().view("<i4")[:, 0] != d).any():
        raise ValueError(f"{path}: rows of differing dimension")
    return np.ascontiguousarray(rows[:, 4:]).view(np.dtype(value).newbyteorder("<")).reshape(n, d)


def read_fvecs(path: str, max_n: int = 0) -> np.ndarray:
    return _read_vecs(path, np.float32, max_n).astype(np.float32, copy=False)


def read_bvecs(path: str, max_n: int = 0) -> np.ndarray:
    return _read_vecs(path, np.uint8, max_n).astype(np.float32)


def read_ivecs(path: str, max_n: int = 0) -> np.ndarray:
    return _read_vecs(path, np.int32, max_n).astype(np.int32, copy=False)


def _write_vecs(path: str, x: np.ndarray, value: np.dtype) -> None:
    x = np.ascontiguousarray(x, dtype=np.dtype(value).newbyteorder("<"))
    n, d = x.shape
    head = np.full((n, 1), d, dtype="<i4").view(np.uint8)
    np.concatenate([head, x.view(np.uint8).reshape(n, -1)], axis=1).tofile(path)


def write_fvecs(path: str, x: np.ndarray) -> None:
    _write_vecs(path, x, np.float32)


def write_bvecs(path: str, x: np.ndarray) -> None:
    _write_vecs(path, x, np.uint8)


def write_ivecs(path: str, x: np.ndarray) -> None:
    _write_vecs(path, x, np.int32)
