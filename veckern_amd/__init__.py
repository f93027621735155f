"""veckern_amd — MI355X (gfx950) product-quantisation search: per-query LUT build, fused ADC scan and top-k.

Python binding of the C ABI in ``include/veckern/veckern.h`` (``lib/libveckern.so``). It mirrors the
reference's C++ host API (``include/veckern/gpu.hpp``: ``PQSearcher``, ``ScanVariant``, ``Tuning``,
``DeviceInfo``, ``Timings``, ``LaunchShape``) with the same names, argument meaning and errors, so tests and
benchmarks read like the reference's own. The kernels run on the GPU only: there is no CPU fallback, and loading
fails loudly when the HIP library has not been built.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass

import numpy as np

__all__ = [
    "ScanVariant", "Tuning", "Timings", "LaunchShape", "DeviceInfo", "PQSearcher", "VkError",
    "variant_name", "is_fused", "needs_m16", "device_info", "device_count", "dispatched_k", "validate_tuning",
    "library", "LIB_PATH", "DeviceArray", "Reranker", "IVFIndex", "ivf_assign", "pq_encode", "pq_assign",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libveckern.so")

VK_OK, VK_ERR_INVALID_ARGUMENT, VK_ERR_RUNTIME, VK_ERR_LOGIC, VK_ERR_DEVICE, VK_ERR_OUT_OF_MEMORY = range(6)


class VkError(RuntimeError):
    """An error reported through the C ABI; ``code`` is the vk_status value."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class VkInvalidArgument(VkError, ValueError):
    """std::invalid_argument in the reference."""


class VkLogicError(VkError):
    """std::logic_error in the reference."""


class ScanVariant(enum.IntEnum):
    """veckern::gpu::ScanVariant (reference gpu.hpp:13-23); FusedWarpF16 is this build's fp16-table v8."""

    GlobalLut = 0
    SharedLut = 1
    SharedLutVec = 2
    Interleaved = 3
    Fused = 4
    FusedReg = 5
    FusedVec = 6
    FusedVecMQ = 7
    FusedWarp = 8
    FusedWarpF16 = 9


class _Neighbor(ctypes.Structure):
    _fields_ = [("dist", ctypes.c_float), ("id", ctypes.c_int32)]


class _Tuning(ctypes.Structure):
    _fields_ = [("scan_threads", ctypes.c_int), ("blocks_per_query", ctypes.c_int),
                ("queries_per_block", ctypes.c_int), ("vectors_per_step", ctypes.c_int)]


class _Timings(ctypes.Structure):
    _fields_ = [("transfer_ms", ctypes.c_double), ("lut_ms", ctypes.c_double), ("scan_ms", ctypes.c_double),
                ("select_ms", ctypes.c_double)]


class _LaunchShape(ctypes.Structure):
    _fields_ = [("threads", ctypes.c_int), ("blocks_x", ctypes.c_int), ("grid_y", ctypes.c_int),
                ("queries_per_block", ctypes.c_int), ("vectors_per_step", ctypes.c_int),
                ("blocks_per_sm", ctypes.c_int), ("waves", ctypes.c_double)]


class _DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("sm_count", ctypes.c_int),
                ("peak_bandwidth_gbs", ctypes.c_double), ("max_smem_per_block", ctypes.c_size_t),
                ("clock_khz", ctypes.c_int), ("warp_size", ctypes.c_int), ("l2_bytes", ctypes.c_size_t),
                ("total_mem_bytes", ctypes.c_size_t)]


NEIGHBOR_DTYPE = np.dtype([("dist", np.float32), ("id", np.int32)])

# Every symbol declared in include/veckern/veckern.h, with its ctypes signature.
_P = ctypes.c_void_p
_SIGNATURES = {
    "vk_last_error": (ctypes.c_char_p, []),
    "vk_abi_version": (ctypes.c_int, []),
    "vk_variant_name": (ctypes.c_char_p, [ctypes.c_int]),
    "vk_is_fused": (ctypes.c_int, [ctypes.c_int]),
    "vk_needs_m16": (ctypes.c_int, [ctypes.c_int]),
    "vk_tuning_default": (None, [ctypes.POINTER(_Tuning)]),
    "vk_tuning_validate": (ctypes.c_int, [ctypes.POINTER(_Tuning)]),
    "vk_dispatched_k": (ctypes.c_int, [ctypes.c_size_t]),
    "vk_get_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "vk_get_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_DeviceInfo)]),
    "vk_searcher_create": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.c_size_t, _P, ctypes.c_size_t,
                                          ctypes.POINTER(_P)]),
    "vk_searcher_destroy": (None, [_P]),
    "vk_searcher_set_tuning": (ctypes.c_int, [_P, ctypes.POINTER(_Tuning)]),
    "vk_searcher_get_tuning": (ctypes.c_int, [_P, ctypes.POINTER(_Tuning)]),
    "vk_searcher_last_launch": (ctypes.c_int, [_P, ctypes.POINTER(_LaunchShape)]),
    "vk_searcher_layout": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P]),
    "vk_search": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, _P,
                                 ctypes.POINTER(_Timings)]),
    "vk_distances": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_int, _P, ctypes.POINTER(_Timings)]),
    "vk_search_device": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, _P,
                                        ctypes.POINTER(_Timings)]),
    "vk_search_device_noalloc": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, _P]),
    "vk_ivf_create": (ctypes.c_int, [_P, ctypes.c_size_t, _P, ctypes.c_size_t, ctypes.c_size_t, _P, _P,
                                     ctypes.c_size_t, ctypes.POINTER(_P)]),
    "vk_ivf_destroy": (None, [_P]),
    "vk_ivf_assign": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.c_size_t, _P, ctypes.c_size_t, _P]),
    "vk_ivf_set_tuning": (ctypes.c_int, [_P, ctypes.POINTER(_Tuning)]),
    "vk_ivf_last_launch": (ctypes.c_int, [_P, ctypes.POINTER(_LaunchShape)]),
    "vk_ivf_search": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _P,
                                     ctypes.POINTER(_Timings)]),
    "vk_ivf_search_device": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _P,
                                            ctypes.POINTER(_Timings)]),
    "vk_pq_encode": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.c_size_t, _P, ctypes.c_size_t, _P]),
    "vk_pq_encode_device": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.c_size_t, _P, ctypes.c_size_t, _P]),
    "vk_pq_assign": (ctypes.c_int, [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P]),
    "vk_reranker_create": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.c_size_t, ctypes.POINTER(_P)]),
    "vk_reranker_destroy": (None, [_P]),
    "vk_rerank": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, ctypes.c_size_t, _P,
                                 ctypes.POINTER(_Timings)]),
    "vk_rerank_device": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, ctypes.c_size_t, _P,
                                        ctypes.POINTER(_Timings)]),
}

_lib = None


def library() -> ctypes.CDLL:
    """Loads lib/libveckern.so once and declares every exported signature. Raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                              "(or `make -C veckern_amd`) first; there is no CPU fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc == VK_OK:
        return
    msg = library().vk_last_error().decode()
    if rc == VK_ERR_INVALID_ARGUMENT:
        raise VkInvalidArgument(rc, msg)
    if rc == VK_ERR_LOGIC:
        raise VkLogicError(rc, msg)
    raise VkError(rc, msg)


@dataclass
class Tuning:
    """veckern::gpu::Tuning (reference gpu.hpp:29-34)."""

    scan_threads: int = 256
    blocks_per_query: int = 0
    queries_per_block: int = 2
    vectors_per_step: int = 4

    def _c(self) -> _Tuning:
        return _Tuning(self.scan_threads, self.blocks_per_query, self.queries_per_block, self.vectors_per_step)


@dataclass
class Timings:
    """veckern::gpu::Timings (reference gpu.hpp:46-50): milliseconds per stage, from HIP events."""

    transfer_ms: float = 0.0
    lut_ms: float = 0.0
    scan_ms: float = 0.0
    select_ms: float = 0.0

    def kernel_ms(self) -> float:
        return self.lut_ms + self.scan_ms + self.select_ms

    def total_ms(self) -> float:
        return self.transfer_ms + self.kernel_ms()


@dataclass
class LaunchShape:
    """veckern::gpu::PQSearcher::LaunchShape (reference gpu.hpp:67-73)."""

    threads: int = 0
    blocks_x: int = 0
    grid_y: int = 0
    queries_per_block: int = 1
    vectors_per_step: int = 1
    blocks_per_sm: int = 0
    waves: float = 0.0


@dataclass
class DeviceInfo:
    """veckern::gpu::DeviceInfo (reference gpu.hpp:36-43) plus architecture, clock, L2 and memory size."""

    name: str
    arch: str
    sm_count: int
    peak_bandwidth_gbs: float
    max_smem_per_block: int
    clock_khz: int
    warp_size: int
    l2_bytes: int
    total_mem_bytes: int


def variant_name(v: int) -> str:
    """Reference gpu.hpp:25, names as searcher.cu:123-136."""
    return library().vk_variant_name(int(v)).decode()


def is_fused(v: int) -> bool:
    """Reference gpu.hpp:26."""
    return bool(library().vk_is_fused(int(v)))


def needs_m16(v: int) -> bool:
    return bool(library().vk_needs_m16(int(v)))


def dispatched_k(k: int) -> int:
    """List length used for k (searcher.cu:86-90); raises VkInvalidArgument for k > 128."""
    K = library().vk_dispatched_k(k)
    if K == 0:
        raise VkInvalidArgument(VK_ERR_INVALID_ARGUMENT, library().vk_last_error().decode())
    return K


def validate_tuning(t: Tuning) -> None:
    """PQSearcher::set_tuning's checks (searcher.cu:450-460) without a searcher."""
    c = t._c()
    _check(library().vk_tuning_validate(ctypes.byref(c)))


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(library().vk_get_device_count(ctypes.byref(n)))
    return n.value


def device_info(device: int = 0) -> DeviceInfo:
    """Reference gpu.hpp:42 device_info()."""
    d = _DeviceInfo()
    _check(library().vk_get_device_info(device, ctypes.byref(d)))
    return DeviceInfo(d.name.decode(), d.arch.decode(), d.sm_count, d.peak_bandwidth_gbs, d.max_smem_per_block,
                      d.clock_khz, d.warp_size, d.l2_bytes, d.total_mem_bytes)


def _timings(t: _Timings) -> Timings:
    return Timings(t.transfer_ms, t.lut_ms, t.scan_ms, t.select_ms)


class PQSearcher:
    """veckern::gpu::PQSearcher (reference gpu.hpp:52-78) over the C ABI.

    ``centroids``: float32 [m][256][d/m] (pq.hpp:20-24); ``codes``: uint8 row-major n x m. Both are copied to the
    device once. Results come back ascending by (dist, id) with {+inf, -1} padding.
    """

    def __init__(self, centroids: np.ndarray, codes: np.ndarray, d: int | None = None):
        lib = library()
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        if codes.ndim != 2:
            raise ValueError("codes must be n x m")
        self.n, self.m = codes.shape
        cent = np.ascontiguousarray(centroids, dtype=np.float32)
        self.d = int(d) if d is not None else int(cent.size // 256)
        self._h = ctypes.c_void_p()
        _check(lib.vk_searcher_create(cent.ctypes.data, self.d, self.m, codes.ctypes.data, self.n,
                                      ctypes.byref(self._h)))

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            library().vk_searcher_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_tuning(self, t: Tuning) -> None:
        c = t._c()
        _check(library().vk_searcher_set_tuning(self._h, ctypes.byref(c)))

    def tuning(self) -> Tuning:
        c = _Tuning()
        _check(library().vk_searcher_get_tuning(self._h, ctypes.byref(c)))
        return Tuning(c.scan_threads, c.blocks_per_query, c.queries_per_block, c.vectors_per_step)

    def layout(self):
        """The v8/v9 code layout (vk_searcher_layout): (ids, rows, lanes). ids: per slot of n padded to 256, the id
        of the vector scanned there, interleaved by four tiles; rows: [m][256] LDS table row of each code value;
        lanes: lanes per table-read pass the layout was built for."""
        ids = np.empty((self.n + 255) // 256 * 256, dtype=np.uint32)
        rows = np.empty((self.m, 256), dtype=np.uint8)
        lanes = ctypes.c_int(0)
        _check(library().vk_searcher_layout(self._h, ids.ctypes.data, ids.size, rows.ctypes.data, rows.size,
                                            ctypes.byref(lanes)))
        return ids, rows, lanes.value

    def last_launch(self) -> LaunchShape:
        s = _LaunchShape()
        _check(library().vk_searcher_last_launch(self._h, ctypes.byref(s)))
        return LaunchShape(s.threads, s.blocks_x, s.grid_y, s.queries_per_block, s.vectors_per_step,
                           s.blocks_per_sm, s.waves)

    def search(self, queries: np.ndarray, k: int, variant: int = ScanVariant.FusedWarp):
        """Returns (dist [nq, k] float32, ids [nq, k] int32, Timings)."""
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.d)
        out = np.empty((q.shape[0], k), dtype=NEIGHBOR_DTYPE)
        t = _Timings()
        _check(library().vk_search(self._h, q.ctypes.data, q.shape[0], k, int(variant), out.ctypes.data,
                                   ctypes.byref(t)))
        return out["dist"].copy(), out["id"].copy(), _timings(t)

    def distances(self, queries: np.ndarray, variant: int = ScanVariant.GlobalLut):
        """Returns (dist [nq, n] float32, Timings); unfused variants v0-v3 only."""
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.d)
        out = np.empty((q.shape[0], self.n), dtype=np.float32)
        t = _Timings()
        _check(library().vk_distances(self._h, q.ctypes.data, q.shape[0], int(variant), out.ctypes.data,
                                      ctypes.byref(t)))
        return out, _timings(t)

    def search_device(self, d_queries: int, nq: int, k: int, variant: int, d_out: int) -> Timings:
        """Device-resident search: d_queries / d_out are device addresses (nq x d float32, nq x k pairs)."""
        t = _Timings()
        _check(library().vk_search_device(self._h, ctypes.c_void_p(d_queries), nq, k, int(variant),
                                          ctypes.c_void_p(d_out), ctypes.byref(t)))
        return _timings(t)

    def search_device_noalloc(self, d_queries: int, nq: int, k: int, variant: int, d_out: int) -> None:
        """search_device without any device allocation (v8 / v9): scratch is the library's static device array."""
        _check(library().vk_search_device_noalloc(self._h, ctypes.c_void_p(d_queries), nq, k, int(variant),
                                                  ctypes.c_void_p(d_out)))


def pq_encode(centroids: np.ndarray, x: np.ndarray) -> np.ndarray:
    """GPU PQ encoding (ProductQuantizer::encode, pq.cpp:70-75): codes n x m, identical to the CPU encoder."""
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    m = c.shape[0]
    xs = np.ascontiguousarray(x, dtype=np.float32)
    n, d = xs.shape
    codes = np.empty((n, m), dtype=np.uint8)
    _check(library().vk_pq_encode(c.ctypes.data, d, m, xs.ctypes.data, n, codes.ctypes.data))
    return codes


def pq_assign(centroids: np.ndarray, sub: np.ndarray) -> np.ndarray:
    """GPU k-means assignment step for one sub-space: nearest of the 256 centroids (256 x dsub) per row of sub."""
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    s = np.ascontiguousarray(sub, dtype=np.float32)
    out = np.empty(s.shape[0], dtype=np.uint32)
    _check(library().vk_pq_assign(c.ctypes.data, c.shape[-1], s.ctypes.data, s.shape[0], out.ctypes.data))
    return out


def ivf_assign(coarse: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Nearest coarse centroid (exact, lower index on ties) of every row of x, on the GPU: int32 list ids."""
    co = np.ascontiguousarray(coarse, dtype=np.float32)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(xs.shape[0], dtype=np.int32)
    _check(library().vk_ivf_assign(co.ctypes.data, co.shape[0], co.shape[1], xs.ctypes.data, xs.shape[0],
                                   out.ctypes.data))
    return out


class IVFIndex:
    """Inverted-file PQ search on the GPU (vk_ivf_*): coarse float32 nlist x d, PQ centroids [m][256][d/m],
    codes uint8 n x m (of the raw vectors), list_ids int32 n (each in [0, nlist)). search() probes each query's
    nprobe nearest lists and returns the k best of their vectors, bit-identical to the exhaustive search restricted
    to those lists.
    """

    def __init__(self, coarse: np.ndarray, centroids: np.ndarray, codes: np.ndarray, list_ids: np.ndarray):
        lib = library()
        co = np.ascontiguousarray(coarse, dtype=np.float32)
        cent = np.ascontiguousarray(centroids, dtype=np.float32)
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        li = np.ascontiguousarray(list_ids, dtype=np.int32)
        self.n, self.m = codes.shape
        self.nlist, self.d = co.shape
        if li.shape != (self.n,):
            raise ValueError("list_ids must have one entry per code row")
        self._h = ctypes.c_void_p()
        _check(lib.vk_ivf_create(co.ctypes.data, self.nlist, cent.ctypes.data, self.d, self.m, codes.ctypes.data,
                                 li.ctypes.data, self.n, ctypes.byref(self._h)))

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            library().vk_ivf_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_tuning(self, t: Tuning) -> None:
        c = t._c()
        _check(library().vk_ivf_set_tuning(self._h, ctypes.byref(c)))

    def last_launch(self) -> LaunchShape:
        s = _LaunchShape()
        _check(library().vk_ivf_last_launch(self._h, ctypes.byref(s)))
        return LaunchShape(s.threads, s.blocks_x, s.grid_y, s.queries_per_block, s.vectors_per_step,
                           s.blocks_per_sm, s.waves)

    def search(self, queries: np.ndarray, nprobe: int, k: int):
        """Returns (dist [nq, k] float32, ids [nq, k] int32, Timings)."""
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.d)
        out = np.empty((q.shape[0], k), dtype=NEIGHBOR_DTYPE)
        t = _Timings()
        _check(library().vk_ivf_search(self._h, q.ctypes.data, q.shape[0], nprobe, k, out.ctypes.data,
                                       ctypes.byref(t)))
        return out["dist"].copy(), out["id"].copy(), _timings(t)

    def search_device(self, d_queries: int, nq: int, nprobe: int, k: int, d_out: int) -> Timings:
        """Device-resident search: d_queries / d_out are device addresses (nq x d float32, nq x k pairs)."""
        t = _Timings()
        _check(library().vk_ivf_search_device(self._h, ctypes.c_void_p(d_queries), nq, nprobe, k,
                                              ctypes.c_void_p(d_out), ctypes.byref(t)))
        return _timings(t)


class Reranker:
    """Exact re-ranking on the GPU (the reference's CPU rerank_exact, cpu_ref.cpp:66-77): base vectors float32
    n x d are copied to the device once; rerank() re-scores nq x r candidates (NEIGHBOR_DTYPE records, ids < 0
    skipped) with the exact squared L2 distance and keeps the k smallest by (dist, id).
    """

    def __init__(self, base: np.ndarray):
        lib = library()
        b = np.ascontiguousarray(base, dtype=np.float32)
        if b.ndim != 2:
            raise ValueError("base must be n x d")
        self.n, self.d = b.shape
        self._h = ctypes.c_void_p()
        _check(lib.vk_reranker_create(b.ctypes.data, self.n, self.d, ctypes.byref(self._h)))

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            library().vk_reranker_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def rerank(self, queries: np.ndarray, candidates: np.ndarray, k: int):
        """Returns (dist [nq, k] float32, ids [nq, k] int32, Timings)."""
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.d)
        c = np.ascontiguousarray(candidates, dtype=NEIGHBOR_DTYPE)
        if c.ndim != 2 or c.shape[0] != q.shape[0]:
            raise ValueError("candidates must be nq x r")
        out = np.empty((q.shape[0], k), dtype=NEIGHBOR_DTYPE)
        t = _Timings()
        _check(library().vk_rerank(self._h, q.ctypes.data, q.shape[0], c.ctypes.data, c.shape[1], k,
                                   out.ctypes.data, ctypes.byref(t)))
        return out["dist"].copy(), out["id"].copy(), _timings(t)

    def rerank_device(self, d_queries: int, nq: int, d_candidates: int, r: int, k: int, d_out: int) -> Timings:
        """Device-resident form: queries nq x d, candidates nq x r pairs, out nq x k pairs (device addresses)."""
        t = _Timings()
        _check(library().vk_rerank_device(self._h, ctypes.c_void_p(d_queries), nq, ctypes.c_void_p(d_candidates),
                                          r, k, ctypes.c_void_p(d_out), ctypes.byref(t)))
        return _timings(t)


class DeviceArray:
    """A device buffer from the HIP runtime that libveckern.so itself uses (no second runtime in the process).

    Plumbing for callers whose inputs should already be resident in HBM (benchmarks, device-path tests).
    """

    _hip = None

    @classmethod
    def _runtime(cls):
        if cls._hip is None:
            library()  # loads libamdhip64.so.7 as a dependency; the handle below refers to that same copy
            hip = ctypes.CDLL("libamdhip64.so.7")
            hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
            hip.hipFree.argtypes = [ctypes.c_void_p]
            hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            hip.hipDeviceSynchronize.argtypes = []
            cls._hip = hip
        return cls._hip

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        rc = self._runtime().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1))
        if rc != 0:
            raise VkError(VK_ERR_OUT_OF_MEMORY, f"hipMalloc({self.nbytes}) failed with {rc}")

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        rc = self._runtime().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, 1)  # hipMemcpyHostToDevice
        if rc != 0:
            raise VkError(VK_ERR_DEVICE, f"hipMemcpy H2D failed with {rc}")

    def download(self, out: np.ndarray) -> np.ndarray:
        if out.nbytes > self.nbytes or not out.flags["C_CONTIGUOUS"]:
            raise ValueError("output must be contiguous and no larger than the device buffer")
        rc = self._runtime().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2)  # hipMemcpyDeviceToHost
        if rc != 0:
            raise VkError(VK_ERR_DEVICE, f"hipMemcpy D2H failed with {rc}")
        return out

    @property
    def address(self) -> int:
        return int(self.ptr.value or 0)

    def free(self) -> None:
        if self.ptr.value:
            self._runtime().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
