"""The allocation-free search (vk_search_device_noalloc) against the device-resident search it mirrors
(vk_search_device), through the C ABI: identical ids and distance bits, on two calls in a row with the second one
smaller (the static scratch keeps the first call's contents), for fp32 (v8) and fp16 (v9) tables and k up to 100.
Also: no device memory is taken by the call, searches beyond the static scratch are rejected before any launch, and
the preconditions (v8/v9 only, code layout already built) are errors.
"""
import ctypes

import numpy as np
import pytest

import veckern_amd as vk
from tests import datagen

pytestmark = pytest.mark.gpu

SENTINEL = np.array([(-7.0, -7)], dtype=vk.NEIGHBOR_DTYPE)


def free_device_bytes():
    hip = vk.DeviceArray._runtime()
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def search_pair(s, queries, k, variant):
    """(vk_search_device result, vk_search_device_noalloc result, free bytes before and after the latter)."""
    nq = queries.shape[0]
    dq = vk.DeviceArray.from_host(np.ascontiguousarray(queries, dtype=np.float32))
    d_ref = vk.DeviceArray(nq * k * vk.NEIGHBOR_DTYPE.itemsize)
    d_new = vk.DeviceArray(nq * k * vk.NEIGHBOR_DTYPE.itemsize)
    try:
        d_new.upload(np.repeat(SENTINEL, nq * k))
        s.search_device(dq.address, nq, k, variant, d_ref.address)
        before = free_device_bytes()
        s.search_device_noalloc(dq.address, nq, k, variant, d_new.address)
        after = free_device_bytes()
        ref = d_ref.download(np.empty((nq, k), dtype=vk.NEIGHBOR_DTYPE))
        new = d_new.download(np.empty((nq, k), dtype=vk.NEIGHBOR_DTYPE))
    finally:
        dq.free()
        d_ref.free()
        d_new.free()
    return ref, new, before, after


def assert_same(ref, new, label):
    assert (new["id"] == ref["id"]).all(), label
    assert (new["dist"].view(np.uint32) == ref["dist"].view(np.uint32)).all(), label


@pytest.mark.parametrize("m,k,variant,q", [(16, 10, vk.ScanVariant.FusedWarp, 4), (32, 100, vk.ScanVariant.FusedWarp, 4),
                                           (16, 10, vk.ScanVariant.FusedWarpF16, 8), (16, 1, vk.ScanVariant.FusedWarp, 1)])
def test_noalloc_matches_search_device_on_two_calls(m, k, variant, q):
    centroids, codes, queries = datagen.random_fixture(200_003, 128, m, 300, seed=31 + m + k)
    with vk.PQSearcher(centroids, codes, 128) as s:
        s.set_tuning(vk.Tuning(queries_per_block=q))
        for nq in (300, 23):  # the second call is smaller: it must not see the first call's scratch contents
            print(f"    [noalloc] m={m} k={k} {vk.variant_name(variant)} Q={q} nq={nq}", flush=True)
            ref, new, before, after = search_pair(s, queries[:nq], k, variant)
            assert_same(ref, new, f"m={m} k={k} {vk.variant_name(variant)} nq={nq}")
            if nq == 23:  # by the second call every kernel of the path has run in this process
                assert after == before, "the allocation-free search changed the device's free memory"


def test_noalloc_single_query_over_many_blocks():
    # one slab spread over up to one block per CU: block-merged partial lists in the static scratch
    centroids, codes, queries = datagen.random_fixture(1_000_003, 128, 16, 3, seed=5)
    with vk.PQSearcher(centroids, codes, 128) as s:
        for nq in (3, 1):
            ref, new, _, _ = search_pair(s, queries[:nq], 10, vk.ScanVariant.FusedWarp)
            assert_same(ref, new, f"nq={nq}")


def test_noalloc_rejects_searches_beyond_its_scratch_before_launch():
    centroids, codes, queries = datagen.random_fixture(100_003, 128, 16, 4, seed=9)
    nq, k = 20_000, 128  # 5000 slabs x 4 queries x 8 lists x 128 pairs x 8 bytes = 164 MB of partial lists
    big = np.tile(queries, (nq // 4, 1))
    with vk.PQSearcher(centroids, codes, 128) as s:
        s.set_tuning(vk.Tuning(queries_per_block=4))
        s.search(queries, 10, vk.ScanVariant.FusedWarp)  # builds the code layout
        dq = vk.DeviceArray.from_host(big)
        dout = vk.DeviceArray(nq * k * vk.NEIGHBOR_DTYPE.itemsize)
        try:
            dout.upload(np.repeat(SENTINEL, nq * k))
            with pytest.raises(vk.VkInvalidArgument, match="beyond its static scratch"):
                s.search_device_noalloc(dq.address, nq, k, vk.ScanVariant.FusedWarp, dout.address)
            untouched = dout.download(np.empty(nq * k, dtype=vk.NEIGHBOR_DTYPE))
            assert (untouched["id"] == -7).all(), "a rejected search wrote results"
            # a search that fits still runs after the rejection
            ref, new, _, _ = search_pair(s, queries, 10, vk.ScanVariant.FusedWarp)
            assert_same(ref, new, "after a rejection")
        finally:
            dq.free()
            dout.free()


def test_noalloc_preconditions():
    centroids, codes, queries = datagen.random_fixture(10_007, 64, 16, 5, seed=3)
    with vk.PQSearcher(centroids, codes, 64) as s:
        dq = vk.DeviceArray.from_host(queries)
        dout = vk.DeviceArray(5 * 10 * vk.NEIGHBOR_DTYPE.itemsize)
        try:
            with pytest.raises(vk.VkLogicError, match="layout is not built"):
                s.search_device_noalloc(dq.address, 5, 10, vk.ScanVariant.FusedWarp, dout.address)
            s.search(queries, 10, vk.ScanVariant.FusedWarp)
            with pytest.raises(vk.VkInvalidArgument, match="v8_fused_warp and v9_fused_warp_f16 only"):
                s.search_device_noalloc(dq.address, 5, 10, vk.ScanVariant.FusedVecMQ, dout.address)
            with pytest.raises(vk.VkError, match="k must be"):
                s.search_device_noalloc(dq.address, 5, 129, vk.ScanVariant.FusedWarp, dout.address)
            s.search_device_noalloc(dq.address, 0, 10, vk.ScanVariant.FusedWarp, dout.address)  # nq = 0: no-op
        finally:
            dq.free()
            dout.free()
