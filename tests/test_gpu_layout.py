"""The v8/v9 code layout a searcher builds on the GPU (slot_order.hip), read back through vk_searcher_layout.

Its invariants: every vector in exactly one slot of [0, n) (ids interleaved by four tiles), padding slots 0, each
sub-space's table rows a permutation of 0..255, and the pass width of the first v8/v9 search's table reads (16
lanes for 16-byte entries, 32 for 8-byte, 64 for 4-byte). Searches through the layout equal the oracle's results
bit for bit; the slot-for-slot equality with the host definition (slot_order.hpp) is checked by
tests/cpp/test_gpu_api.cpp.
"""
import numpy as np
import pytest

import veckern_amd as vk
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def interleaved(slot):
    tile, lane = slot // 64, slot % 64
    return (tile // 4) * 256 + lane * 4 + tile % 4


def check_layout(ids, rows, n, m):
    n_pad = (n + 255) // 256 * 256
    assert ids.shape == (n_pad,) and rows.shape == (m, 256)
    slots = np.arange(n_pad)
    by_slot = ids[interleaved(slots)]
    assert np.array_equal(np.sort(by_slot[:n]), np.arange(n, dtype=np.uint32)), "every vector in one slot"
    assert not by_slot[n:].any(), "padding slots hold 0"
    assert all(np.array_equal(np.sort(rows[s]), np.arange(256)) for s in range(m)), "rows are permutations"


@pytest.mark.parametrize("q, lanes", [(0, 16), (4, 16), (2, 32), (1, 64)])
def test_layout_invariants_and_width(q, lanes):
    rng = np.random.default_rng(3 + q)
    n, d, m = 30_011, 64, 32
    centroids = rng.standard_normal((m, 256, d // m)).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    queries = rng.standard_normal((5, d)).astype(np.float32)
    with vk.PQSearcher(centroids, codes, d) as s:
        if q:
            s.set_tuning(vk.Tuning(queries_per_block=q))
            got_d, got_i, _ = s.search(queries, 10, vk.ScanVariant.FusedWarp)
            exp = orc.adc_search(centroids, d, codes, queries, 10)
            assert np.array_equal(got_i, exp["id"]) and np.array_equal(got_d.view(np.uint32), exp["dist"].view(np.uint32))
        ids, rows, got_lanes = s.layout()
        assert got_lanes == lanes
        check_layout(ids, rows, n, m)
        # A later search with another width reuses the layout as built and still returns the oracle's results.
        s.set_tuning(vk.Tuning(queries_per_block=2 if q != 2 else 4))
        got_d, got_i, _ = s.search(queries, 7, vk.ScanVariant.FusedWarp)
        exp = orc.adc_search(centroids, d, codes, queries, 7)
        assert np.array_equal(got_i, exp["id"]) and np.array_equal(got_d.view(np.uint32), exp["dist"].view(np.uint32))
        assert s.layout()[2] == lanes


def test_layout_rows_move_co_read_entries_apart():
    # Clustered codes whose vectors draw each sub-space's entry from a set that shares one bank group (entry % 16):
    # with rows = codes every pass would queue its entries in one group; the fitted rows must spread them.
    rng = np.random.default_rng(8)
    n, d, m = 64 * 256, 32, 16
    cluster = rng.integers(0, 64, size=n)
    codes = np.empty((n, m), dtype=np.uint8)
    for s in range(m):
        base = (cluster * 7 + s * 3) % 16
        codes[:, s] = (cluster * 4 + rng.integers(0, 4, size=n)) if s < 4 else base + 16 * rng.integers(0, 16, size=n)
    centroids = rng.standard_normal((m, 256, d // m)).astype(np.float32)
    with vk.PQSearcher(centroids, codes, d) as s:
        ids, rows, lanes = s.layout()
        assert lanes == 16
        check_layout(ids, rows, n, m)
        order = ids[interleaved(np.arange(n))]
        def load(groups_of):
            total = 0
            for p0 in range(0, n, 16):
                for sub in range(m):
                    e = np.unique(codes[order[p0:p0 + 16], sub])
                    total += np.bincount(groups_of(sub, e), minlength=16).max()
            return total / (n // 16 * m)
        plain = load(lambda sub, e: e % 16)
        fitted = load(lambda sub, e: rows[sub, e] % 16)
        print(f"\n    bank load of the GPU layout: rows = codes {plain:.3f}, fitted rows {fitted:.3f}")
        assert fitted < 0.8 * plain


def test_layout_beyond_64_subspaces_is_built_on_the_host():
    # m = 128: the GPU builder's LDS sizing covers m <= 64, so the searcher builds this layout with the host
    # definition; its tables (128 KB for one query) still fit, so the search runs at one query per block.
    rng = np.random.default_rng(21)
    n, d, m = 5_003, 256, 128
    centroids = rng.standard_normal((m, 256, d // m)).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    queries = rng.standard_normal((6, d)).astype(np.float32)
    with vk.PQSearcher(centroids, codes, d) as s:
        got_d, got_i, _ = s.search(queries, 10, vk.ScanVariant.FusedWarp)
        assert s.last_launch().queries_per_block == 1
        exp = orc.adc_search(centroids, d, codes, queries, 10)
        assert np.array_equal(got_i, exp["id"]) and np.array_equal(got_d.view(np.uint32), exp["dist"].view(np.uint32))
        ids, rows, lanes = s.layout()
        assert lanes == 64
        check_layout(ids, rows, n, m)
