"""GPU results against the golden fixtures written from the reference's own CPU code (tests/golden/*.npz):
distances of every unfused variant and searches of every fused variant, bit for bit. tiny_diffs.npz puts
subnormal values in the LUT, so a GPU LUT build that flushed denormals to zero would fail here."""
import os

import numpy as np
import pytest

import veckern_amd as vk

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["clustered_m8.npz", "clustered_m16.npz", "ties_m16.npz", "tiny_diffs.npz"]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("name", FIXTURES)
def test_gpu_matches_reference_golden(name):
    z = np.load(os.path.join(GOLDEN, name))
    d, m = int(z["d"]), z["codes"].shape[1]
    with vk.PQSearcher(z["centroids"], z["codes"], d) as s:
        for v in vk.ScanVariant:
            if vk.is_fused(v) or (vk.needs_m16(v) and m % 16):
                continue
            got, _ = s.distances(z["queries"], v)
            assert (bits(got) == bits(z["dists"])).all(), f"{name} {vk.variant_name(v)} distances"
        ks = sorted(int(key[len("search_k"):-3]) for key in z.files if key.startswith("search_k") and key.endswith("_id"))
        for v in vk.ScanVariant:
            # v4 is rejected before launch; v9's fp16 tables are checked against their own restatement
            if v in (vk.ScanVariant.Fused, vk.ScanVariant.FusedWarpF16) or (vk.needs_m16(v) and m % 16):
                continue
            for q in ((1, 2, 4, 8) if v == vk.ScanVariant.FusedWarp else (2,)):
                s.set_tuning(vk.Tuning(queries_per_block=q))
                for k in ks:
                    dist, ids, _ = s.search(z["queries"], k, v)
                    assert (ids == z[f"search_k{k}_id"]).all(), f"{name} {vk.variant_name(v)} Q={q} k={k} ids"
                    assert (bits(dist) == bits(z[f"search_k{k}_dist"])).all(), f"{name} {vk.variant_name(v)} k={k}"
