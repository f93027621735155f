"""GPU PQ encoding and the k-means assignment step (vk_pq_encode / vk_pq_assign) against the oracle's restatement
of the reference's nearest_centroid (pq.cpp:11-22): codes must be identical, ties (duplicated centroids) going to
the lowest index. Training with the GPU assignment is checked against CPU training in tests/cpp/test_gpu_api.cpp.
"""
import numpy as np
import pytest

import veckern_amd as vk
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def case(seed, n, d, m, ties=False, scale=1.0):
    rng = np.random.default_rng(seed)
    if ties:
        cent = rng.integers(0, 3, size=(m, 256, d // m)).astype(np.float32)
        x = rng.integers(0, 3, size=(n, d)).astype(np.float32)
    else:
        cent = (rng.standard_normal((m, 256, d // m)) * scale).astype(np.float32)
        x = (rng.standard_normal((n, d)) * scale).astype(np.float32)
    cent[:, 200] = cent[:, 7]  # a duplicated centroid in every sub-space
    return cent, x


@pytest.mark.parametrize("d,m", [(128, 16), (128, 32), (128, 64), (64, 4), (96, 48), (30, 10), (128, 1)])
def test_encode_matches_oracle(d, m):
    cent, x = case(80 + m, 20_011, d, m)
    assert (vk.pq_encode(cent, x) == orc.pq_encode(cent, x)).all()


@pytest.mark.parametrize("scale", [1e-20, 1e15])
def test_encode_extreme_scales_and_ties(scale):
    cent, x = case(81, 5_003, 64, 16, scale=scale)
    assert (vk.pq_encode(cent, x) == orc.pq_encode(cent, x)).all()
    cent, x = case(82, 5_003, 64, 16, ties=True)
    assert (vk.pq_encode(cent, x) == orc.pq_encode(cent, x)).all()


def test_assign_matches_oracle():
    cent, x = case(83, 50_000, 8, 1)
    got = vk.pq_assign(cent[0], x)
    assert (got == orc.pq_encode(cent, x)[:, 0]).all()


def test_encode_rejects_bad_shapes():
    cent, x = case(84, 10, 64, 16)
    codes = np.empty((10, 16), dtype=np.uint8)
    lib = vk.library()
    assert lib.vk_pq_encode(cent.ctypes.data, 64, 0, x.ctypes.data, 10, codes.ctypes.data) != 0  # m = 0
    assert lib.vk_pq_encode(cent.ctypes.data, 64, 7, x.ctypes.data, 10, codes.ctypes.data) != 0  # d % m != 0
    assert lib.vk_pq_encode(None, 64, 16, x.ctypes.data, 10, codes.ctypes.data) != 0
