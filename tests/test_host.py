"""Host tools on the CPU (lib/libveckern_cpu.so): the Philox generator, synthetic data, the PQ codec and the
recall helpers, plus the C++ host test program."""
import os
import subprocess

import numpy as np
import pytest

from oracle import binding as orc
from veckern_amd import NEIGHBOR_DTYPE, host

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp", "_build")


def test_philox_known_answers():
    # Random123 philox4x32-10 known-answer vectors (Salmon et al., SC 2011).
    assert [hex(v) for v in host.philox4x32_10([0, 0, 0, 0], [0, 0])] == \
        ["0x6627e8d5", "0xe169c58d", "0xbc57ac4c", "0x9b00dbd8"]
    assert [hex(v) for v in host.philox4x32_10([0xffffffff] * 4, [0xffffffff] * 2)] == \
        ["0x408f276d", "0x41c83b0e", "0xa20bc7c6", "0x6d5451fd"]
    assert [hex(v) for v in host.philox4x32_10([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344],
                                               [0xa4093822, 0x299f31d0])] == \
        ["0xd16cfe09", "0x94fdcceb", "0x5001e420", "0x24126ea1"]


def test_normal_stream_moments_and_range_independence():
    v = host.normal_values(3, 31, 0, 400_000)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1) < 0.01
    assert (host.normal_values(3, 31, 1000, 50) == v[1000:1050]).all()


def test_mixture_rows_are_addressable_and_clustered():
    a = host.gaussian_mixture(32, 50, 0.3, 7, 0, 2000)
    b = host.gaussian_mixture(32, 50, 0.3, 7, 1500, 500)
    assert (a[1500:] == b).all()
    assert not (a[0] == a[1]).all()
    # the nearest other row is far closer than a typical pair (sigma 0.3 around N(0, 1) centres)
    d2 = ((a[:200, None, :] - a[None, :, :]) ** 2).sum(-1)
    np.fill_diagonal(d2[:, :200], np.inf)
    assert np.median(d2.min(1)) < 0.25 * np.median(d2)


def test_uniform_codes_are_uniform_and_addressable():
    c = host.uniform_codes(0, 100_000, 16, 1)
    counts = np.bincount(c.ravel(), minlength=256)
    expected = c.size / 256
    assert ((counts - expected) ** 2 / expected).sum() < 400  # chi-square, 255 degrees of freedom
    assert (host.uniform_codes(777, 10, 16, 1) == c[777:787]).all()


def test_pq_encode_is_nearest_centroid():
    x = host.gaussian_mixture(32, 20, 0.3, 2, 0, 3000)
    cent = host.pq_train(x, 8, 5, seed=4)
    codes = host.pq_encode(cent, x)
    sub = x.reshape(3000, 8, 4)
    d2 = ((sub[:, :, None, :] - cent[None, :, :, :]) ** 2).sum(-1)
    chosen = np.take_along_axis(d2, codes[:, :, None].astype(np.int64), axis=2)[..., 0]
    assert (chosen <= d2.min(-1) * (1 + 1e-5) + 1e-9).all()
    assert (host.pq_train(x, 8, 5, seed=4) == cent).all()


def test_exact_knn_matches_numpy_and_recall_matches_oracle():
    base = host.gaussian_mixture(24, 30, 0.3, 5, 0, 3000)
    q = host.gaussian_mixture(24, 30, 0.3, 5, 1 << 40, 20)
    gt = host.exact_knn(base, q, 10)
    d2 = ((q.astype(np.float64)[:, None, :] - base[None, :, :]) ** 2).sum(-1)
    assert (gt["id"] == np.argsort(d2, axis=1, kind="stable")[:, :10]).all()
    rng = np.random.default_rng(0)
    found = np.zeros((20, 12), dtype=NEIGHBOR_DTYPE)
    found["id"] = rng.integers(-1, 3000, size=(20, 12))
    found["id"][:, :5] = gt["id"][:, :5]
    truth = gt["id"].astype(np.int32)
    for k in (1, 5, 10):
        assert host.recall_at_k(found, truth, k) == orc.recall_at_k(found, truth, k)


def test_rerank_improves_pq_recall():
    base = host.gaussian_mixture(32, 20, 0.3, 6, 0, 4000)
    q = host.gaussian_mixture(32, 20, 0.3, 6, 1 << 40, 12)
    cent = host.pq_train(base, 8, 10)
    codes = host.pq_encode(cent, base)
    gt = host.exact_knn(base, q, 10)["id"].astype(np.int32)
    approx = orc.adc_search(cent, 32, codes, q, 100)
    approx_nb = np.zeros(approx.shape, dtype=NEIGHBOR_DTYPE)
    approx_nb["dist"], approx_nb["id"] = approx["dist"], approx["id"]
    reranked = host.rerank_exact(base, q, approx_nb, 10)
    pq_recall = host.recall_at_k(approx_nb, gt, 10)
    rr_recall = host.recall_at_k(reranked, gt, 10)
    assert rr_recall >= pq_recall and rr_recall > 0.8


@pytest.mark.parametrize("program", ["test_host", "test_planning"])
def test_cpp_host_programs(program, tmp_path):
    exe = os.path.join(CPP, program)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} not built: run `make -C tests/cpp`")
    r = subprocess.run([exe], cwd=tmp_path, capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_vector_file_known_answers(tmp_path):
    # the reference's fvecs case (test_cpu.cpp:117-135): rows r*10 + j, d=4, at most 2 rows read
    rows = (np.arange(3)[:, None] * 10 + np.arange(4)[None, :]).astype(np.float32)
    p = str(tmp_path / "t.fvecs")
    host.write_fvecs(p, rows)
    raw = np.fromfile(p, dtype="<i4")
    assert raw.size == 15 and (raw[::5] == 4).all()  # int32 dimension before each row
    got = host.read_fvecs(p, max_n=2)
    assert got.shape == (2, 4) and got.ravel()[4] == 10.0 and got.ravel()[7] == 13.0
    ids = np.array([[0, 1, 2], [100, 101, 102]], dtype=np.int32)
    host.write_ivecs(str(tmp_path / "t.ivecs"), ids)
    assert (host.read_ivecs(str(tmp_path / "t.ivecs")) == ids).all()
    host.write_bvecs(str(tmp_path / "t.bvecs"), np.array([[7, 250]], dtype=np.uint8))
    b = host.read_bvecs(str(tmp_path / "t.bvecs"))
    assert b.dtype == np.float32 and b.tolist() == [[7.0, 250.0]]


def test_vector_file_errors(tmp_path):
    p = str(tmp_path / "bad.fvecs")
    host.write_fvecs(p, np.ones((2, 3), np.float32))
    with open(p, "ab") as f:
        f.write(b"\x00\x00")  # a truncated third row
    with pytest.raises(ValueError):
        host.read_fvecs(p)
    q = str(tmp_path / "mixed.fvecs")
    with open(q, "wb") as f:
        np.array([2], "<i4").tofile(f)
        np.ones(2, "<f4").tofile(f)
        np.array([1], "<i4").tofile(f)
        np.ones(2, "<f4").tofile(f)  # second row claims d=1 but the byte count matches two rows of d=2
    with pytest.raises(ValueError):
        host.read_fvecs(q)
    with pytest.raises(FileNotFoundError):
        host.read_fvecs(str(tmp_path / "missing.fvecs"))
