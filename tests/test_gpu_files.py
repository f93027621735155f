"""The file-input path of the benchmark CLI on the GPU (reference bench_main.cpp:101-106, 132-135 with the readers
of io.cpp:12-52): base and query vectors from .fvecs or .bvecs files, ground truth from an .ivecs file holding more
ids per row than k (SIFT1M's ground truth has 100). The recall the CLI reports for v8 and v9 must equal the recall
of the oracle's search over the same PQ codebook, and the CLI's own exact ground truth must give the same value as
the file's."""
import csv
import os
import subprocess

import numpy as np
import pytest

from oracle import binding as orc
from veckern_amd import host

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "veckern_amd", "bin", "veckern_bench")
N, D, M, NQ, K, TRAIN, ITERS = 20_000, 32, 16, 64, 10, 5_000, 4


def run_cli(tmp_path, label, *args):
    out = str(tmp_path / "results.csv")
    cmd = [EXE, "--m", str(M), "--k", str(K), "--train", str(TRAIN), "--iters", str(ITERS), "--reps", "1",
           "--eval-queries", str(NQ), "--variants", "v8,v9", "--csv", out, "--label", label, *args]
    print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=180)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    with open(out) as f:
        return {row["variant"]: row for row in csv.DictReader(f) if row["label"] == label}


def expected_recalls(base, queries, truth):
    cent = host.pq_train(base[:TRAIN], M, ITERS, seed=1)
    codes = host.pq_encode(cent, base)
    fp32 = orc.recall_at_k(orc.adc_search(cent, D, codes, queries, K), truth, K)
    fp16 = orc.recall_at_k(orc.adc_search_f16(cent, D, codes, queries, K), truth, K)
    return fp32, fp16


def test_fvecs_inputs_with_ivecs_ground_truth(tmp_path):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} not built: run `make -C veckern_amd`")
    base = host.gaussian_mixture(D, 50, 0.3, 5, 0, N)
    queries = host.gaussian_mixture(D, 50, 0.3, 5, 1 << 40, NQ)
    truth = host.exact_knn(base, queries, 100)["id"]
    host.write_fvecs(str(tmp_path / "base.fvecs"), base)
    host.write_fvecs(str(tmp_path / "query.fvecs"), queries)
    host.write_ivecs(str(tmp_path / "gt.ivecs"), truth)
    files = ["--base", str(tmp_path / "base.fvecs"), "--query", str(tmp_path / "query.fvecs")]
    with_gt = run_cli(tmp_path, "gt", *files, "--gt", str(tmp_path / "gt.ivecs"))
    own_gt = run_cli(tmp_path, "own", *files)
    fp32, fp16 = expected_recalls(base, queries, truth)
    assert 0.2 < fp32 <= 1.0
    for rows in (with_gt, own_gt):
        assert int(rows["v8_fused_warp"]["n"]) == N and int(rows["v8_fused_warp"]["d"]) == D
        assert float(rows["v8_fused_warp"]["recall"]) == pytest.approx(fp32, abs=1e-6)
        assert float(rows["v9_fused_warp_f16"]["recall"]) == pytest.approx(fp16, abs=1e-6)
        # the CPU search path's row (all NQ queries, the default --cpu-queries 100 capped at nq) scores the same
        assert float(rows["cpu_reference"]["recall"]) == pytest.approx(fp32, abs=1e-6)


def test_bvecs_inputs(tmp_path):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} not built: run `make -C veckern_amd`")
    # byte vectors like SIFT1B's: the mixture scaled into 0..255 and rounded
    raw = host.gaussian_mixture(D, 50, 0.3, 9, 0, N + NQ)
    lo, hi = raw.min(), raw.max()
    b = np.rint((raw - lo) / (hi - lo) * 255).astype(np.uint8)
    host.write_bvecs(str(tmp_path / "base.bvecs"), b[:N])
    host.write_bvecs(str(tmp_path / "query.bvecs"), b[N:])
    rows = run_cli(tmp_path, "bytes", "--base", str(tmp_path / "base.bvecs"), "--query",
                   str(tmp_path / "query.bvecs"))
    base, queries = b[:N].astype(np.float32), b[N:].astype(np.float32)
    truth = host.exact_knn(base, queries, K)["id"]
    fp32, fp16 = expected_recalls(base, queries, truth)
    assert float(rows["v8_fused_warp"]["recall"]) == pytest.approx(fp32, abs=1e-6)
    assert float(rows["v9_fused_warp_f16"]["recall"]) == pytest.approx(fp16, abs=1e-6)


def test_default_variant_list_runs_every_launched_variant(tmp_path):
    # `--variants all` (the reference's default): one row per variant this build launches, v4 reported without a row
    # (it is rejected before launch), plus the CPU search path's row; every GPU row scores the CPU row's recall
    out = str(tmp_path / "all.csv")
    cmd = [EXE, "--n", "60000", "--d", "64", "--m", "16", "--nq", "40", "--k", "10", "--train", "5000", "--iters", "3",
           "--reps", "1", "--eval-queries", "40", "--cpu-queries", "40", "--csv", out, "--label", "all"]
    print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "v4_fused: no row" in r.stdout
    rows = list(csv.DictReader(open(out)))
    assert [row["variant"] for row in rows] == ["cpu_reference", "v0_global_lut", "v1_shared_lut", "v2_shared_lut_vec",
                                                "v3_interleaved", "v5_fused_reg", "v6_fused_vec", "v7_fused_vec_mq",
                                                "v8_fused_warp"]
    cpu = float(rows[0]["recall"])
    assert all(float(row["recall"]) == pytest.approx(cpu, abs=1e-9) for row in rows), rows
