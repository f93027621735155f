"""The reference's own callers run against this repository's headers and libraries.

oracle/Makefile (`make -C oracle callers`) compiles the reference's bench driver (bench/bench_main.cpp, GPU section
enabled) and its CPU and GPU test programs (tests/test_cpu.cpp, tests/test_gpu.cpp) where they lie, against
include/veckern of this repository, linked to libveckern_cpu / libveckern_gpu / libveckern. That they compile and
link shows the headers are a drop-in for the reference's callers; here they run:
  - the reference's CPU tests (on the CPU: TopK known answers, PQ invariants, staged == fused, recall, fvecs);
  - on the GPU, the reference's GPU tests (every ScanVariant against the CPU path at its 1e-3 / 99 % bar, launch
    shapes, tuning validation) and its bench driver, whose CSV rows must carry the reference's header.
The binaries live in oracle/_ref/callers (built here, where the reference checkout is; they travel to the GPU host
like the rest of oracle/_ref). Without them these tests skip.
"""
import csv
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLERS = os.path.join(ROOT, "oracle", "_ref", "callers")
REFERENCE_CSV_HEADER = ("label,variant,n,d,m,nq,k,rerank,threads,blocks_x,grid_y,qpb,ilp,blocks_per_sm,waves,lut_ms,"
                        "scan_ms,select_ms,transfer_ms,total_ms,qps,code_gbs,recall").split(",")


def binary(name):
    path = os.path.join(CALLERS, name)
    if not os.path.exists(path):
        pytest.skip(f"{path} not built (make -C oracle callers, with the reference checkout present)")
    return path


def run(args, timeout, cwd=None):
    print("\n    +", " ".join(args), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout, cwd=cwd)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    return r


def test_reference_cpu_tests_pass_against_this_library():
    r = run([binary("ref_test_cpu")], 600)
    assert r.returncode == 0 and " 0 failed" in r.stdout


@pytest.mark.gpu
def test_reference_gpu_tests_pass_against_this_library():
    # v4 (ScanVariant::Fused) is rejected before launch in this build (std::logic_error), so the reference's cases
    # that loop over every fused variant fail on it; every other case passes, and no failure has another cause.
    r = run([binary("ref_test_gpu")], 600)
    fails = [line for line in r.stdout.splitlines() if line.startswith("[ FAIL ]")]
    assert all("v4_fused is not launched" in line for line in fails), fails
    assert sorted(line[len("[ FAIL ] "):].split(":")[0] for line in fails) == [
        "search covers every K template (k = 1, 16, 33, 100)", "search matches CPU for all variants, k = 10",
        "tuning overrides keep results correct"], fails
    passes = [line for line in r.stdout.splitlines() if line.startswith("[ PASS ]")]
    assert len(passes) == 7, r.stdout


@pytest.mark.gpu
def test_reference_bench_driver_runs_on_this_library(tmp_path):
    out = tmp_path / "ref.csv"
    r = run([binary("ref_bench"), "--n", "200000", "--nq", "200", "--k", "10", "--variants", "v2,v5,v7,v8",
             "--cpu-queries", "50", "--eval-queries", "50", "--reps", "3", "--csv", str(out), "--label", "callers"],
            900, cwd=tmp_path)
    assert r.returncode == 0
    rows = list(csv.reader(open(out)))
    assert rows[0] == REFERENCE_CSV_HEADER
    variants = [row[1] for row in rows[1:]]
    assert variants == ["cpu_reference", "v2_shared_lut_vec", "v5_fused_reg", "v7_fused_vec_mq", "v8_fused_warp"]
    recalls = {row[1]: float(row[-1]) for row in rows[1:]}
    # every GPU variant returns the CPU path's neighbours, so their recall is the CPU row's
    assert all(abs(v - recalls["cpu_reference"]) < 1e-9 for v in recalls.values()), recalls
