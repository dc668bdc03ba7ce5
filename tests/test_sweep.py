"""The benchmark executable and the regime-sweep runner, without a GPU:
the grids' case lists (the reference's loop nesting, scripts/run_grid.sh:11-14)
and argument handling, which runs before any HIP call."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH_DIR = os.path.join(ROOT, "varblockspmm_amd", "bench")
sys.path.insert(0, BENCH_DIR)

import run_grid  # noqa: E402

REFERENCE_HEADER = ("method,block_rows,degree,distribution,locality,rhs,seed,gpu_median_ms,gpu_p95_ms,"
                    "hot_median_ms,hot_p95_ms,useful_gflops,launches,workspace_bytes")


@pytest.fixture(scope="module")
def executable():
    subprocess.run(["make", "-s", "-C", BENCH_DIR], check=True, capture_output=True)
    return os.path.join(BENCH_DIR, "vbsr_benchmark")


def test_config5_grid_is_the_128_case_sweep():
    cases = run_grid.cases("config5")
    assert len(cases) == 128
    assert [c["seed"] for c in cases] == list(range(128))  # seed = case index
    keys = {(c["distribution"], c["locality"], c["degree"], c["rhs"]) for c in cases}
    assert len(keys) == 128
    assert {c["distribution"] for c in cases} == {"tied8to64", "low", "high", "bimodal8or64"}
    assert {c["locality"] for c in cases} == {"clamped", "random"}
    assert {c["degree"] for c in cases} == {1, 4, 8, 16}
    assert {c["rhs"] for c in cases} == {8, 16, 32, 64}
    # Nesting distribution -> locality -> degree -> rhs, rhs fastest.
    assert [c["rhs"] for c in cases[:5]] == [8, 16, 32, 64, 8]
    assert cases[4]["degree"] == 4 and cases[16]["locality"] == "random" and cases[32]["distribution"] == "low"


def test_reference_grid_matches_run_grid_sh():
    cases = run_grid.cases("reference", seed=3)
    assert len(cases) == 128 and {c["seed"] for c in cases} == {3}
    assert [c["distribution"] for c in cases[::32]] == ["uniform", "low", "high", "bimodal"]
    assert {c["degree"] for c in cases} == {2, 4, 8, 16}
    assert {c["locality"] for c in cases} == {"local", "random"}
    with pytest.raises(ValueError):
        run_grid.cases("nope")


def test_benchmark_rejects_bad_arguments(executable):
    for args in (["--bogus"], ["--rows"], ["--distribution", "gauss"], ["--locality", "near"], ["--reps", "0"],
                 ["--input", "ones"]):
        result = subprocess.run([executable] + args, capture_output=True, text=True)
        assert result.returncode == 2, args
        assert result.stderr.startswith("error: "), args
    result = subprocess.run([executable, "--help"], capture_output=True, text=True)
    assert result.returncode == 0 and "usage" in result.stderr


def test_csv_header_extends_the_reference_schema():
    with open(os.path.join(BENCH_DIR, "vbsr_benchmark.hip")) as handle:
        source = handle.read()
    flattened = source.replace('"\n                 "', "")
    assert REFERENCE_HEADER + ",cold_median_ms" in flattened


def test_runner_reports_a_missing_executable(tmp_path):
    with pytest.raises(SystemExit):
        run_grid.main(["--exe", str(tmp_path / "absent"), "--out", str(tmp_path / "x.csv")])
