"""GPU parity over the whole regime sweep, at a reduced size, plus the
benchmark executable and the sweep runner end to end.

Every case of both grids (the 128-case config-5 sweep, with seed = case
index, and the reference's publication grid) is generated at 48 block rows
(its distribution, locality, degree and RHS as in the grid) and Plan::execute
is checked against the oracle with the bars of test_gpu_parity.py.  Every
eighth case also checks the order-preserving kernel bit for bit.
"""

import csv
import io
import os
import subprocess
import sys

import pytest

import oracle_ffi as o
import varblockspmm_amd as vb
from test_gpu_parity import Case, note

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH_DIR = os.path.join(ROOT, "varblockspmm_amd", "bench")
sys.path.insert(0, BENCH_DIR)

import run_grid  # noqa: E402

SWEEP_ROWS = 48
CASES = [("config5", i, c) for i, c in enumerate(run_grid.cases("config5"))] + \
        [("reference", i, c) for i, c in enumerate(run_grid.cases("reference", seed=2))]


@pytest.mark.parametrize("grid,index,case", CASES,
                         ids=[f"{g}-{i}-{c['distribution']}-{c['locality']}-d{c['degree']}-n{c['rhs']}"
                              for g, i, c in CASES])
def test_sweep_case_parity(grid, index, case):
    note(f"sweep {grid} case {index}: {case}")
    host = vb.generate(SWEEP_ROWS, SWEEP_ROWS, case["degree"], case["distribution"], case["locality"], case["seed"])
    c = Case(host, case["rhs"], 1000 + index)
    try:
        plan = vb.Plan(c.matrix, case["rhs"])
        first = c.run_plan(plan)
        c.check_tolerance(first, "plan")
        again = c.run_plan(plan)
        assert first.tobytes() == again.tobytes(), "plan not bit-stable"
        plan.close()
        if index % 8 == 0:
            scalar = c.run_scalar()
            expected = o.fmaf_order(c.oracle, c.b, case["rhs"])
            assert scalar.tobytes() == expected.tobytes(), "order-preserving kernel differs from fmaf order"
    finally:
        c.close()


def test_benchmark_executable_end_to_end():
    executable = os.path.join(BENCH_DIR, "vbsr_benchmark")
    assert os.path.exists(executable), "varblockspmm_amd/bench/vbsr_benchmark is not built"
    note("vbsr_benchmark --rows 64 --reps 3 --warmup 1")
    result = subprocess.run([executable, "--rows", "64", "--degree", "4", "--rhs", "32", "--reps", "3", "--warmup",
                             "1", "--distribution", "high", "--locality", "random", "--input", "random"],
                            capture_output=True, text=True, timeout=110)
    assert result.returncode == 0, result.stderr
    rows = list(csv.DictReader(io.StringIO(result.stdout)))
    assert [r["method"] for r in rows] == ["row_owned_hybrid", "row_owned_scalar", "scalar_csr_rocsparse",
                                           "slot_grouped_rocblas"]
    for r in rows:
        assert r["block_rows"] == "64" and r["rhs"] == "32" and r["locality"] == "random"
        assert float(r["gpu_median_ms"]) > 0 and float(r["cold_median_ms"]) > 0
        assert float(r["gpu_p95_ms"]) >= float(r["gpu_median_ms"])
        assert r["identical"] == "1"
        assert float(r["useful_gflops"]) > 0
    assert [r["launches"] for r in rows] == ["1", "1", "1", "4"]  # the grouped plan: one launch per slot
    assert rows[0]["workspace_bytes"] == "0" and rows[1]["workspace_bytes"] == "0"
    assert int(rows[2]["workspace_bytes"]) >= 0 and rows[3]["workspace_bytes"] == "0"


def test_run_grid_writes_one_header(tmp_path):
    out = tmp_path / "grid.csv"
    note("run_grid --limit 3 --rows 32")
    run_grid.main(["--grid", "config5", "--rows", "32", "--reps", "2", "--warmup", "1", "--limit", "3", "--no-cold",
                   "--out", str(out)])
    lines = out.read_text().splitlines()
    assert lines[0].startswith("method,block_rows,degree,distribution")
    assert sum(line.startswith("method,") for line in lines) == 1
    rows = list(csv.DictReader(io.StringIO(out.read_text())))
    assert len(rows) == 12  # 3 cases x 4 methods
    assert [r["seed"] for r in rows[::4]] == ["0", "1", "2"]
