"""GPU parity over the whole regime sweep, at its full size and at a reduced
size, plus the benchmark executable and the sweep runner end to end.

Configuration 5's 128 cases, and the 128 instances of the reference's
publication grid at seed 1, run at their own size (4096 block rows) against
the threaded oracle.

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

import numpy as np
import pytest

import oracle_ffi as o
import varblockspmm_amd as vb
from test_gpu_parity import ELEMENTWISE_TOL, NORMWISE_TOL, REL_L2_TOL, Case, note

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


FULL_ROWS = 4096
THREADS = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS", "8"))))
CONFIG5 = list(enumerate(run_grid.cases("config5")))


def check_full_size(case):
    """Plan::execute on the case's matrix at FULL_ROWS block rows, checked against the oracle's
    cpu_reference (rows over OpenMP threads, bit-identical to the serial one) with the bars of
    test_gpu_parity.py, and bit-stable across two runs.  B is the reference test's generator with the
    case's seed."""
    rhs, seed = case["rhs"], case["seed"]
    host = vb.generate(FULL_ROWS, FULL_ROWS, case["degree"], case["distribution"], case["locality"], seed)
    oracle = o.HostMatrix(host.block_rows, host.block_cols, **host.arrays())
    b = o.make_random_input(host.scalar_cols * rhs, seed)
    matrix = vb.Matrix(host)
    try:
        stream = torch.cuda.Stream(device="cuda:0")
        b_dev = torch.from_numpy(b).to("cuda:0")
        c_dev = torch.full((host.scalar_rows * rhs,), float("nan"), device="cuda:0")
        plan = vb.Plan(matrix, rhs)
        runs = []
        for _ in range(2):
            c_dev.fill_(float("nan"))
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                plan.execute(b_dev, c_dev, stream)
            stream.synchronize()
            runs.append(c_dev.cpu().numpy())
        plan.close()
        assert runs[0].tobytes() == runs[1].tobytes(), "plan not bit-stable"
        result = runs[0]
        assert np.all(np.isfinite(result)), "NaN/Inf (unwritten or polluted outputs)"
        reference = o.cpu_reference_threads(oracle, b, rhs, THREADS)
        bound = o.abs_product_sum_threads(oracle, b, rhs, THREADS)
        max_abs, rel_l2, normwise, elementwise = o.parity_errors(result, reference, bound)
        note(f"  max_abs={max_abs:.3g} rel_l2={rel_l2:.3g} normwise={normwise:.3g} elementwise={elementwise:.3g}")
        assert max_abs <= 5e-4 and rel_l2 <= 5e-5  # tests/test_main.cpp:35
        assert normwise <= NORMWISE_TOL and rel_l2 <= REL_L2_TOL and elementwise <= ELEMENTWISE_TOL
    finally:
        matrix.close()


@pytest.mark.parametrize("index,case", CONFIG5,
                         ids=[f"{i}-{c['distribution']}-{c['locality']}-d{c['degree']}-n{c['rhs']}" for i, c in CONFIG5])
def test_config5_full_size_parity(index, case):
    """BASELINE configuration 5 at its own size: each of the 128 cases at 4096 block rows (the generator
    makes a different matrix at another row count, not a smaller copy)."""
    note(f"config5 full size case {index}: {case}")
    check_full_size(case)


REFERENCE_GRID = list(enumerate(run_grid.cases("reference", seed=1)))


@pytest.mark.parametrize("index,case", REFERENCE_GRID,
                         ids=[f"{i}-{c['distribution']}-{c['locality']}-d{c['degree']}-n{c['rhs']}"
                              for i, c in REFERENCE_GRID])
def test_reference_grid_full_size_parity(index, case):
    """The reference's publication grid (scripts/run_grid.sh:11-14) at seed 1: the 128 instances of
    data/publication/regime_map_seed1.csv (the same matrices: tests/test_oracle.py checks their
    Sigma h*w against that file), each at 4096 block rows, with the reference generator's own
    distributions and cyclic local columns."""
    note(f"reference grid full size case {index}: {case}")
    check_full_size(case)


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
