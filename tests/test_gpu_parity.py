"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Bars (written per check below):
  - MFMA row-owned path: within the reference test's tolerance
    (max|err| <= 5e-4, rel-L2 <= 5e-5, tests/test_main.cpp:35) and the
    library's bounds: normwise max|C - Cref| / max|Cref| <= 1e-5,
    rel-L2 <= 1e-5, max|C - Cref| / max(sum |a||b|) <= 1e-6; bit-identical
    across runs.
  - Order-preserving kernel: bit-identical to the oracle's fmaf emulation of
    the reference kernels' order.
Every output buffer is poisoned with NaN before a run, so unwritten elements
fail the check.
"""

import os
import subprocess
import sys

import numpy as np
import pytest

import oracle_ffi as o
import varblockspmm_amd as vb
from reference_cases import reference_cases
import test_oracle

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEVICE = "cuda:0"

NORMWISE_TOL = 1e-5
REL_L2_TOL = 1e-5
ELEMENTWISE_TOL = 1e-6


def note(message):
    print(message, flush=True)
    sys.stdout.flush()


def as_oracle(host):
    return o.HostMatrix(host.block_rows, host.block_cols, **host.arrays())


class Case:
    """A host matrix with its device copy, B, and oracle results for one RHS width."""

    def __init__(self, host, rhs, seed, stream=None):
        self.host = host
        self.rhs = rhs
        self.oracle = as_oracle(host)
        self.b = o.make_random_input(host.scalar_cols * rhs, seed)
        self.matrix = vb.Matrix(host)
        self.stream = stream if stream is not None else torch.cuda.Stream(device=DEVICE)
        self.b_dev = torch.from_numpy(self.b).to(DEVICE)
        self.c_dev = torch.empty(host.scalar_rows * rhs, dtype=torch.float32, device=DEVICE)
        self._reference = None
        self._bound = None

    @property
    def reference(self):
        if self._reference is None:
            self._reference = o.cpu_reference(self.oracle, self.b, self.rhs)
        return self._reference

    @property
    def bound(self):
        if self._bound is None:
            self._bound = o.abs_product_sum(self.oracle, self.b, self.rhs)
        return self._bound

    def run(self, launch):
        self.c_dev.fill_(float("nan"))
        torch.cuda.current_stream(DEVICE).synchronize()
        with torch.cuda.stream(self.stream):
            launch()
        self.stream.synchronize()
        return self.c_dev.cpu().numpy().copy()

    def run_plan(self, plan):
        return self.run(lambda: plan.execute(self.b_dev, self.c_dev, self.stream))

    def run_scalar(self):
        view = self.matrix.device_view()
        return self.run(lambda: vb.launch_row_owned_scalar(view, self.b_dev, self.c_dev, self.rhs, self.stream))

    def check_tolerance(self, result, name):
        assert np.all(np.isfinite(result)), f"{name}: NaN/Inf (unwritten or polluted outputs)"
        max_abs, rel_l2, normwise, elementwise = o.parity_errors(result, self.reference, self.bound)
        note(f"  {name}: max_abs={max_abs:.3g} rel_l2={rel_l2:.3g} normwise={normwise:.3g} "
             f"elementwise={elementwise:.3g}")
        assert max_abs <= 5e-4 and rel_l2 <= 5e-5, name  # tests/test_main.cpp:35
        assert normwise <= NORMWISE_TOL and rel_l2 <= REL_L2_TOL and elementwise <= ELEMENTWISE_TOL, name

    def close(self):
        self.matrix.close()


@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: "{}-d{}-n{}-{}-s{}".format(*c))
def test_reference_parameter_matrix(case):
    distribution, degree, rhs, locality, seed = case
    note(f"case {case}")
    c = Case(vb.generate(9, 17, degree, distribution, locality, seed), rhs, seed)
    plan = vb.Plan(c.matrix, rhs, "row_owned")
    assert plan.launch_count() == 1
    first = c.run_plan(plan)
    c.check_tolerance(first, "mfma")
    np.testing.assert_array_equal(c.run_plan(plan), first, err_msg="mfma not bit-identical across runs")
    scalar = c.run_scalar()
    np.testing.assert_array_equal(scalar, o.fmaf_order(c.oracle, c.b, rhs), err_msg="scalar != fmaf emulation")
    c.check_tolerance(scalar, "scalar")
    c.close()


BASELINE_CONFIGS = [
    # (name, rows, degree, distribution, locality, rhs, seed)
    ("config1-cpu-shape", 1024, 4, "high", "clamped", 8, 1),
    ("config1-cyclic", 1024, 4, "high", "local", 8, 1),
    ("config2", 1024, 8, "low", "random", 16, 2),
    ("config3-metric", 4096, 8, "high", "random", 32, 1),
    ("config3-n8", 4096, 8, "high", "random", 8, 1),
    ("config3-n16", 4096, 8, "high", "random", 16, 1),
    ("config3-n64", 4096, 8, "high", "random", 64, 1),
    ("config4-literal-bimodal", 4096, 16, "bimodal8or64", "random", 64, 3),
    ("config4-reference-bimodal", 4096, 16, "bimodal", "random", 64, 3),
]


@pytest.mark.parametrize("config", BASELINE_CONFIGS, ids=lambda c: c[0])
def test_baseline_configs(config):
    name, rows, degree, distribution, locality, rhs, seed = config
    note(f"config {config}")
    c = Case(vb.generate(rows, rows, degree, distribution, locality, seed), rhs, seed)
    plan = vb.Plan(c.matrix, rhs)
    first = c.run_plan(plan)
    c.check_tolerance(first, name)
    np.testing.assert_array_equal(c.run_plan(plan), first, err_msg="not bit-identical across runs")
    c.close()


@pytest.mark.parametrize("config", [("config2", 1024, 8, "low", "random", 16, 2),
                                    ("config3-n8", 4096, 8, "high", "random", 8, 1)], ids=lambda c: c[0])
def test_order_preserving_kernel_full_size(config):
    name, rows, degree, distribution, locality, rhs, seed = config
    note(f"scalar kernel {config}")
    c = Case(vb.generate(rows, rows, degree, distribution, locality, seed), rhs, seed)
    np.testing.assert_array_equal(c.run_scalar(), o.fmaf_order(c.oracle, c.b, rhs))
    c.close()


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
def test_public_launcher_matches_plan(rhs):
    """launch_row_owned with the matrix's schedule is exactly Plan::execute."""
    note(f"launcher rhs={rhs}")
    c = Case(vb.generate(300, 280, 6, "high", "random", 5), rhs, 5)
    view = c.matrix.device_view()
    launched = c.run(lambda: vb.launch_row_owned(view, c.matrix.row_schedule(), c.b_dev, c.c_dev, rhs, c.stream))
    plan = vb.Plan(c.matrix, rhs)
    np.testing.assert_array_equal(c.run_plan(plan), launched)
    c.check_tolerance(launched, "launcher")
    c.close()


def test_launchers_reject_panels_of_the_wrong_size():
    """A device panel one float short (or long) is refused before any launch, by every entry point."""
    note("wrong-size panels")
    rhs = 16
    c = Case(vb.generate(40, 40, 4, "high", "random", 3), rhs, 3)
    view, schedule = c.matrix.device_view(), c.matrix.row_schedule()
    short_b = torch.empty(c.b.size - 1, dtype=torch.float32, device=DEVICE)
    long_c = torch.empty(c.c_dev.numel() + 1, dtype=torch.float32, device=DEVICE)
    plan = vb.Plan(c.matrix, rhs)
    for b, cc in ((short_b, c.c_dev), (c.b_dev, long_c)):
        with pytest.raises(ValueError, match="expected"):
            vb.launch_row_owned(view, schedule, b, cc, rhs, c.stream)
        with pytest.raises(ValueError, match="expected"):
            vb.launch_row_owned_scalar(view, b, cc, rhs, c.stream)
        with pytest.raises(ValueError, match="expected"):
            plan.execute(b, cc, c.stream)
    plan.close()
    c.close()


def test_entry_points_reject_overlapping_panels():
    """A C panel that shares memory with B is refused before any launch, by every entry point (the
    reference's B and C are __restrict__, row_owned.cu:12-13)."""
    note("overlapping panels")
    rhs = 16
    c = Case(vb.generate(40, 40, 4, "high", "random", 3), rhs, 3)
    view, schedule = c.matrix.device_view(), c.matrix.row_schedule()
    b_count, c_count = c.b.size, c.c_dev.numel()
    storage = torch.zeros(b_count + c_count, dtype=torch.float32, device=DEVICE)
    b = storage[:b_count]
    overlapping_c = storage[b_count - 4:b_count - 4 + c_count]
    plan = vb.Plan(c.matrix, rhs)
    csr = vb.ScalarCsrPlan(c.host, rhs)
    grouped = vb.GroupedGemmPlan(c.host, rhs)
    for run in (lambda: vb.launch_row_owned(view, schedule, b, overlapping_c, rhs, c.stream),
                lambda: vb.launch_row_owned_scalar(view, b, overlapping_c, rhs, c.stream),
                lambda: plan.execute(b, overlapping_c, c.stream),
                lambda: csr.execute(b, overlapping_c, c.stream),
                lambda: grouped.execute(b, overlapping_c, c.stream)):
        with pytest.raises(ValueError, match="overlap"):
            run()
    assert csr.workspace_bytes() == 0  # refused before the first execute set anything up
    csr.close()
    grouped.close()
    with pytest.raises(ValueError, match="device pointers"):
        plan.execute(None, c.c_dev, c.stream)
    # The same storage split without overlap runs, and matches the oracle.
    touching_c = storage[b_count:]
    b.copy_(c.b_dev)
    touching_c.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(c.stream):
        plan.execute(b, touching_c, c.stream)
    c.stream.synchronize()
    c.check_tolerance(touching_c.cpu().numpy(), "C right after B in one allocation")
    plan.close()
    c.close()


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
def test_misaligned_b_stays_on_the_mfma_kernel(rhs):
    """B panels 4, 8 and 12 bytes past a 16-byte boundary: the tuned kernel loads them 4 bytes at a
    time, through the launcher and Plan::execute, with the same bits as an aligned B."""
    note(f"misaligned B rhs={rhs}")
    c = Case(vb.generate(40, 40, 4, "bimodal8or64", "random", 9), rhs, 9)
    plan = vb.Plan(c.matrix, rhs)
    aligned = c.run_plan(plan)
    c.check_tolerance(aligned, "aligned B")
    view, schedule = c.matrix.device_view(), c.matrix.row_schedule()
    for shift in (1, 2, 3):
        storage = torch.empty(c.b.size + 4, dtype=torch.float32, device=DEVICE)
        shifted = storage[shift:shift + c.b.size]
        shifted.copy_(c.b_dev)
        assert shifted.data_ptr() % 16 == 4 * shift
        np.testing.assert_array_equal(c.run(lambda: plan.execute(shifted, c.c_dev, c.stream)), aligned)
        np.testing.assert_array_equal(
            c.run(lambda: vb.launch_row_owned(view, schedule, shifted, c.c_dev, rhs, c.stream)), aligned)
    plan.close()
    c.close()


def misaligned_c(c):
    """A NaN-filled C panel that starts 4 bytes past a 16-byte boundary, and its storage."""
    storage = torch.full((c.c_dev.numel() + 4,), float("nan"), dtype=torch.float32, device=DEVICE)
    shifted = storage[1:1 + c.c_dev.numel()]
    assert shifted.data_ptr() % 16 == 4
    return storage, shifted


def run_into(c, launch):
    torch.cuda.synchronize()
    with torch.cuda.stream(c.stream):
        launch()
    c.stream.synchronize()


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
def test_misaligned_c_stays_on_the_mfma_kernel(rhs):
    """A C panel 4 bytes past a 16-byte boundary takes the tuned kernel (at RHS 8, rows of 56 and 64
    store 16 bytes per lane at 4-byte alignment): the launcher accepts it, and both it and
    Plan::execute give the same bits as with an aligned C, without writing outside the panel."""
    note(f"misaligned C rhs={rhs}")
    c = Case(vb.generate(40, 40, 4, "bimodal8or64", "random", 19), rhs, 19)
    plan = vb.Plan(c.matrix, rhs)
    aligned = c.run_plan(plan)
    c.check_tolerance(aligned, "aligned C")
    view = c.matrix.device_view()
    for launch in (lambda cc: plan.execute(c.b_dev, cc, c.stream),
                   lambda cc: vb.launch_row_owned(view, c.matrix.row_schedule(), c.b_dev, cc, rhs, c.stream)):
        storage, shifted = misaligned_c(c)
        run_into(c, lambda: launch(shifted))
        np.testing.assert_array_equal(shifted.cpu().numpy(), aligned)
        assert torch.isnan(storage[0]) and torch.isnan(storage[1 + c.c_dev.numel():]).all()
    c.close()


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
def test_infinite_b_matches_reference_semantics(rhs):
    """+Inf in one B entry: every output whose row touches it with a positive A
    value is +Inf, never NaN (padding lanes must not form 0 * Inf)."""
    note(f"inf B rhs={rhs}")
    host = hand_made([8, 24, 40, 56], [8, 24, 40], [[0, 1, 2], [2, 0], [1], [0, 2]], seed=4)
    values = np.abs(host.values) + 0.5  # strictly positive A
    host = vb.HostMatrix(host.block_rows, host.block_cols, **{**host.arrays(), "values": values})
    c = Case(host, rhs, 31)
    b = np.abs(c.b).reshape(rhs, host.scalar_cols)
    b[:, host.col_scalar_off[0] + 5] = np.inf  # last k of a half step of the 8-wide column 0
    b[:, host.col_scalar_off[2] + 37] = np.inf  # inside the half step of the 40-wide column 2
    c.b = b.reshape(-1).copy()
    c.b_dev = torch.from_numpy(c.b).to(DEVICE)
    result = c.run_plan(vb.Plan(c.matrix, rhs)).reshape(rhs, host.scalar_rows)
    expected = o.cpu_reference(c.oracle, c.b, rhs).reshape(rhs, host.scalar_rows)
    assert not np.any(np.isnan(result))
    np.testing.assert_array_equal(np.isinf(result), np.isinf(expected))
    finite = np.isfinite(expected)
    np.testing.assert_allclose(result[finite], expected[finite], rtol=1e-5, atol=1e-5)
    c.close()


def hand_made(row_size, col_size, rows_blocks, seed=0):
    """A host matrix from per-row block-column lists (empty rows and repeats allowed)."""
    rng = np.random.default_rng(seed)
    row_ptr = np.concatenate([[0], np.cumsum([len(b) for b in rows_blocks])])
    block_col = np.array([c for b in rows_blocks for c in b], dtype=np.int32)
    owners = np.repeat(np.arange(len(row_size)), [len(b) for b in rows_blocks])
    counts = np.array(row_size)[owners] * np.array(col_size)[block_col] if len(block_col) else np.zeros(0)
    value_off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return vb.HostMatrix(len(row_size), len(col_size), row_ptr=row_ptr, block_col=block_col, row_size=row_size,
                         col_size=col_size, row_scalar_off=np.concatenate([[0], np.cumsum(row_size)]),
                         col_scalar_off=np.concatenate([[0], np.cumsum(col_size)]), value_off=value_off,
                         values=rng.uniform(-1, 1, int(value_off[-1])).astype(np.float32))


EDGE_MATRICES = {
    # empty rows, a repeated block column, unsorted columns, every height
    "empty-repeat-unsorted": lambda: hand_made([8, 16, 24, 32, 40, 48, 56, 64], [8, 24, 64, 40, 16],
                                                [[1, 1, 0], [], [4, 2], [0], [], [3, 2, 1, 0, 4], [2], [4, 4]]),
    "all-empty": lambda: hand_made([8, 64, 24], [8, 8], [[], [], []]),
    "single-row": lambda: hand_made([40], [56, 8, 64], [[0, 1, 2]]),
    "all-8": lambda: hand_made([8] * 20, [8] * 20, [[(i + j) % 20 for j in range(5)] for i in range(20)]),
    "all-64": lambda: hand_made([64] * 12, [64] * 12, [[(i * 5 + j) % 12 for j in range(4)] for i in range(12)]),
    "narrow-wide": lambda: hand_made([8, 64] * 8, [64, 8] * 8, [[j for j in range(16) if (i + j) % 3 == 0]
                                                                 for i in range(16)]),
    # rows of 0-4 k steps (packed four to a workgroup, one per wave, of every height) beside rows of 5 and 7
    # steps (one workgroup each); 11 light rows leave a packed workgroup with idle waves
    "packed-light": lambda: hand_made([8, 16, 24, 32, 40, 48, 56, 64, 64, 8, 40, 16, 24, 56],
                                      [8, 16, 24, 64, 40],
                                      [[], [0], [2], [0, 1, 2], [3], [3, 0], [4], [1, 4], [2, 2], [3, 4], [1], [0, 0],
                                       [4, 0], []]),
    # 100 blocks of width 64 in one row: 400 k steps, more than one workgroup
    # segment holds (256), so the row is accumulated across segments
    "long-row": lambda: hand_made([16, 40, 8], [64] * 100 + [8] * 20,
                                  [list(range(100)), list(range(0, 120, 3)), list(range(100, 120))]),
}


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
@pytest.mark.parametrize("name", list(EDGE_MATRICES))
def test_edge_matrices(name, rhs):
    note(f"edge {name} rhs={rhs}")
    host = EDGE_MATRICES[name]()
    host.validate()
    c = Case(host, rhs, 17)
    result = c.run_plan(vb.Plan(c.matrix, rhs))
    c.check_tolerance(result, name)
    empty = np.diff(host.row_ptr) == 0
    out = result.reshape(rhs, host.scalar_rows)
    for i in np.nonzero(empty)[0]:
        assert np.all(out[:, host.row_scalar_off[i]:host.row_scalar_off[i + 1]] == 0.0)
    np.testing.assert_array_equal(c.run_scalar(), o.fmaf_order(c.oracle, c.b, rhs))
    c.close()


WIDE_B_MATRICES = {**EDGE_MATRICES,
                   "generated-high": lambda: vb.generate(48, 48, 8, "high", "random", 3),
                   "generated-bimodal": lambda: vb.generate(40, 40, 4, "bimodal", "local", 5)}


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
@pytest.mark.parametrize("name", list(WIDE_B_MATRICES))
def test_wide_b_addressing_is_bit_identical(name, rhs):
    """B read through 64-bit lane addresses (the form launch_row_owned and the plan take past the
    32-bit offset bound), forced at small K: bit-identical to the offset form, with finite B and with
    +Inf in the first eight entries of every second block column, which the upper half of the
    preceding column's half step would read (so a lane that loads where the offset form gets zeros
    turns 0 * Inf into NaN)."""
    note(f"wide B {name} rhs={rhs}")
    host = WIDE_B_MATRICES[name]()
    c = Case(host, rhs, 23)
    view, schedule = c.matrix.device_view(), c.matrix.row_schedule()
    for label in ("finite", "inf"):
        if label == "inf":
            b = c.b.reshape(rhs, host.scalar_cols).copy()
            for col in range(1, host.block_cols, 2):
                start = int(host.col_scalar_off[col])
                b[:, start:start + 8] = np.inf
            c.b = b.reshape(-1).copy()
            c.b_dev = torch.from_numpy(c.b).to(DEVICE)
        narrow = c.run(lambda: vb.launch_row_owned(view, schedule, c.b_dev, c.c_dev, rhs, c.stream))
        wide = c.run(lambda: vb.launch_row_owned_wide_b(view, schedule, c.b_dev, c.c_dev, rhs, c.stream))
        assert narrow.tobytes() == wide.tobytes(), f"{name} rhs={rhs} {label}: wide B differs"
        if label == "finite":
            c.check_tolerance(wide, f"{name} wide B")
    c.close()


@pytest.mark.parametrize("tiles", [0, 1], ids=["split-k", "tile-split"])
@pytest.mark.parametrize("name", list(WIDE_B_MATRICES))
def test_rhs64_kernels_on_edge_matrices(name, tiles):
    """RHS 64 with each of its two kernels forced through the schedule's rhs64_tiles field (the
    matrix's rule picks one; both must be right for any matrix): within tolerance of the oracle, empty
    rows zero, bit-identical across runs, and the 64-bit B form bit-identical to the offset form, also
    with +Inf where the upper lanes of a half step would read."""
    rhs = 64
    note(f"rhs64 kernel tiles={tiles} {name}")
    host = WIDE_B_MATRICES[name]()
    c = Case(host, rhs, 29)
    view, schedule = c.matrix.device_view(), c.matrix.row_schedule()
    schedule.rhs64_tiles = tiles
    narrow = lambda: vb.launch_row_owned(view, schedule, c.b_dev, c.c_dev, rhs, c.stream)
    first = c.run(narrow)
    c.check_tolerance(first, f"{name} tiles={tiles}")
    out = first.reshape(rhs, host.scalar_rows)
    for i in np.nonzero(np.diff(host.row_ptr) == 0)[0]:
        assert np.all(out[:, host.row_scalar_off[i]:host.row_scalar_off[i + 1]] == 0.0)
    assert c.run(narrow).tobytes() == first.tobytes(), "not bit-identical across runs"
    wide = c.run(lambda: vb.launch_row_owned_wide_b(view, schedule, c.b_dev, c.c_dev, rhs, c.stream))
    assert wide.tobytes() == first.tobytes(), "wide B differs"
    b = c.b.reshape(rhs, host.scalar_cols).copy()
    for col in range(1, host.block_cols, 2):
        start = int(host.col_scalar_off[col])
        b[:, start:start + 8] = np.inf
    c.b_dev = torch.from_numpy(b.reshape(-1).copy()).to(DEVICE)
    assert c.run(narrow).tobytes() == c.run(
        lambda: vb.launch_row_owned_wide_b(view, schedule, c.b_dev, c.c_dev, rhs, c.stream)).tobytes()
    c.close()


@pytest.mark.parametrize("shape", [(4096, 8, "high", 1, 1), (256, 16, "high", 1, 0)], ids=["4096-d8", "256-d16"])
def test_rhs64_plan_takes_the_rule_kernel(shape):
    """The plan's RHS 64 launch is the kernel the matrix's rule names (the tile split at 4096 block rows of
    degree 8, the split-k kernel at 256 rows of degree 16): bit-identical to launch_row_owned with that
    kernel forced, within tolerance of the oracle, and within tolerance of the other kernel."""
    rows, degree, distribution, seed, expected = shape
    note(f"rhs64 rule {shape}")
    c = Case(vb.generate(rows, rows, degree, distribution, "random", seed), 64, seed)
    schedule = c.matrix.row_schedule()
    assert schedule.rhs64_tiles == expected
    planned = c.run_plan(vb.Plan(c.matrix, 64))
    c.check_tolerance(planned, f"plan {shape}")
    view = c.matrix.device_view()
    for tiles in (0, 1):
        schedule.rhs64_tiles = tiles
        forced = c.run(lambda: vb.launch_row_owned(view, schedule, c.b_dev, c.c_dev, 64, c.stream))
        if tiles == expected:
            assert forced.tobytes() == planned.tobytes()
        else:
            c.check_tolerance(forced, f"forced tiles={tiles} {shape}")
    c.close()


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
def test_unused_b_entries_never_reach_c(rhs):
    """NaN in every B row that no block references (including the rows right
    after each used 8-wide column and the panel's end) must not leak into C."""
    note(f"unused-B NaN rhs={rhs}")
    col_size = [8, 16, 8, 24, 8, 64, 8, 40, 8]
    used = [0, 2, 4, 6, 8]  # 8-wide columns, each followed by an unused one
    host = hand_made([16, 8, 48, 64, 24], col_size, [[0, 2], [4, 6, 8], [8], [0, 4, 6], [2, 8]], seed=3)
    c = Case(host, rhs, 23)
    offs = host.col_scalar_off
    b = c.b.reshape(rhs, host.scalar_cols).copy()
    clean = b.copy()
    for j in range(len(col_size)):
        if j not in used:
            b[:, offs[j]:offs[j + 1]] = np.nan
            clean[:, offs[j]:offs[j + 1]] = 0.0
    c.b = clean.reshape(-1)
    c.b_dev = torch.from_numpy(b.reshape(-1).copy()).to(DEVICE)
    c.check_tolerance(c.run_plan(vb.Plan(c.matrix, rhs)), "nan-guarded")
    np.testing.assert_array_equal(c.run_scalar(), o.fmaf_order(c.oracle, c.b, rhs))
    c.close()


@pytest.mark.parametrize("probe", test_oracle.order_probes(), ids=lambda p: p[0])
def test_order_preserving_kernel_gives_the_closed_form_bits(probe):
    """launch_row_owned_scalar on inputs whose bits depend on the summation order and on fusion: only
    blocks in row_ptr order, k ascending and one fused multiply-add per term give these bits (the
    closed forms are derived in tests/test_oracle.py, independently of the emulation)."""
    name, m, b, rhs, want_fmaf, want_reference = probe
    note(f"order probe {name}")
    host = vb.HostMatrix(m.block_rows, m.block_cols, **{n: getattr(m, n) for n in o.HostMatrix.FIELDS})
    c = Case(host, rhs, 1)
    c.b = b.copy()
    c.b_dev = torch.from_numpy(c.b).to(DEVICE)
    np.testing.assert_array_equal(c.run_scalar(), want_fmaf)
    np.testing.assert_array_equal(vb.cpu_reference(host, b, rhs), want_reference)
    # The MFMA plan sums in its own order: on inputs built to cancel, only the elementwise bound
    # (|C - Cref| <= 1e-6 * sum |a||b|) is meaningful.
    result = c.run_plan(vb.Plan(c.matrix, rhs))
    assert np.all(np.abs(result.astype(np.float64) - c.reference) <= ELEMENTWISE_TOL * c.bound), name
    c.close()


# ---- the VALU variant of the row-owned kernel (the measured alternative to MFMA) ----------------


@pytest.mark.parametrize("case", reference_cases()[::5] + [("high", 8, rhs, "random", 1) for rhs in (8, 16, 32, 64)],
                         ids=lambda c: "{}-d{}-n{}-{}-s{}".format(*c))
def test_valu_variant_matches_the_oracle(case):
    """launch_row_owned_valu: the same schedule with plain FP32 multiply-adds; within tolerance of the
    oracle and bit-identical across runs (every thirteenth reference case, or so, and configuration 3's
    matrix at 1,024 block rows at every width)."""
    distribution, degree, rhs, locality, seed = case
    rows, cols = (9, 17) if seed != 1 else (1024, 1024)
    note(f"valu case {case}")
    c = Case(vb.generate(rows, cols, degree, distribution, locality, seed), rhs, seed)
    view, schedule = c.matrix.device_view(), c.matrix.row_schedule()
    launch = lambda: vb.launch_row_owned_valu(view, schedule, c.b_dev, c.c_dev, rhs, c.stream)
    first = c.run(launch)
    c.check_tolerance(first, "valu")
    np.testing.assert_array_equal(c.run(launch), first)
    c.close()


# ---- the split-row path (the reference's reserved Kernel::SplitRow) -----------------------------


@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: "{}-d{}-n{}-{}-s{}".format(*c))
def test_split_row_reference_parameter_matrix(case):
    """Kernel::SplitRow on the reference test's parameter matrix: within tolerance of the oracle,
    bit-identical across runs, two launches."""
    distribution, degree, rhs, locality, seed = case
    note(f"split-row case {case}")
    c = Case(vb.generate(9, 17, degree, distribution, locality, seed), rhs, seed)
    plan = vb.Plan(c.matrix, rhs, "split_row")
    assert plan.launch_count() == 2
    first = c.run_plan(plan)
    c.check_tolerance(first, "split-row")
    np.testing.assert_array_equal(c.run_plan(plan), first, err_msg="split-row not bit-identical across runs")
    plan.close()
    c.close()


SPLIT_CASES = [
    # (name, rows, degree, distribution, locality, rhs, seed, the matrix's split rule holds)
    ("few-rows-32-n8", 32, 16, "high", "random", 8, 1, True),
    ("few-rows-32-n64", 32, 16, "high", "random", 64, 1, True),
    ("few-rows-128-n32", 128, 16, "high", "random", 32, 1, True),
    ("few-rows-256-n32", 256, 16, "high", "random", 32, 1, False),
    ("few-rows-64-d4", 64, 4, "high", "random", 16, 2, False),
    ("config3-n32", 4096, 8, "high", "random", 32, 1, False),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: c[0])
def test_split_row_against_oracle_and_auto_choice(case):
    """Kernel::SplitRow at few rows (where the split is advised) and at configuration 3 (where it is not):
    within tolerance of the oracle and bit-stable.  Kernel::Auto is the row-owned kernel at every shape, as
    in the reference (docs/design.md:17): one launch, the same bits as an explicit RowOwned plan.  The
    advice holds exactly where the matrix's rule does and rhs >= 16."""
    name, rows, degree, distribution, locality, rhs, seed, rule = case
    note(f"split-row {name}")
    c = Case(vb.generate(rows, rows, degree, distribution, locality, seed), rhs, seed)
    split = vb.Plan(c.matrix, rhs, "split_row")
    first = c.run_plan(split)
    c.check_tolerance(first, name)
    np.testing.assert_array_equal(c.run_plan(split), first)
    assert vb.split_row_advised(c.matrix, rhs) == (rule and rhs >= 16)
    auto = vb.Plan(c.matrix, rhs, "auto")
    assert auto.launch_count() == 1
    np.testing.assert_array_equal(c.run_plan(auto), c.run_plan(vb.Plan(c.matrix, rhs, "row_owned")))
    split.close()
    auto.close()
    c.close()


@pytest.mark.parametrize("name", ["empty-repeat-unsorted", "all-empty", "single-row", "long-row", "packed-light"])
def test_split_row_edge_matrices(name):
    """Empty rows (a zero-step part each), a row of 400 steps (parts beyond one workgroup segment),
    packed parts of every height."""
    note(f"split-row edge {name}")
    host = EDGE_MATRICES[name]()
    for rhs in (8, 64):
        c = Case(host, rhs, 19)
        c.check_tolerance(c.run_plan(vb.Plan(c.matrix, rhs, "split_row")), f"split-row {name} rhs={rhs}")
        c.close()


def test_launch_split_row_with_a_caller_workspace():
    """vbsr_launch_split_row: a caller's workspace of the reported size gives the split-row plan's bits;
    a smaller one, a misaligned one, or one overlapping B or C is refused before any launch."""
    note("launch_split_row")
    rhs = 32
    c = Case(vb.generate(48, 48, 16, "high", "random", 4), rhs, 4)
    expected = c.run_plan(vb.Plan(c.matrix, rhs, "split_row"))
    nbytes = vb.split_row_workspace_bytes(c.matrix, rhs)
    # The split schedule's rule: parts of 8 steps here (1,184 steps, far below 8 x 2048), at least one per row;
    # one partial slab (h x rhs floats) per part.
    widths = c.host.col_size[c.host.block_col]
    steps = np.add.reduceat(widths // 16 + (widths % 16 != 0), c.host.row_ptr[:-1])
    parts = np.maximum(1, -(-steps // 8))
    assert nbytes == 4 * rhs * int(np.sum(parts * c.host.row_size))
    workspace = torch.empty(nbytes // 4 + 16, dtype=torch.float32, device=DEVICE)
    result = c.run(lambda: vb.launch_split_row(c.matrix, c.b_dev, c.c_dev, rhs, workspace, nbytes, c.stream))
    np.testing.assert_array_equal(result, expected)
    with pytest.raises(ValueError, match="too small"):
        vb.launch_split_row(c.matrix, c.b_dev, c.c_dev, rhs, workspace, nbytes - 4, c.stream)
    with pytest.raises(ValueError, match="aligned"):
        vb.launch_split_row(c.matrix, c.b_dev, c.c_dev, rhs, workspace.data_ptr() + 2, nbytes, c.stream)
    with pytest.raises(ValueError, match="overlap"):
        vb.launch_split_row(c.matrix, c.b_dev, c.c_dev, rhs, c.c_dev, nbytes, c.stream)
    with pytest.raises(ValueError):
        vb.launch_split_row(c.matrix, c.b_dev, c.c_dev, rhs, None, nbytes, c.stream)
    torch.cuda.synchronize()
    c.close()


def test_device_matrix_errors():
    note("device errors")
    host = vb.generate(6, 6, 2, "high", "random", 1)
    bad = host.copy()
    bad.row_size[0] = 7
    with pytest.raises(ValueError):
        vb.Matrix(bad)
    shifted = host.copy()
    shifted.row_scalar_off = shifted.row_scalar_off + 8
    shifted.validate()  # accepted by validate, as in the reference
    with pytest.raises(ValueError):
        vb.Matrix(shifted)  # rejected for device use
    m = vb.Matrix(host)
    for rhs in (0, 7, 33, 128):
        with pytest.raises(ValueError):
            vb.Plan(m, rhs)
    for kernel in (3, -1):
        with pytest.raises(ValueError):
            vb.Plan(m, 8, kernel)
    assert vb.Plan(m, 8, "split_row").launch_count() == 2
    plan = vb.Plan(m, 32, "auto")
    assert plan.launch_count() == 1
    b = torch.zeros(m.scalar_cols * 32, device=DEVICE)
    with pytest.raises(ValueError):
        plan.execute(b, torch.zeros(m.scalar_rows * 32 - 1, device=DEVICE))
    with pytest.raises(ValueError):
        plan.execute(b.double(), torch.zeros(m.scalar_rows * 32, device=DEVICE))
    view = m.device_view()
    assert (view.block_rows, view.block_cols, view.nnzb) == (6, 6, 12)
    assert (view.scalar_rows, view.scalar_cols) == (host.scalar_rows, host.scalar_cols)
    m.close()


def test_cpp_api_program():
    """The reference test program restated over the C++ API (tests/cpp/test_api.cpp)."""
    binary = os.path.join(ROOT, "tests", "cpp", "test_api")
    note("C++ API program")
    if not os.path.exists(binary):
        pytest.fail("tests/cpp/test_api is not built (run __graft_entry__.build())")
    result = subprocess.run([binary], capture_output=True, text=True, timeout=300)
    note(result.stdout.strip() + result.stderr.strip())
    assert result.returncode == 0
    assert result.stdout.startswith("PASS")


# ---- the rocSPARSE scalar-CSR baseline (reference ScalarCsrPlan) -----------

def run_csr(c, plan, b_dev=None, c_dev=None):
    b_dev = c.b_dev if b_dev is None else b_dev
    c_dev = c.c_dev if c_dev is None else c_dev
    c_dev.fill_(float("nan"))
    torch.cuda.current_stream(DEVICE).synchronize()
    with torch.cuda.stream(c.stream):
        plan.execute(b_dev, c_dev, c.stream)
    c.stream.synchronize()
    return c_dev.cpu().numpy().copy()


@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: f"{c[0]}-d{c[1]}-n{c[2]}-{c[3]}-s{c[4]}")
def test_scalar_csr_plan_reference_matrix(case):
    """tests/test_main.cpp:84-97: the library baseline on every parameter case."""
    distribution, degree, rhs, locality, seed = case
    note(f"csr {case}")
    host = vb.generate(9, 17, degree, distribution, locality, seed)
    c = Case(host, rhs, seed)
    try:
        plan = vb.ScalarCsrPlan(host, rhs)
        assert plan.workspace_bytes() == 0
        c.check_tolerance(run_csr(c, plan), "rocSPARSE CSR")
        c.check_tolerance(run_csr(c, plan), "rocSPARSE CSR (second run)")
        plan.close()
    finally:
        c.close()


@pytest.mark.parametrize("config", [("config2", 1024, 8, "low", "random", 16, 2),
                                    ("config3", 4096, 8, "high", "random", 32, 1)], ids=lambda c: c[0])
def test_scalar_csr_plan_baseline_configs(config):
    name, rows, degree, distribution, locality, rhs, seed = config
    note(f"csr {config}")
    host = vb.generate(rows, rows, degree, distribution, locality, seed)
    c = Case(host, rhs, seed)
    try:
        plan = vb.ScalarCsrPlan(host, rhs)
        c.check_tolerance(run_csr(c, plan), f"rocSPARSE CSR {name}")
        plan.close()
    finally:
        c.close()


def test_scalar_csr_plan_follows_new_dense_pointers():
    """The dense descriptors made at the first execute take the next call's B and C."""
    host = vb.generate(40, 40, 4, "high", "random", 21)
    c = Case(host, 16, 21)
    try:
        plan = vb.ScalarCsrPlan(host, 16)
        c.check_tolerance(run_csr(c, plan), "first pointers")
        b2 = (c.b_dev * 2.0).contiguous()
        c2 = torch.empty_like(c.c_dev)
        doubled = run_csr(c, plan, b2, c2)
        np.testing.assert_allclose(doubled, 2.0 * c.reference, rtol=1e-5, atol=1e-4)
        plan.close()
    finally:
        c.close()


# ---- the rocBLAS slot-grouped baseline (reference GroupedGemmPlan) ---------

@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: f"{c[0]}-d{c[1]}-n{c[2]}-{c[3]}-s{c[4]}")
def test_grouped_gemm_plan_reference_matrix(case):
    """tests/test_main.cpp:86-99: the grouped-GEMM baseline on every parameter case."""
    distribution, degree, rhs, locality, seed = case
    note(f"grouped {case}")
    host = vb.generate(9, 17, degree, distribution, locality, seed)
    c = Case(host, rhs, seed)
    try:
        plan = vb.GroupedGemmPlan(host, rhs)
        assert plan.launch_count() == degree
        c.check_tolerance(run_csr(c, plan), "grouped rocBLAS")
        plan.close()
    finally:
        c.close()


def test_grouped_gemm_plan_config3_and_empty_rows():
    note("grouped config3 + empty rows")
    host = vb.generate(4096, 4096, 8, "high", "random", 1)
    c = Case(host, 32, 1)
    try:
        plan = vb.GroupedGemmPlan(host, 32)
        c.check_tolerance(run_csr(c, plan), "grouped rocBLAS config3")
        plan.close()
    finally:
        c.close()
    empty = hand_made([8, 16, 24, 32], [8, 64, 40], [[], [0, 2], [], [1]])
    c = Case(empty, 16, 3)
    try:
        plan = vb.GroupedGemmPlan(empty, 16)
        c.check_tolerance(run_csr(c, plan), "grouped rocBLAS empty rows")  # empty rows must come out 0
        plan.close()
    finally:
        c.close()


@pytest.mark.parametrize("rhs", [8, 64])
def test_one_shot_baselines(rhs):
    """cusparse_scalar_baseline and slot_split_baseline (reference vbsr.hpp:163-168): one call builds the
    plan, executes it, waits for the stream and releases it; the result equals the persistent plan's bit
    for bit and is within tolerance of the oracle; an unsupported RHS is an invalid argument."""
    note(f"one-shot baselines rhs={rhs}")
    c = Case(vb.generate(40, 40, 4, "high", "random", 9), rhs, 9)
    try:
        for one_shot, plan_type in ((vb.cusparse_scalar_baseline, vb.ScalarCsrPlan),
                                    (vb.slot_split_baseline, vb.GroupedGemmPlan)):
            result = c.run(lambda: one_shot(c.host, c.b_dev, c.c_dev, rhs, c.stream))
            c.check_tolerance(result, one_shot.__name__)
            plan = plan_type(c.host, rhs)
            assert run_csr(c, plan).tobytes() == result.tobytes()
            plan.close()
            with pytest.raises(ValueError):
                one_shot(c.host, c.b_dev, c.c_dev[: c.host.scalar_rows * 12], 12, c.stream)
    finally:
        c.close()


# ---- the largest B offsets ------------------------------------------------

def largest_offset_case(scalar_cols, rhs):
    """Three block rows over scalar_cols / 64 - 1 block columns of width 64 followed by one of 24 and
    one of 40, using the first, a middle and the last (40-wide) block column, and a B panel
    (ld = scalar_cols) that is zero except where those columns are read.  The last block column ends
    at scalar_cols, so its 8-column half step reads the panel's last B rows at every RHS column: the
    largest offsets of both step kinds.  The panel is scalar_cols * rhs floats (4.6-4.9 GB);
    np.zeros leaves its untouched pages unallocated on the host."""
    ncols = scalar_cols // 64 + 1
    col_size = [64] * (ncols - 2) + [24, 40]
    assert sum(col_size) == scalar_cols
    host = hand_made([16, 40, 8], col_size, [[0, ncols - 1], [ncols // 2], [ncols - 1]], seed=5)
    rng = np.random.default_rng(9)
    b = np.zeros(scalar_cols * rhs, dtype=np.float32)
    for col in sorted({0, ncols // 2, ncols - 1}):
        start, end = int(host.col_scalar_off[col]), int(host.col_scalar_off[col + 1])
        for n in range(rhs):
            b[n * scalar_cols + start:n * scalar_cols + end] = rng.uniform(-1, 1, end - start).astype(np.float32)
    return host, b


def check_against_oracle(host, b, rhs, result, name):
    oracle = as_oracle(host)
    reference = o.cpu_reference(oracle, b, rhs)
    bound = o.abs_product_sum(oracle, b, rhs)
    assert np.all(np.isfinite(result)), name
    max_abs, rel_l2, normwise, elementwise = o.parity_errors(result, reference, bound)
    note(f"  {name}: max_abs={max_abs:.3g} rel_l2={rel_l2:.3g} normwise={normwise:.3g} elementwise={elementwise:.3g}")
    assert max_abs <= 5e-4 and rel_l2 <= 5e-5, name
    assert normwise <= NORMWISE_TOL and rel_l2 <= REL_L2_TOL and elementwise <= ELEMENTWISE_TOL, name


@pytest.mark.parametrize("scalar_cols,rhs", [(71_582_784, 16), (153_391_680, 8), (71_582_784, 64)])
def test_largest_b_offsets_take_the_mfma_kernel(scalar_cols, rhs):
    """The largest K (in whole 64-wide block columns) the MFMA kernel takes: its 32-bit B offsets
    within a 16-column tile reach (min(rhs, 16) - 1) * K * 4 + 64 bytes, 64 bytes or more below
    the out-of-range offset 0xfffffff0.  At RHS 64 both the split-k kernel and the tile split
    (forced through the schedule's rhs64_tiles) read every 16-column tile at those offsets."""
    note(f"largest offsets: K={scalar_cols} rhs={rhs} (B {scalar_cols * rhs * 4 / 2**30:.1f} GiB)")
    host, b = largest_offset_case(scalar_cols, rhs)
    matrix = vb.Matrix(host)
    try:
        stream = torch.cuda.Stream(device=DEVICE)
        b_dev = torch.from_numpy(b).to(DEVICE)
        c_dev = torch.full((host.scalar_rows * rhs,), float("nan"), device=DEVICE)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            vb.launch_row_owned(matrix.device_view(), matrix.row_schedule(), b_dev, c_dev, rhs, stream)
        stream.synchronize()
        check_against_oracle(host, b, rhs, c_dev.cpu().numpy(), "launch_row_owned")
        if rhs == 64:
            for tiles in (0, 1):
                schedule = matrix.row_schedule()
                schedule.rhs64_tiles = tiles
                c_dev.fill_(float("nan"))
                torch.cuda.synchronize()
                with torch.cuda.stream(stream):
                    vb.launch_row_owned(matrix.device_view(), schedule, b_dev, c_dev, rhs, stream)
                stream.synchronize()
                check_against_oracle(host, b, rhs, c_dev.cpu().numpy(), f"launch_row_owned, rhs64_tiles={tiles}")
        c_dev.fill_(float("nan"))
        torch.cuda.synchronize()
        plan = vb.Plan(matrix, rhs)
        with torch.cuda.stream(stream):
            plan.execute(b_dev, c_dev, stream)
        stream.synchronize()
        check_against_oracle(host, b, rhs, c_dev.cpu().numpy(), "plan")
        plan.close()
        del b_dev, c_dev
    finally:
        matrix.close()


@pytest.mark.parametrize("scalar_cols,rhs", [(71_582_848, 16), (153_391_744, 8), (71_582_848, 64)])
def test_k_past_the_offset_limit_stays_on_the_mfma_kernel(scalar_cols, rhs):
    """One block column past the largest K the 32-bit B offsets reach: launch_row_owned and the plan
    address B with 64-bit lane pointers instead, match the oracle, agree bit for bit with
    launch_row_owned_wide_b and with each other, and repeat bit for bit; the split-row path (same
    kernel, over row parts) matches the oracle too; the VALU variant, which keeps the offset bound,
    refuses the matrix.  At RHS 64 the same holds for the split-k kernel and the tile split, each
    forced through the schedule's rhs64_tiles."""
    note(f"past the offset limit: K={scalar_cols} rhs={rhs} (B {scalar_cols * rhs * 4 / 2**30:.1f} GiB)")
    host, b = largest_offset_case(scalar_cols, rhs)
    matrix = vb.Matrix(host)
    try:
        stream = torch.cuda.Stream(device=DEVICE)
        b_dev = torch.from_numpy(b).to(DEVICE)
        c_dev = torch.full((host.scalar_rows * rhs,), float("nan"), device=DEVICE)
        view, schedule = matrix.device_view(), matrix.row_schedule()

        def run(launch):
            c_dev.fill_(float("nan"))
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                launch()
            stream.synchronize()
            return c_dev.cpu().numpy().copy()

        first = run(lambda: vb.launch_row_owned(view, schedule, b_dev, c_dev, rhs, stream))
        check_against_oracle(host, b, rhs, first, "launch_row_owned past the limit")
        assert run(lambda: vb.launch_row_owned(view, schedule, b_dev, c_dev, rhs, stream)).tobytes() == first.tobytes()
        wide = run(lambda: vb.launch_row_owned_wide_b(view, schedule, b_dev, c_dev, rhs, stream))
        assert wide.tobytes() == first.tobytes(), "launch_row_owned_wide_b differs"
        plan = vb.Plan(matrix, rhs)
        assert plan.launch_count() == 1
        planned = run(lambda: plan.execute(b_dev, c_dev, stream))
        assert planned.tobytes() == first.tobytes(), "plan differs from launch_row_owned"
        split = run(lambda: vb.launch_split_row_static(matrix, b_dev, c_dev, rhs, stream))
        check_against_oracle(host, b, rhs, split, "split-row path past the limit")
        if rhs == 64:
            for tiles in (0, 1):
                forced = matrix.row_schedule()
                forced.rhs64_tiles = tiles
                got = run(lambda: vb.launch_row_owned(view, forced, b_dev, c_dev, rhs, stream))
                check_against_oracle(host, b, rhs, got, f"rhs64_tiles={tiles} past the limit")
                wide_forced = run(lambda: vb.launch_row_owned_wide_b(view, forced, b_dev, c_dev, rhs, stream))
                assert wide_forced.tobytes() == got.tobytes(), f"rhs64_tiles={tiles}: wide form differs"
        with pytest.raises(ValueError):
            vb.launch_row_owned_valu(view, schedule, b_dev, c_dev, rhs, stream)
        plan.close()
        del b_dev, c_dev
    finally:
        matrix.close()


def values_past_2_31_case():
    """2^15 filler block rows of 16 zero 64 x 64 blocks (exactly 2^31 values), then one block row of
    each height with random blocks of every width, whose values start at element 2^31 (byte 8 GiB)."""
    widths = [64, 8, 24, 40, 56, 16, 32, 48] * 8
    filler_rows, per_row = 1 << 15, 16
    tail_heights = [8, 24, 40, 56, 64, 16, 32, 48]
    rows_blocks = [[8 * (j % 8) for j in range(per_row)]] * filler_rows  # width-64 columns, each twice
    rows_blocks = rows_blocks + [[(r * 7 + j * 5) % len(widths) for j in range(5)] for r in range(len(tail_heights))]
    row_size = np.array([64] * filler_rows + tail_heights, dtype=np.int32)
    col_size = np.array(widths, dtype=np.int32)
    row_ptr = np.concatenate([[0], np.cumsum([len(b) for b in rows_blocks])])
    block_col = np.fromiter((c for b in rows_blocks for c in b), dtype=np.int32, count=int(row_ptr[-1]))
    owners = np.repeat(np.arange(len(row_size)), np.diff(row_ptr))
    value_off = np.concatenate([[0], np.cumsum(row_size[owners].astype(np.int64) * col_size[block_col])])
    first_tail_block = filler_rows * per_row
    assert value_off[first_tail_block] == 1 << 31
    values = np.zeros(int(value_off[-1]), dtype=np.float32)  # untouched zero pages until copied
    values[1 << 31:] = np.random.default_rng(5).uniform(-1, 1, len(values) - (1 << 31)).astype(np.float32)
    row_scalar_off = np.concatenate([[0], np.cumsum(row_size)])
    col_scalar_off = np.concatenate([[0], np.cumsum(col_size)])
    host = vb.HostMatrix(len(row_size), len(col_size), row_ptr=row_ptr, block_col=block_col, row_size=row_size,
                         col_size=col_size, row_scalar_off=row_scalar_off, col_scalar_off=col_scalar_off,
                         value_off=value_off, values=values)
    # The tail rows on their own, for the oracle.
    tail = vb.HostMatrix(len(tail_heights), len(col_size), row_ptr=row_ptr[filler_rows:] - first_tail_block,
                         block_col=block_col[first_tail_block:], row_size=row_size[filler_rows:], col_size=col_size,
                         row_scalar_off=row_scalar_off[filler_rows:] - row_scalar_off[filler_rows],
                         col_scalar_off=col_scalar_off, value_off=value_off[first_tail_block:] - (1 << 31),
                         values=values[1 << 31:])
    return host, tail, int(row_scalar_off[filler_rows])


def test_values_past_2_31_use_64_bit_offsets():
    """Blocks whose values start past element 2^31 of A: both kernels must read them through 64-bit
    value offsets.  The filler rows' C stays exactly 0; the last rows match the oracle, and the
    order-preserving kernel matches the fmaf emulation bit for bit."""
    free, _ = torch.cuda.mem_get_info(DEVICE)
    if free < 12 * 2**30:
        pytest.skip("needs 12 GiB of free device memory")
    note("values past 2^31: building the 8 GiB matrix")
    host, tail, first_tail_row = values_past_2_31_case()
    tail_oracle = as_oracle(tail)
    matrix = vb.Matrix(host)
    try:
        stream = torch.cuda.Stream(device=DEVICE)
        for rhs in (8, 16, 32, 64):
            note(f"values past 2^31: rhs={rhs}")
            b = o.make_random_input(host.scalar_cols * rhs, 40 + rhs)
            b_dev = torch.from_numpy(b).to(DEVICE)
            c_dev = torch.full((host.scalar_rows * rhs,), float("nan"), device=DEVICE)
            torch.cuda.synchronize()
            plan = vb.Plan(matrix, rhs)
            with torch.cuda.stream(stream):
                plan.execute(b_dev, c_dev, stream)
            stream.synchronize()
            out = c_dev.cpu().numpy().reshape(rhs, host.scalar_rows)
            assert np.all(out[:, :first_tail_row] == 0.0), "filler rows"
            check_against_oracle(tail, b, rhs, out[:, first_tail_row:].reshape(-1), f"plan rhs={rhs}")
            if rhs == 8:
                c_dev.fill_(float("nan"))
                torch.cuda.synchronize()
                with torch.cuda.stream(stream):
                    vb.launch_row_owned_scalar(matrix.device_view(), b_dev, c_dev, rhs, stream)
                stream.synchronize()
                out = c_dev.cpu().numpy().reshape(rhs, host.scalar_rows)
                assert np.all(out[:, :first_tail_row] == 0.0), "filler rows (scalar)"
                expected = o.fmaf_order(tail_oracle, b, rhs).reshape(rhs, -1)
                np.testing.assert_array_equal(out[:, first_tail_row:], expected, err_msg="scalar != fmaf emulation")
            plan.close()
            del b_dev, c_dev
    finally:
        matrix.close()


# ---- execute is stateless: concurrent streams, graph capture ---------------

def test_concurrent_executes_on_two_streams():
    """A row-owned plan keeps no state (no workspace, no atomics): two plans of one matrix run
    concurrently on two streams with their own B and C, and each matches its serial result."""
    host = vb.generate(512, 512, 8, "high", "random", 31)
    matrix = vb.Matrix(host)
    try:
        runs = []
        for rhs, seed in ((32, 1), (16, 2)):
            b = torch.from_numpy(o.make_random_input(host.scalar_cols * rhs, seed)).to(DEVICE)
            c = torch.full((host.scalar_rows * rhs,), float("nan"), device=DEVICE)
            runs.append((vb.Plan(matrix, rhs), b, c, torch.cuda.Stream(device=DEVICE)))
        interleave_and_compare(runs, events=False)
        for plan, _, _, _ in runs:
            plan.close()
    finally:
        matrix.close()


def interleave_and_compare(runs, events, oracle_checks=None):
    """Runs each (plan, B, C, stream) once alone, then 20 times interleaved across the streams (with an
    event after each execute that the other stream waits on, if `events`), and checks every final C bit
    for bit against its serial run and, where given, against the oracle."""
    serial = []
    for plan, b, c, stream in runs:
        with torch.cuda.stream(stream):
            plan.execute(b, c, stream)
        stream.synchronize()
        serial.append(c.cpu().numpy().copy())
        c.fill_(float("nan"))
    torch.cuda.synchronize()
    for _ in range(20):
        for i, (plan, b, c, stream) in enumerate(runs):
            with torch.cuda.stream(stream):
                plan.execute(b, c, stream)
                if events:
                    done = torch.cuda.Event()
                    done.record(stream)
                    runs[(i + 1) % len(runs)][3].wait_event(done)
    torch.cuda.synchronize()
    for i, ((plan, b, c, stream), expected) in enumerate(zip(runs, serial)):
        out = c.cpu().numpy()
        assert out.tobytes() == expected.tobytes(), f"run {i}: interleaved result differs from the serial run"
        if oracle_checks is not None:
            oracle_checks[i](out)


@pytest.mark.parametrize("kernel", ["auto", "split_row"])
def test_one_plan_on_two_streams_at_few_long_rows(kernel):
    """32 block rows of degree 16 at RHS 64, where the split-row path is advised.  A default plan (Auto:
    the row-owned kernel, stateless as the reference's) executes on two streams at once with different B
    and C -- the same plan handle on both streams, as two copies of a vbsr::Plan share it -- and every
    result equals its serial run and the oracle.  An explicit SplitRow plan shares one workspace across its
    executes, so there the streams are ordered by events, as documented, and the results are exact too."""
    rhs = 64
    host = vb.generate(32, 32, 16, "high", "random", 1)
    matrix = vb.Matrix(host)
    try:
        assert vb.split_row_advised(matrix, rhs)
        plan = vb.Plan(matrix, rhs, kernel)
        assert plan.launch_count() == (2 if kernel == "split_row" else 1)
        oracle_host = o.HostMatrix(host.block_rows, host.block_cols, **host.arrays())
        runs, checks = [], []
        for seed in (21, 22):
            b_host = o.make_random_input(host.scalar_cols * rhs, seed)
            expected = o.cpu_reference(oracle_host, b_host, rhs)
            bound = o.abs_product_sum(oracle_host, b_host, rhs)

            def check(out, expected=expected, bound=bound, seed=seed):
                _, rel_l2, normwise, elementwise = o.parity_errors(out, expected, bound)
                assert normwise <= 1e-5 and rel_l2 <= 1e-5 and elementwise <= 1e-6, f"seed {seed}"

            b = torch.from_numpy(b_host).to(DEVICE)
            c = torch.full((host.scalar_rows * rhs,), float("nan"), device=DEVICE)
            runs.append((plan, b, c, torch.cuda.Stream(device=DEVICE)))
            checks.append(check)
        interleave_and_compare(runs, events=kernel == "split_row", oracle_checks=checks)
        plan.close()
    finally:
        matrix.close()


@pytest.mark.parametrize("kernel,rhs,rows", [("auto", 32, 256), ("auto", 64, 2048), ("split_row", 32, 256)])
def test_plan_execute_replays_from_a_hip_graph(kernel, rhs, rows):
    """execute enqueues its kernels (one, or two on the split-row path, which uses the plan's own
    workspace) and allocates nothing, so it can be captured into a HIP graph; every replay, with eager
    work and synchronisations between replays, equals the eager result.  At RHS 64 and 2048 rows the
    plan runs the tile-split kernel."""
    host = vb.generate(rows, rows, 8, "high", "random", 41)
    c = Case(host, rhs, 41)
    try:
        if rhs == 64:
            assert c.matrix.row_schedule().rhs64_tiles == 1
        plan = vb.Plan(c.matrix, rhs, kernel)
        assert plan.launch_count() == (2 if kernel == "split_row" else 1)
        eager = c.run_plan(plan)
        c.check_tolerance(eager, "eager")
        capture_stream = torch.cuda.Stream(device=DEVICE)
        graph = torch.cuda.CUDAGraph()
        c.c_dev.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=capture_stream):
            plan.execute(c.b_dev, c.c_dev, capture_stream)
        for replay in range(5):
            c.c_dev.fill_(float("nan"))       # eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert c.c_dev.cpu().numpy().tobytes() == eager.tobytes(), f"replay {replay}"
        plan.close()
    finally:
        c.close()
