"""Host side of the library (no GPU): generate, validate and the test-input
generator, checked against the oracle bit for bit, plus the C ABI surface."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import oracle_ffi as o
import varblockspmm_amd as vb
from reference_cases import reference_cases

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def as_oracle(host):
    return o.HostMatrix(host.block_rows, host.block_cols, **host.arrays())


def assert_same_matrix(product, oracle):
    assert (product.block_rows, product.block_cols) == (oracle.block_rows, oracle.block_cols)
    for name in o.HostMatrix.FIELDS:
        np.testing.assert_array_equal(getattr(product, name), getattr(oracle, name), err_msg=name)


@pytest.mark.parametrize("distribution", list(vb.DISTRIBUTIONS))
@pytest.mark.parametrize("locality", list(vb.LOCALITIES))
@pytest.mark.parametrize("shape", [(9, 17, 4, 11), (33, 20, 16, 12), (25, 25, 1, 13)])
def test_generate_matches_oracle(distribution, locality, shape):
    R, C, d, seed = shape
    product = vb.generate(R, C, d, distribution, locality, seed)
    oracle = o.generate(R, C, d, distribution, locality, seed)
    assert_same_matrix(product, oracle)


def test_generate_matches_oracle_at_benchmark_size():
    """BASELINE configuration 2's matrix (1024 rows, degree 8, low variance, random, seed 2)."""
    assert_same_matrix(vb.generate(1024, 1024, 8, "low", "random", 2), o.generate(1024, 1024, 8, "low", "random", 2))


def test_generate_rejects_bad_options():
    for args in [(0, 4, 1), (4, 0, 1), (4, 4, 0), (4, 4, 17), (4, 3, 4)]:
        with pytest.raises(ValueError):
            vb.generate(*args)
    with pytest.raises(ValueError):
        vb.generate(4, 4, 1, distribution=9)
    with pytest.raises(ValueError):
        vb.generate(4, 4, 1, locality=7)


def test_make_random_input_matches_oracle():
    for count, seed in [(1, 0), (1000, 11), (4097, (1 << 32) + 3)]:
        np.testing.assert_array_equal(vb.make_random_input(count, seed), o.make_random_input(count, seed))


def test_validate_matches_oracle_rule_by_rule():
    import test_oracle

    base = vb.generate(4, 4, 2, "high", "local", 1)
    base.validate()
    for description, mutate, rule in test_oracle.mutations():
        m = as_oracle(base).copy()
        mutate(m)
        product = vb.HostMatrix(m.block_rows, m.block_cols, **{n: getattr(m, n) for n in o.HostMatrix.FIELDS})
        assert o.validate(m) == rule, description
        with pytest.raises(ValueError):
            product.validate()


def test_validate_accepts_what_the_reference_accepts():
    import test_oracle

    m = test_oracle._rows_with_empty()
    vb.HostMatrix(m.block_rows, m.block_cols, **{n: getattr(m, n) for n in o.HostMatrix.FIELDS}).validate()
    shifted = vb.generate(6, 6, 2, "high", "random", 3)
    shifted.row_scalar_off = shifted.row_scalar_off + 8
    shifted.validate()


# ---- the C ABI surface ------------------------------------------------------------------------------


def declared_symbols():
    with open(os.path.join(ROOT, "include", "vbsr.h")) as handle:
        text = handle.read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(vbsr_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = vb.library()
    names = declared_symbols()
    assert len(names) >= 18
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(vb.SIGNATURES)


def test_library_links_no_oracle_code():
    out = subprocess.run(["nm", "-D", "--defined-only", vb.LIBRARY_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "orc_" not in out
    assert "liboracle" not in subprocess.run(["ldd", vb.LIBRARY_PATH], capture_output=True, text=True).stdout


def test_library_holds_gfx950_code_objects():
    out = subprocess.run(["strings", vb.LIBRARY_PATH], capture_output=True, text=True, check=True).stdout
    assert "gfx950" in out


def test_cpp_api_header_compiles():
    source = ('#include <varblockspmm/vbsr.hpp>\n'
              'int main() { vbsr::GeneratorOptions o; o.block_rows = 3; (void)o; return 0; }\n')
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(ROOT, "include"), "-x", "c++", "-"], input=source, text=True, check=True)


def test_null_arguments_are_rejected_without_a_gpu():
    lib = vb.library()
    assert lib.vbsr_validate(None) == vb.VBSR_INVALID_ARGUMENT
    assert b"null" in lib.vbsr_last_error()
    assert lib.vbsr_plan_execute(None, None, None, None) == vb.VBSR_INVALID_ARGUMENT
    assert lib.vbsr_matrix_device_view(None, None) == vb.VBSR_INVALID_ARGUMENT
    assert lib.vbsr_plan_launch_count(None) == 0
    lib.vbsr_matrix_destroy(None)
    lib.vbsr_plan_destroy(None)


def test_validate_rejects_null_arrays_and_negative_lengths():
    """The C view can carry a null array or a negative length, which the reference's vectors cannot:
    validate rejects both instead of reading through them."""
    lib = vb.library()
    host = vb.generate(9, 17, 4, "high", "local", 11)
    for name in ("row_ptr", "block_col", "row_size", "col_size", "row_scalar_off", "col_scalar_off", "value_off",
                 "values"):
        view = host._view()
        setattr(view, name, None)
        assert lib.vbsr_validate(ctypes.byref(view)) == vb.VBSR_INVALID_ARGUMENT, name
        assert b"null array" in lib.vbsr_last_error(), name
    for name in ("block_col_len", "values_len"):
        view = host._view()
        setattr(view, name, -1)
        assert lib.vbsr_validate(ctypes.byref(view)) == vb.VBSR_INVALID_ARGUMENT, name
    assert lib.vbsr_validate(ctypes.byref(host._view())) == vb.VBSR_OK


def test_reciprocal_division_used_by_the_mfma_kernel_is_exact():
    """row_owned_mfma.hip finds the block column of each loaded float as (f * ceil(2^16 / h)) >> 16
    instead of f / h: exact for every float index f < 1024 of a step and every block height."""
    for h in range(8, 65, 8):
        recip = -(-65536 // h)
        f = np.arange(1024, dtype=np.uint64)
        np.testing.assert_array_equal((f * recip) >> 16, f // h, err_msg=f"h={h}")


def test_launchers_reject_bad_rhs_before_touching_the_gpu():
    view = vb.DeviceView()
    view.block_rows = 4
    for rhs in (0, 7, 12, 128):
        with pytest.raises(ValueError):
            vb.launch_row_owned(view, vb.RowSchedule(), None, None, rhs)
        with pytest.raises(ValueError):
            vb.launch_row_owned_scalar(view, None, None, rhs)


def test_launchers_reject_null_and_overlapping_panels_before_touching_the_gpu():
    """The C ABI refuses a null B or C, a B or C that is not 4-byte aligned, and a C whose range
    (scalar_rows * rhs floats) meets B's (scalar_cols * rhs floats): C is written while B is read.  Addresses here are never
    dereferenced; every call is refused on the host."""
    view = vb.DeviceView()
    view.block_rows, view.scalar_rows, view.scalar_cols = 4, 96, 80
    rhs = 8
    b = 0x7f0000000000
    b_end = b + 80 * rhs * 4
    launchers = (lambda bb, cc: vb.launch_row_owned(view, vb.RowSchedule(), bb, cc, rhs),
                 lambda bb, cc: vb.launch_row_owned_scalar(view, bb, cc, rhs))
    for launch in launchers:
        for bb, cc in ((None, b_end), (b, None), (None, None)):
            with pytest.raises(ValueError, match="device pointers"):
                launch(bb, cc)
        for bb, cc in ((b + 2, b_end), (b, b_end + 2)):
            with pytest.raises(ValueError, match="4-byte aligned"):
                launch(bb, cc)
        # C starting inside B, C ending inside B, C equal to B, C covering B.
        for cc in (b_end - 4, b - 96 * rhs * 4 + 4, b, b - 256):
            with pytest.raises(ValueError, match="overlap"):
                launch(b, cc)


def test_launchers_reject_a_schedule_without_its_launch_order_before_touching_the_gpu():
    """A schedule is the matrix's own (vbsr_matrix_row_schedule), whose every launch order holds at
    least one workgroup when the matrix has block rows.  A zeroed struct, or one whose RHS 64 choice
    (rhs64_tiles) names an order it does not hold, is refused on the host instead of launching
    nothing or reading through a null pointer.  Addresses here are never dereferenced."""
    view = vb.DeviceView()
    view.block_rows, view.scalar_rows, view.scalar_cols = 4, 96, 80
    b, c = 0x7f0000000000, 0x7f0000100000
    for rhs in (8, 16, 32, 64):
        with pytest.raises(ValueError, match="launch order"):
            vb.launch_row_owned(view, vb.RowSchedule(), b, c, rhs)
    fake = 0x7f0000200000
    for rows_tile, groups_tile in ((None, 0), (fake, 0), (None, 8)):
        s = vb.RowSchedule()
        s.steps = s.rows = s.rows_wide = s.rows_rhs64 = fake
        s.groups = s.groups_rhs64 = 8
        s.rows_tile, s.groups_tile, s.rhs64_tiles = rows_tile, groups_tile, 1
        with pytest.raises(ValueError, match="launch order"):
            vb.launch_row_owned(view, s, b, c, 64)


def test_launchers_check_torch_panels_before_touching_the_gpu():
    """The Python launchers check what the C ABI cannot see: a torch panel must be a contiguous
    float32 device tensor of exactly scalar_cols * rhs (B) or scalar_rows * rhs (C) floats."""
    torch = pytest.importorskip("torch")
    view = vb.DeviceView()
    view.block_rows, view.scalar_rows, view.scalar_cols = 4, 96, 80
    host_b = torch.zeros(80 * 8)  # right size, but host memory
    for launch in (lambda b, c: vb.launch_row_owned(view, vb.RowSchedule(), b, c, 8),
                   lambda b, c: vb.launch_row_owned_scalar(view, b, c, 8)):
        with pytest.raises(ValueError, match="device tensor"):
            launch(host_b, None)
        with pytest.raises(ValueError, match="device tensor"):
            launch(None, torch.zeros(96 * 8, dtype=torch.float64))


def test_csr_plan_rejects_bad_input_before_touching_the_gpu():
    host = vb.generate(4, 6, 2, "high", "random", 5)
    for rhs in (0, 12, 128):
        with pytest.raises(ValueError):
            vb.ScalarCsrPlan(host, rhs)
    bad = host.copy()
    bad.row_size[0] = 7
    with pytest.raises(ValueError):
        vb.ScalarCsrPlan(bad, 8)
    lib = vb.library()
    assert lib.vbsr_csr_plan_create(None, 8, None) == vb.VBSR_INVALID_ARGUMENT
    assert lib.vbsr_csr_plan_execute(None, None, None, None) == vb.VBSR_INVALID_ARGUMENT
    assert lib.vbsr_csr_plan_workspace_bytes(None) == 0
    lib.vbsr_csr_plan_destroy(None)


def test_grouped_gemm_plan_rejects_bad_input_before_touching_the_gpu():
    host = vb.generate(4, 6, 2, "high", "random", 5)
    for rhs in (0, 24, 128):
        with pytest.raises(ValueError):
            vb.GroupedGemmPlan(host, rhs)
    bad = host.copy()
    bad.row_size[0] = 7
    with pytest.raises(ValueError):
        vb.GroupedGemmPlan(bad, 8)
    lib = vb.library()
    assert lib.vbsr_gemm_plan_create(None, 8, None) == vb.VBSR_INVALID_ARGUMENT
    assert lib.vbsr_gemm_plan_execute(None, None, None, None) == vb.VBSR_INVALID_ARGUMENT
    assert lib.vbsr_gemm_plan_launch_count(None) == 0
    lib.vbsr_gemm_plan_destroy(None)


# ---- cpu_reference (vbsr.hpp:82-87; vbsr.cpp:167-201), exported by the library ----------------------------


@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: "{}-d{}-n{}-{}-s{}".format(*c))
def test_cpu_reference_is_bit_identical_to_the_oracle(case):
    """The library's cpu_reference against the oracle's restatement of the reference's, bit for bit, on the
    reference test's own parameter matrix (tests/test_main.cpp:145-161, the cases it calls cpu_reference on
    at :73)."""
    distribution, degree, rhs, locality, seed = case
    host = vb.generate(9, 17, degree, distribution, locality, seed)
    b = vb.make_random_input(host.scalar_cols * rhs, seed)
    np.testing.assert_array_equal(vb.cpu_reference(host, b, rhs), o.cpu_reference(as_oracle(host), b, rhs))


def test_cpu_reference_is_bit_identical_to_the_oracle_at_configuration_1():
    """BASELINE configuration 1, the CPU-only one: 1024 block rows, degree 4, high sizes, clamped local
    columns, RHS 8, seed 1."""
    host = vb.generate(1024, 1024, 4, "high", "clamped", 1)
    b = vb.make_random_input(host.scalar_cols * 8, 1)
    np.testing.assert_array_equal(vb.cpu_reference(host, b, 8), o.cpu_reference(as_oracle(host), b, 8))


def test_cpu_reference_accepts_any_rhs_and_shifted_row_offsets():
    """Like the reference's, it takes any non-negative RHS width (not only the kernels' four), and row offsets
    that start above 0 (those C rows stay zero)."""
    host = vb.generate(6, 7, 2, "bimodal", "random", 5)
    for rhs in (1, 3, 12):
        b = vb.make_random_input(host.scalar_cols * rhs, rhs)
        np.testing.assert_array_equal(vb.cpu_reference(host, b, rhs), o.cpu_reference(as_oracle(host), b, rhs))
    assert len(vb.cpu_reference(host, np.zeros(0, np.float32), 0)) == 0
    shifted = host.copy()
    shifted.row_scalar_off = shifted.row_scalar_off + 16
    b = vb.make_random_input(host.scalar_cols * 8, 2)
    c = vb.cpu_reference(shifted, b, 8).reshape(8, -1)
    assert np.all(c[:, :16] == 0)
    np.testing.assert_array_equal(c[:, 16:], vb.cpu_reference(host, b, 8).reshape(8, -1))


def test_cpu_reference_rejects_what_the_reference_rejects_and_invalid_matrices():
    host = vb.generate(4, 6, 2, "high", "random", 5)
    b = vb.make_random_input(host.scalar_cols * 8, 1)
    for bad_b in (b[:-1], np.concatenate([b, b[:1]])):
        with pytest.raises(ValueError, match="B size"):  # vbsr.cpp:169-171
            vb.cpu_reference(host, bad_b, 8)
    with pytest.raises(ValueError, match="B size"):
        vb.cpu_reference(host, b, -8)
    bad = host.copy()
    bad.row_size[0] = 7
    with pytest.raises(ValueError):
        vb.cpu_reference(bad, b, 8)
    negative = host.copy()
    negative.col_scalar_off = negative.col_scalar_off - 8
    with pytest.raises(ValueError, match="negative"):
        vb.cpu_reference(negative, b, 8)
    lib = vb.library()
    assert lib.vbsr_cpu_reference(None, None, 0, 8, None, 0) == vb.VBSR_INVALID_ARGUMENT


def test_cpu_reference_holds_the_closed_forms():
    """Identity blocks copy B's slices; a unit B column extracts A's columns (independent of the oracle)."""
    host = vb.generate(5, 5, 1, "high", "random", 9)
    h = host.row_size
    w = host.col_size[host.block_col]
    host.values = np.concatenate([np.eye(hh, ww, dtype=np.float32).ravel(order="F") for hh, ww in zip(h, w)])
    host.value_off = np.concatenate([[0], np.cumsum(h * w)]).astype(np.int64)
    host.validate()
    rhs = 8
    b = vb.make_random_input(host.scalar_cols * rhs, 4)
    c = vb.cpu_reference(host, b, rhs).reshape(rhs, -1)
    bb = b.reshape(rhs, -1)
    for i in range(host.block_rows):
        r0, c0 = host.row_scalar_off[i], host.col_scalar_off[host.block_col[i]]
        m = min(h[i], w[i])
        np.testing.assert_array_equal(c[:, r0:r0 + m], bb[:, c0:c0 + m])
        assert np.all(c[:, r0 + m:r0 + h[i]] == 0)
