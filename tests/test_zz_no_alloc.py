"""The allocation-free split-row entry point (vbsr_launch_split_row_static), called through the C ABI,
against the entry point it varies (vbsr_launch_split_row with a caller-owned workspace): the same
kernels in the same order, so the results must be bit-identical; both are also checked against the
oracle with the parity bars of test_gpu_parity.py.  Two calls in a row, the second on a smaller
matrix, so the shared scratch holds the first call's partial slabs when the second starts."""

import numpy as np
import pytest

import oracle_ffi as o
import varblockspmm_amd as vb

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEVICE = "cuda:0"


def run(launch, c_dev):
    c_dev.fill_(float("nan"))
    torch.cuda.synchronize()
    launch()
    torch.cuda.synchronize()
    return c_dev.cpu().numpy().copy()


def test_static_scratch_launcher_matches_the_workspace_launcher():
    lib = vb.library()
    for rows, degree, distribution, rhs, seed in ((64, 16, "high", 64, 5), (24, 8, "bimodal", 32, 6)):
        print(f"static scratch: rows={rows} degree={degree} {distribution} rhs={rhs} seed={seed}", flush=True)
        host = vb.generate(rows, rows, degree, distribution, "random", seed)
        matrix = vb.Matrix(host)
        b = o.make_random_input(host.scalar_cols * rhs, seed)
        b_dev = torch.from_numpy(b).to(DEVICE)
        c_dev = torch.empty(host.scalar_rows * rhs, dtype=torch.float32, device=DEVICE)
        nbytes = vb.split_row_workspace_bytes(matrix, rhs)
        assert 0 < nbytes <= 16 << 20
        workspace = torch.empty(nbytes // 4, dtype=torch.float32, device=DEVICE)
        expected = run(lambda: vb.launch_split_row(matrix, b_dev, c_dev, rhs, workspace, nbytes), c_dev)
        status = lib.vbsr_launch_split_row_static(matrix._handle, b_dev.data_ptr(), c_dev.data_ptr(), rhs, None)
        assert status == vb.VBSR_OK, lib.vbsr_last_error()
        torch.cuda.synchronize()
        result = c_dev.cpu().numpy().copy()
        np.testing.assert_array_equal(result, expected)
        oracle = o.HostMatrix(host.block_rows, host.block_cols, **host.arrays())
        max_abs, rel_l2, normwise, elementwise = o.parity_errors(result, o.cpu_reference(oracle, b, rhs),
                                                                 o.abs_product_sum(oracle, b, rhs))
        assert np.all(np.isfinite(result))
        assert max_abs <= 5e-4 and rel_l2 <= 5e-5  # tests/test_main.cpp:35
        assert normwise <= 1e-5 and rel_l2 <= 1e-5 and elementwise <= 1e-6
        matrix.close()


def test_static_scratch_launcher_rejects_a_workspace_beyond_the_scratch():
    """Configuration 3 at RHS 64 needs about 113 MB of partial slabs: refused before any launch."""
    lib = vb.library()
    host = vb.generate(4096, 4096, 8, "high", "random", 1)
    matrix = vb.Matrix(host)
    rhs = 64
    assert vb.split_row_workspace_bytes(matrix, rhs) > 16 << 20
    b_dev = torch.zeros(host.scalar_cols * rhs, device=DEVICE)
    c_dev = torch.zeros(host.scalar_rows * rhs, device=DEVICE)
    status = lib.vbsr_launch_split_row_static(matrix._handle, b_dev.data_ptr(), c_dev.data_ptr(), rhs, None)
    assert status == vb.VBSR_INVALID_ARGUMENT
    assert b"static scratch" in lib.vbsr_last_error()
    torch.cuda.synchronize()
    matrix.close()
