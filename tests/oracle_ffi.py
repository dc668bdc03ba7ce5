"""ctypes bindings for the CPU oracle (oracle/liboracle.so).

Test infrastructure: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py only, always as the checker.
"""

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")

DISTRIBUTIONS = {"uniform": 0, "low": 1, "high": 2, "bimodal": 3, "bimodal8or64": 4, "tied8to64": 5}
LOCALITIES = {"random": 0, "local": 1, "clamped": 2}


class OrcMatrix(ctypes.Structure):
    _fields_ = [
        ("block_rows", ctypes.c_int32), ("block_cols", ctypes.c_int32),
        ("nnzb", ctypes.c_int64), ("value_count", ctypes.c_int64),
        ("row_ptr", ctypes.POINTER(ctypes.c_int32)), ("block_col", ctypes.POINTER(ctypes.c_int32)),
        ("row_size", ctypes.POINTER(ctypes.c_int32)), ("col_size", ctypes.POINTER(ctypes.c_int32)),
        ("row_scalar_off", ctypes.POINTER(ctypes.c_int64)), ("col_scalar_off", ctypes.POINTER(ctypes.c_int64)),
        ("value_off", ctypes.POINTER(ctypes.c_int64)), ("values", ctypes.POINTER(ctypes.c_float)),
    ]


_VIEW_FIELDS = [("row_ptr", ctypes.c_int32), ("block_col", ctypes.c_int32), ("row_size", ctypes.c_int32),
                ("col_size", ctypes.c_int32), ("row_scalar_off", ctypes.c_int64),
                ("col_scalar_off", ctypes.c_int64), ("value_off", ctypes.c_int64), ("values", ctypes.c_float)]


class OrcView(ctypes.Structure):
    _fields_ = [("block_rows", ctypes.c_int32), ("block_cols", ctypes.c_int32)] + [
        item for name, ctype in _VIEW_FIELDS
        for item in ((name, ctypes.POINTER(ctype)), (name + "_len", ctypes.c_int64))]


class MT64(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64 * 312), ("index", ctypes.c_int)]


class MT32(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint32 * 624), ("index", ctypes.c_int)]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            build()
        L = ctypes.CDLL(ORACLE_LIB)
        L.orc_mt64_next.restype = ctypes.c_uint64
        L.orc_mt64_next.argtypes = [ctypes.POINTER(MT64)]
        L.orc_mt32_next.restype = ctypes.c_uint32
        L.orc_mt32_next.argtypes = [ctypes.POINTER(MT32)]
        L.orc_mt64_seed.argtypes = [ctypes.POINTER(MT64), ctypes.c_uint64]
        L.orc_mt32_seed.argtypes = [ctypes.POINTER(MT32), ctypes.c_uint32]
        L.orc_uniform_pm1_from_u64.restype = ctypes.c_float
        L.orc_uniform_pm1_from_u64.argtypes = [ctypes.c_uint64]
        L.orc_uniform_pm1_from_u32.restype = ctypes.c_float
        L.orc_uniform_pm1_from_u32.argtypes = [ctypes.c_uint32]
        L.orc_generate.argtypes = [ctypes.c_int32] * 5 + [ctypes.c_uint64, ctypes.POINTER(OrcMatrix)]
        L.orc_generate_structure.argtypes = L.orc_generate.argtypes
        L.orc_matrix_free.argtypes = [ctypes.POINTER(OrcMatrix)]
        L.orc_validate.argtypes = [ctypes.POINTER(OrcView), ctypes.POINTER(ctypes.c_int)]
        for name, out_type in (("orc_cpu_reference", ctypes.c_float), ("orc_fmaf_order", ctypes.c_float),
                               ("orc_abs_product_sum", ctypes.c_double)):
            getattr(L, name).argtypes = [ctypes.POINTER(OrcView), ctypes.POINTER(ctypes.c_float), ctypes.c_int64,
                                         ctypes.c_int32, ctypes.POINTER(out_type)]
        L.orc_cpu_reference_threads.argtypes = [ctypes.POINTER(OrcView), ctypes.POINTER(ctypes.c_float),
                                                ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                                ctypes.POINTER(ctypes.c_float)]
        L.orc_abs_product_sum_threads.argtypes = [ctypes.POINTER(OrcView), ctypes.POINTER(ctypes.c_float),
                                                  ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                                  ctypes.POINTER(ctypes.c_double)]
        L.orc_make_random_input.argtypes = [ctypes.c_int64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_float)]
        L.orc_useful_flops.restype = ctypes.c_double
        L.orc_useful_flops.argtypes = [ctypes.POINTER(OrcView), ctypes.c_int32]
        _lib = L
    return _lib


class HostMatrix:
    """numpy-held host VBSR matrix with the reference HostMatrix fields."""

    FIELDS = ("row_ptr", "block_col", "row_size", "col_size", "row_scalar_off", "col_scalar_off",
              "value_off", "values")
    DTYPES = {"row_ptr": np.int32, "block_col": np.int32, "row_size": np.int32, "col_size": np.int32,
              "row_scalar_off": np.int64, "col_scalar_off": np.int64, "value_off": np.int64,
              "values": np.float32}

    def __init__(self, block_rows, block_cols, **arrays):
        self.block_rows = int(block_rows)
        self.block_cols = int(block_cols)
        for name in self.FIELDS:
            setattr(self, name, np.ascontiguousarray(arrays[name], dtype=self.DTYPES[name]))

    def copy(self):
        return HostMatrix(self.block_rows, self.block_cols,
                          **{name: getattr(self, name).copy() for name in self.FIELDS})

    @property
    def scalar_rows(self):
        return int(self.row_scalar_off[-1]) if len(self.row_scalar_off) else 0

    @property
    def scalar_cols(self):
        return int(self.col_scalar_off[-1]) if len(self.col_scalar_off) else 0

    @property
    def nnzb(self):
        return len(self.block_col)

    def sum_hw(self):
        owner = np.repeat(np.arange(self.block_rows), np.diff(self.row_ptr))
        return int(np.sum(self.row_size[owner].astype(np.int64) * self.col_size[self.block_col]))

    def view(self):
        """An OrcView over this matrix; keep self alive while it is used."""
        v = OrcView()
        v.block_rows = self.block_rows
        v.block_cols = self.block_cols
        for name, ctype in _VIEW_FIELDS:
            array = getattr(self, name)
            setattr(v, name, array.ctypes.data_as(ctypes.POINTER(ctype)))
            setattr(v, name + "_len", len(array))
        return v

    def dense(self):
        """Dense float64 expansion (brute-force checks on tiny matrices)."""
        dense = np.zeros((self.scalar_rows, self.scalar_cols))
        for i in range(self.block_rows):
            h = int(self.row_size[i])
            r0 = int(self.row_scalar_off[i])
            for blk in range(self.row_ptr[i], self.row_ptr[i + 1]):
                c = int(self.block_col[blk])
                w = int(self.col_size[c])
                c0 = int(self.col_scalar_off[c])
                block = self.values[self.value_off[blk]:self.value_off[blk + 1]].reshape(w, h).T
                dense[r0:r0 + h, c0:c0 + w] += block
        return dense


def generate(block_rows, block_cols, degree, distribution="high", locality="random", seed=1):
    L = lib()
    m = OrcMatrix()
    dist = DISTRIBUTIONS[distribution] if isinstance(distribution, str) else int(distribution)
    loc = LOCALITIES[locality] if isinstance(locality, str) else int(locality)
    status = L.orc_generate(block_rows, block_cols, degree, dist, loc, seed, ctypes.byref(m))
    if status == 1:
        raise ValueError("invalid generator dimensions")
    if status != 0:
        raise MemoryError("oracle generator out of memory")
    try:
        R, C, nnzb, nv = m.block_rows, m.block_cols, m.nnzb, m.value_count

        def take(ptr, n, dtype):
            return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True) if n else np.zeros(0, dtype)

        return HostMatrix(R, C,
                          row_ptr=take(m.row_ptr, R + 1, np.int32), block_col=take(m.block_col, nnzb, np.int32),
                          row_size=take(m.row_size, R, np.int32), col_size=take(m.col_size, C, np.int32),
                          row_scalar_off=take(m.row_scalar_off, R + 1, np.int64),
                          col_scalar_off=take(m.col_scalar_off, C + 1, np.int64),
                          value_off=take(m.value_off, nnzb + 1, np.int64), values=take(m.values, nv, np.float32))
    finally:
        L.orc_matrix_free(ctypes.byref(m))


def validate(matrix):
    """Returns the failed rule code (0 when valid)."""
    rule = ctypes.c_int(0)
    view = matrix.view()
    status = lib().orc_validate(ctypes.byref(view), ctypes.byref(rule))
    return 0 if status == 0 else rule.value


def _product(name, matrix, b, rhs, dtype):
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty(matrix.scalar_rows * rhs, dtype=dtype)
    view = matrix.view()
    ctype = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    status = getattr(lib(), name)(ctypes.byref(view), b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(b),
                                  rhs, out.ctypes.data_as(ctypes.POINTER(ctype)))
    if status != 0:
        raise ValueError("B size")
    return out


def cpu_reference(matrix, b, rhs):
    """C = A*B, column-major M x rhs, double per-block dots (vbsr.cpp:167-201)."""
    return _product("orc_cpu_reference", matrix, b, rhs, np.float32)


def cpu_reference_threads(matrix, b, rhs, threads):
    """cpu_reference with block rows spread over `threads` OpenMP threads; bit-identical to it."""
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty(matrix.scalar_rows * rhs, dtype=np.float32)
    view = matrix.view()
    status = lib().orc_cpu_reference_threads(ctypes.byref(view), b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                             len(b), rhs, threads, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    if status != 0:
        raise ValueError("B size or thread count")
    return out


def fmaf_order(matrix, b, rhs):
    """Bit-exact emulation of the reference kernels' fmaf chain."""
    return _product("orc_fmaf_order", matrix, b, rhs, np.float32)


def abs_product_sum(matrix, b, rhs):
    return _product("orc_abs_product_sum", matrix, b, rhs, np.float64)


def abs_product_sum_threads(matrix, b, rhs, threads):
    """abs_product_sum with block rows spread over `threads` OpenMP threads; bit-identical to it."""
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty(matrix.scalar_rows * rhs, dtype=np.float64)
    view = matrix.view()
    status = lib().orc_abs_product_sum_threads(ctypes.byref(view), b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                               len(b), rhs, threads,
                                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    if status != 0:
        raise ValueError("B size or thread count")
    return out


def make_random_input(count, seed):
    out = np.empty(count, dtype=np.float32)
    lib().orc_make_random_input(count, seed, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def useful_flops(matrix, rhs):
    view = matrix.view()
    return lib().orc_useful_flops(ctypes.byref(view), rhs)


def parity_errors(result, reference, bound):
    """(max_abs, rel_l2, normwise, elementwise-vs-max-bound) error metrics.

    max_abs and rel_l2 are the reference test's (tests/test_main.cpp:19-35);
    normwise = max|C - Cref| / max|Cref|; the last is
    max|C - Cref| / max(sum |a||b|).
    """
    result = np.asarray(result, dtype=np.float64)
    reference = np.asarray(reference, dtype=np.float64)
    err = result - reference
    max_abs = float(np.max(np.abs(err))) if err.size else 0.0
    rel_l2 = float(np.sqrt(np.sum(err * err) / (np.sum(reference * reference) + 1e-30)))
    normwise = max_abs / (float(np.max(np.abs(reference))) + 1e-30) if err.size else 0.0
    elementwise = max_abs / (float(np.max(bound)) + 1e-30) if err.size else 0.0
    return max_abs, rel_l2, normwise, elementwise
