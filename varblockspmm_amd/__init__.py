"""Python host mirror of the VBSR SpMM library's C ABI (include/vbsr.h).

Names follow the reference C++ API (King-Clawthorne/VarBlockSpMM,
include/varblockspmm/vbsr.hpp): ``HostMatrix``, ``validate``, ``generate``,
``Matrix``, ``Plan`` (``execute``, ``launch_count``), ``launch_row_owned`` and
``launch_row_owned_scalar``.  Errors keep the reference's split:
``ValueError`` where it throws std::invalid_argument, ``RuntimeError`` where it
throws std::runtime_error.

Every computation runs in libvarblockspmm_amd.so (HIP kernels for gfx950).
There is no CPU fallback: importing raises if the library is not built.
Device buffers and streams are passed as integers (device addresses, stream
handles) or as torch tensors / torch streams, whose addresses are taken.
"""

import ctypes
import os

import numpy as np

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(PACKAGE_DIR, "libvarblockspmm_amd.so")

VBSR_OK, VBSR_INVALID_ARGUMENT, VBSR_RUNTIME_ERROR = 0, 1, 2

DISTRIBUTIONS = {"uniform": 0, "low": 1, "high": 2, "bimodal": 3, "bimodal8or64": 4, "tied8to64": 5}
LOCALITIES = {"random": 0, "local": 1, "clamped": 2}
KERNELS = {"auto": 0, "row_owned": 1, "split_row": 2}

_ARRAYS = (("row_ptr", ctypes.c_int32, np.int32), ("block_col", ctypes.c_int32, np.int32),
           ("row_size", ctypes.c_int32, np.int32), ("col_size", ctypes.c_int32, np.int32),
           ("row_scalar_off", ctypes.c_int64, np.int64), ("col_scalar_off", ctypes.c_int64, np.int64),
           ("value_off", ctypes.c_int64, np.int64), ("values", ctypes.c_float, np.float32))


class HostView(ctypes.Structure):
    _fields_ = [("block_rows", ctypes.c_int32), ("block_cols", ctypes.c_int32)] + [
        item for name, ctype, _ in _ARRAYS
        for item in ((name, ctypes.POINTER(ctype)), (name + "_len", ctypes.c_int64))]


class DeviceView(ctypes.Structure):
    _fields_ = [("block_rows", ctypes.c_int32), ("block_cols", ctypes.c_int32), ("nnzb", ctypes.c_int32),
                ("scalar_rows", ctypes.c_int64), ("scalar_cols", ctypes.c_int64),
                ("row_ptr", ctypes.c_void_p), ("block_col", ctypes.c_void_p), ("row_size", ctypes.c_void_p),
                ("col_size", ctypes.c_void_p), ("row_scalar_off", ctypes.c_void_p),
                ("col_scalar_off", ctypes.c_void_p), ("value_off", ctypes.c_void_p), ("values", ctypes.c_void_p)]


class GeneratorOptions(ctypes.Structure):
    _fields_ = [("block_rows", ctypes.c_int32), ("block_cols", ctypes.c_int32), ("degree", ctypes.c_int32),
                ("rhs_width", ctypes.c_int32), ("distribution", ctypes.c_int32), ("locality", ctypes.c_int32),
                ("seed", ctypes.c_uint64)]


class RowSchedule(ctypes.Structure):
    _fields_ = [("steps", ctypes.c_void_p), ("rows", ctypes.c_void_p), ("groups", ctypes.c_int64),
                ("step_limit", ctypes.c_int32), ("rows_wide", ctypes.c_void_p), ("rows_rhs64", ctypes.c_void_p),
                ("groups_rhs64", ctypes.c_int64), ("rows_tile", ctypes.c_void_p), ("groups_tile", ctypes.c_int64),
                ("rhs64_tiles", ctypes.c_int32)]


class PlanOptions(ctypes.Structure):
    _fields_ = [("rhs_width", ctypes.c_int32), ("kernel", ctypes.c_int32)]


# Every symbol include/vbsr.h declares, with its ctypes signature.
_P = ctypes.c_void_p
SIGNATURES = {
    "vbsr_last_error": (ctypes.c_char_p, []),
    "vbsr_validate": (ctypes.c_int, [ctypes.POINTER(HostView)]),
    "vbsr_generate": (ctypes.c_int, [ctypes.POINTER(GeneratorOptions), ctypes.POINTER(_P)]),
    "vbsr_host_matrix_view": (ctypes.c_int, [_P, ctypes.POINTER(HostView)]),
    "vbsr_host_matrix_destroy": (None, [_P]),
    "vbsr_make_random_input": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_float)]),
    "vbsr_cpu_reference": (ctypes.c_int, [ctypes.POINTER(HostView), ctypes.POINTER(ctypes.c_float), ctypes.c_int64,
                                          ctypes.c_int32, ctypes.POINTER(ctypes.c_float), ctypes.c_int64]),
    "vbsr_matrix_create": (ctypes.c_int, [ctypes.POINTER(HostView), ctypes.POINTER(_P)]),
    "vbsr_matrix_destroy": (None, [_P]),
    "vbsr_matrix_device_view": (ctypes.c_int, [_P, ctypes.POINTER(DeviceView)]),
    "vbsr_matrix_scalar_rows": (ctypes.c_int64, [_P]),
    "vbsr_matrix_scalar_cols": (ctypes.c_int64, [_P]),
    "vbsr_matrix_row_schedule": (ctypes.c_int, [_P, ctypes.POINTER(RowSchedule)]),
    "vbsr_plan_create": (ctypes.c_int, [_P, ctypes.POINTER(PlanOptions), ctypes.POINTER(_P)]),
    "vbsr_plan_destroy": (None, [_P]),
    "vbsr_plan_execute": (ctypes.c_int, [_P, _P, _P, _P]),
    "vbsr_plan_launch_count": (ctypes.c_int, [_P]),
    "vbsr_launch_row_owned": (ctypes.c_int, [ctypes.POINTER(DeviceView), ctypes.POINTER(RowSchedule), _P, _P,
                                             ctypes.c_int32, _P]),
    "vbsr_launch_row_owned_wide_b": (ctypes.c_int, [ctypes.POINTER(DeviceView), ctypes.POINTER(RowSchedule), _P, _P,
                                                    ctypes.c_int32, _P]),
    "vbsr_launch_row_owned_scalar": (ctypes.c_int, [ctypes.POINTER(DeviceView), _P, _P, ctypes.c_int32, _P]),
    "vbsr_launch_row_owned_valu": (ctypes.c_int, [ctypes.POINTER(DeviceView), ctypes.POINTER(RowSchedule), _P, _P,
                                                  ctypes.c_int32, _P]),
    "vbsr_split_row_workspace_bytes": (ctypes.c_int, [_P, ctypes.c_int32, ctypes.POINTER(ctypes.c_int64)]),
    "vbsr_matrix_split_row_advised": (ctypes.c_int, [_P, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32)]),
    "vbsr_launch_split_row": (ctypes.c_int, [_P, _P, _P, ctypes.c_int32, _P, ctypes.c_int64, _P]),
    "vbsr_launch_split_row_static": (ctypes.c_int, [_P, _P, _P, ctypes.c_int32, _P]),
    "vbsr_csr_plan_create": (ctypes.c_int, [ctypes.POINTER(HostView), ctypes.c_int32, ctypes.POINTER(_P)]),
    "vbsr_csr_plan_destroy": (None, [_P]),
    "vbsr_csr_plan_execute": (ctypes.c_int, [_P, _P, _P, _P]),
    "vbsr_csr_plan_workspace_bytes": (ctypes.c_int64, [_P]),
    "vbsr_gemm_plan_create": (ctypes.c_int, [ctypes.POINTER(HostView), ctypes.c_int32, ctypes.POINTER(_P)]),
    "vbsr_gemm_plan_destroy": (None, [_P]),
    "vbsr_gemm_plan_execute": (ctypes.c_int, [_P, _P, _P, _P]),
    "vbsr_gemm_plan_launch_count": (ctypes.c_int, [_P]),
    "vbsr_scalar_csr_baseline": (ctypes.c_int, [ctypes.POINTER(HostView), _P, _P, ctypes.c_int32, _P]),
    "vbsr_slot_split_baseline": (ctypes.c_int, [ctypes.POINTER(HostView), _P, _P, ctypes.c_int32, _P]),
}

_lib = None


def library():
    """The loaded libvarblockspmm_amd.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise ImportError(f"{LIBRARY_PATH} is missing: build it with `python -c "
                              f"'import __graft_entry__ as g; g.build()'` (make -C varblockspmm_amd/csrc)")
        lib = ctypes.CDLL(LIBRARY_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def _check(status):
    if status == VBSR_OK:
        return
    message = library().vbsr_last_error().decode(errors="replace")
    if status == VBSR_INVALID_ARGUMENT:
        raise ValueError(message)
    raise RuntimeError(message)


def _address(obj):
    """Device address of a torch tensor, or an integer address (0 = null)."""
    if obj is None:
        return None
    if hasattr(obj, "data_ptr"):
        return obj.data_ptr() or None
    return int(obj) or None


def _check_panel(panel, expected, name):
    """For torch tensors, checks what the C ABI cannot: dtype, layout, device and size."""
    if not hasattr(panel, "data_ptr"):
        return
    import torch
    if panel.dtype != torch.float32 or not panel.is_contiguous() or not panel.is_cuda:
        raise ValueError(f"{name} must be a contiguous float32 device tensor")
    if panel.numel() != expected:
        raise ValueError(f"{name} holds {panel.numel()} floats, expected {expected}")


def _stream(stream):
    if stream is None:
        return None
    if hasattr(stream, "cuda_stream"):
        return stream.cuda_stream or None
    return int(stream) or None


class HostMatrix:
    """Host VBSR matrix with the reference HostMatrix fields (vbsr.hpp:16-29), held as numpy arrays."""

    def __init__(self, block_rows, block_cols, **arrays):
        self.block_rows = int(block_rows)
        self.block_cols = int(block_cols)
        for name, _, dtype in _ARRAYS:
            setattr(self, name, np.ascontiguousarray(arrays[name], dtype=dtype))

    @property
    def scalar_rows(self):
        return int(self.row_scalar_off[-1]) if len(self.row_scalar_off) else 0

    @property
    def scalar_cols(self):
        return int(self.col_scalar_off[-1]) if len(self.col_scalar_off) else 0

    @property
    def nnzb(self):
        return len(self.block_col)

    def copy(self):
        return HostMatrix(self.block_rows, self.block_cols, **{n: getattr(self, n).copy() for n, _, _ in _ARRAYS})

    def arrays(self):
        return {name: getattr(self, name) for name, _, _ in _ARRAYS}

    def _view(self):
        view = HostView()
        view.block_rows = self.block_rows
        view.block_cols = self.block_cols
        for name, ctype, dtype in _ARRAYS:
            array = getattr(self, name)
            if array.dtype != dtype or not array.flags.c_contiguous:
                array = np.ascontiguousarray(array, dtype=dtype)
                setattr(self, name, array)
            setattr(view, name, array.ctypes.data_as(ctypes.POINTER(ctype)))
            setattr(view, name + "_len", len(array))
        return view

    def validate(self):
        """HostMatrix::validate (vbsr.cpp:29-82); raises ValueError."""
        view = self._view()
        _check(library().vbsr_validate(ctypes.byref(view)))


def validate(matrix):
    matrix.validate()


def generate(block_rows=1024, block_cols=1024, degree=4, distribution="high", locality="local", seed=1,
             rhs_width=32):
    """generate (vbsr.hpp:80; generator.cpp:7-88).  distribution: uniform|low|high|bimodal (reference)
    or bimodal8or64|tied8to64; locality: local (cyclic, reference), random, clamped."""
    options = GeneratorOptions(block_rows, block_cols, degree, rhs_width,
                               DISTRIBUTIONS[distribution] if isinstance(distribution, str) else int(distribution),
                               LOCALITIES[locality] if isinstance(locality, str) else int(locality), seed)
    lib = library()
    handle = ctypes.c_void_p()
    _check(lib.vbsr_generate(ctypes.byref(options), ctypes.byref(handle)))
    try:
        view = HostView()
        _check(lib.vbsr_host_matrix_view(handle, ctypes.byref(view)))
        arrays = {}
        for name, _, dtype in _ARRAYS:
            length = getattr(view, name + "_len")
            pointer = getattr(view, name)
            arrays[name] = (np.ctypeslib.as_array(pointer, shape=(length,)).astype(dtype, copy=True)
                            if length else np.zeros(0, dtype))
        return HostMatrix(view.block_rows, view.block_cols, **arrays)
    finally:
        lib.vbsr_host_matrix_destroy(handle)


def make_random_input(count, seed):
    """The reference test's B (tests/test_main.cpp:42-51) as a float32 numpy array."""
    out = np.empty(int(count), dtype=np.float32)
    _check(library().vbsr_make_random_input(int(count), int(seed), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
    return out


def cpu_reference(matrix, B, rhs_width):
    """cpu_reference (vbsr.hpp:82-87; vbsr.cpp:167-201): C = A*B on the host in the reference's arithmetic
    (double sum per block, FP32 across blocks).  B and the returned C are column-major float32 numpy arrays;
    raises ValueError ("B size") when B does not hold scalar_cols * rhs_width floats."""
    b = np.ascontiguousarray(B, dtype=np.float32)
    rhs = int(rhs_width)
    c = np.empty(max(0, matrix.scalar_rows * rhs), dtype=np.float32)
    view = matrix._view()
    fp = ctypes.POINTER(ctypes.c_float)
    _check(library().vbsr_cpu_reference(ctypes.byref(view), b.ctypes.data_as(fp), len(b), rhs, c.ctypes.data_as(fp),
                                        len(c)))
    return c


class Matrix:
    """Owning device copy of a validated matrix (reference Matrix, vbsr.hpp:41-64), on the current HIP device."""

    def __init__(self, host):
        view = host._view()
        handle = ctypes.c_void_p()
        _check(library().vbsr_matrix_create(ctypes.byref(view), ctypes.byref(handle)))
        self._handle = handle

    def close(self):
        if getattr(self, "_handle", None):
            library().vbsr_matrix_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def device_view(self):
        view = DeviceView()
        _check(library().vbsr_matrix_device_view(self._handle, ctypes.byref(view)))
        return view

    def row_schedule(self):
        """The row schedule Plan passes to launch_row_owned (a RowSchedule)."""
        schedule = RowSchedule()
        _check(library().vbsr_matrix_row_schedule(self._handle, ctypes.byref(schedule)))
        return schedule

    @property
    def scalar_rows(self):
        return library().vbsr_matrix_scalar_rows(self._handle)

    @property
    def scalar_cols(self):
        return library().vbsr_matrix_scalar_cols(self._handle)


class Plan:
    """Reusable execution plan (reference Plan, vbsr.hpp:104-119).  The Matrix must outlive the plan."""

    def __init__(self, matrix, rhs_width=32, kernel="auto"):
        options = PlanOptions(int(rhs_width), KERNELS[kernel] if isinstance(kernel, str) else int(kernel))
        handle = ctypes.c_void_p()
        _check(library().vbsr_plan_create(matrix._handle, ctypes.byref(options), ctypes.byref(handle)))
        self._handle = handle
        self._matrix = matrix
        self.rhs_width = int(rhs_width)

    def close(self):
        if getattr(self, "_handle", None):
            library().vbsr_plan_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def execute(self, B, C, stream=None):
        """Enqueues C = A*B (column-major device buffers) on `stream`; asynchronous."""
        _check_panel(B, self._matrix.scalar_cols * self.rhs_width, "B")
        _check_panel(C, self._matrix.scalar_rows * self.rhs_width, "C")
        _check(library().vbsr_plan_execute(self._handle, _address(B), _address(C), _stream(stream)))

    def launch_count(self):
        return library().vbsr_plan_launch_count(self._handle)


def launch_row_owned(device_view, schedule, B, C, rhs, stream=None):
    """launch_row_owned (vbsr.hpp:158-159): the tuned kernel on a device view with its matrix's schedule."""
    _check_panel(B, device_view.scalar_cols * int(rhs), "B")
    _check_panel(C, device_view.scalar_rows * int(rhs), "C")
    _check(library().vbsr_launch_row_owned(ctypes.byref(device_view), ctypes.byref(schedule), _address(B),
                                           _address(C), int(rhs), _stream(stream)))


def launch_row_owned_wide_b(device_view, schedule, B, C, rhs, stream=None):
    """launch_row_owned with B read through 64-bit lane addresses at any K (the form it takes past
    the 32-bit offset bound); bit-identical to launch_row_owned."""
    _check_panel(B, device_view.scalar_cols * int(rhs), "B")
    _check_panel(C, device_view.scalar_rows * int(rhs), "C")
    _check(library().vbsr_launch_row_owned_wide_b(ctypes.byref(device_view), ctypes.byref(schedule), _address(B),
                                                  _address(C), int(rhs), _stream(stream)))


def launch_row_owned_valu(device_view, schedule, B, C, rhs, stream=None):
    """The row-owned kernel with plain FP32 multiply-adds instead of MFMA tiles (the measured alternative)."""
    _check_panel(B, device_view.scalar_cols * int(rhs), "B")
    _check_panel(C, device_view.scalar_rows * int(rhs), "C")
    _check(library().vbsr_launch_row_owned_valu(ctypes.byref(device_view), ctypes.byref(schedule), _address(B),
                                                _address(C), int(rhs), _stream(stream)))


def launch_row_owned_scalar(device_view, B, C, rhs, stream=None):
    """launch_row_owned_scalar (vbsr.hpp:161): the reference-order kernel."""
    _check_panel(B, device_view.scalar_cols * int(rhs), "B")
    _check_panel(C, device_view.scalar_rows * int(rhs), "C")
    _check(library().vbsr_launch_row_owned_scalar(ctypes.byref(device_view), _address(B), _address(C), int(rhs),
                                                  _stream(stream)))


def split_row_workspace_bytes(matrix, rhs):
    """Bytes of device workspace the split-row path needs for `matrix` at `rhs`."""
    out = ctypes.c_int64()
    _check(library().vbsr_split_row_workspace_bytes(matrix._handle, int(rhs), ctypes.byref(out)))
    return out.value


def split_row_advised(matrix, rhs):
    """Whether the split-row path is expected to beat the row-owned kernel for `matrix` at `rhs` (few row-owned
    workgroups, long rows, rhs >= 16).  Plans never act on it by themselves: Kernel::Auto is the row-owned
    kernel, as in the reference."""
    out = ctypes.c_int32()
    _check(library().vbsr_matrix_split_row_advised(matrix._handle, int(rhs), ctypes.byref(out)))
    return bool(out.value)


def launch_split_row(matrix, B, C, rhs, workspace, workspace_bytes=None, stream=None):
    """The split-row path (the reference's reserved Kernel::SplitRow) with a caller-owned workspace: partial slabs
    of each row's parts into `workspace`, then their fixed-order sum into C.  Two launches."""
    _check_panel(B, matrix.scalar_cols * int(rhs), "B")
    _check_panel(C, matrix.scalar_rows * int(rhs), "C")
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size() if hasattr(workspace, "numel") else 0
    _check(library().vbsr_launch_split_row(matrix._handle, _address(B), _address(C), int(rhs), _address(workspace),
                                           int(workspace_bytes), _stream(stream)))


def launch_split_row_static(matrix, B, C, rhs, stream=None):
    """The split-row path with the library's static device scratch as its workspace (16 MiB per device):
    allocates nothing; calls that overlap on one device race."""
    _check_panel(B, matrix.scalar_cols * int(rhs), "B")
    _check_panel(C, matrix.scalar_rows * int(rhs), "C")
    _check(library().vbsr_launch_split_row_static(matrix._handle, _address(B), _address(C), int(rhs),
                                                  _stream(stream)))


class ScalarCsrPlan:
    """The rocSPARSE scalar-CSR baseline (reference ScalarCsrPlan, vbsr.hpp:121-136): the host matrix is
    expanded to CSR and copied to the device; execute runs rocsparse_spmm.  Not thread-safe."""

    def __init__(self, host, rhs_width):
        handle = ctypes.c_void_p()
        view = host._view()
        _check(library().vbsr_csr_plan_create(ctypes.byref(view), int(rhs_width), ctypes.byref(handle)))
        self._handle = handle
        self.rhs_width = int(rhs_width)
        self.scalar_rows = host.scalar_rows
        self.scalar_cols = host.scalar_cols

    def close(self):
        if getattr(self, "_handle", None):
            library().vbsr_csr_plan_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def execute(self, B, C, stream=None):
        """Enqueues C = A*B on `stream`; the first call also allocates the workspace."""
        _check_panel(B, self.scalar_cols * self.rhs_width, "B")
        _check_panel(C, self.scalar_rows * self.rhs_width, "C")
        _check(library().vbsr_csr_plan_execute(self._handle, _address(B), _address(C), _stream(stream)))

    def workspace_bytes(self):
        return library().vbsr_csr_plan_workspace_bytes(self._handle)


class GroupedGemmPlan:
    """The rocBLAS slot-grouped baseline (reference GroupedGemmPlan, vbsr.hpp:138-152): slot s holds the
    s-th block of every block row, grouped by block shape; one batched GEMM per (slot, shape).
    Not thread-safe."""

    def __init__(self, host, rhs_width):
        handle = ctypes.c_void_p()
        view = host._view()
        _check(library().vbsr_gemm_plan_create(ctypes.byref(view), int(rhs_width), ctypes.byref(handle)))
        self._handle = handle
        self.rhs_width = int(rhs_width)
        self.scalar_rows = host.scalar_rows
        self.scalar_cols = host.scalar_cols

    def close(self):
        if getattr(self, "_handle", None):
            library().vbsr_gemm_plan_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def execute(self, B, C, stream=None):
        """Enqueues C = A*B on `stream` (C is zeroed first)."""
        _check_panel(B, self.scalar_cols * self.rhs_width, "B")
        _check_panel(C, self.scalar_rows * self.rhs_width, "C")
        _check(library().vbsr_gemm_plan_execute(self._handle, _address(B), _address(C), _stream(stream)))

    def launch_count(self):
        return library().vbsr_gemm_plan_launch_count(self._handle)

    def workspace_bytes(self):
        return 0


def cusparse_scalar_baseline(host, B, C, rhs, stream=None):
    """One-shot, synchronising library baseline (reference cusparse_scalar_baseline, vbsr.hpp:163-165): the
    rocSPARSE ScalarCsrPlan built, executed on `stream`, waited for and released."""
    _check_panel(B, host.scalar_cols * int(rhs), "B")
    _check_panel(C, host.scalar_rows * int(rhs), "C")
    view = host._view()
    _check(library().vbsr_scalar_csr_baseline(ctypes.byref(view), _address(B), _address(C), int(rhs),
                                              _stream(stream)))


def slot_split_baseline(host, B, C, rhs, stream=None):
    """One-shot, synchronising grouped baseline (reference slot_split_baseline, vbsr.hpp:166-168): the rocBLAS
    GroupedGemmPlan built, executed on `stream`, waited for and released."""
    _check_panel(B, host.scalar_cols * int(rhs), "B")
    _check_panel(C, host.scalar_rows * int(rhs), "C")
    view = host._view()
    _check(library().vbsr_slot_split_baseline(ctypes.byref(view), _address(B), _address(C), int(rhs),
                                              _stream(stream)))
