// C++ API of the MI355X VBSR SpMM library: the same names, argument meaning
// and exception types as the reference's public header
// (King-Clawthorne/VarBlockSpMM include/varblockspmm/vbsr.hpp), implemented
// header-only over the C ABI in <vbsr.h>.  Streams are hipStream_t.
//
// Differences from the reference header:
//  - cpu_reference validates the matrix before reading it (the reference
//    reads an invalid one out of bounds).
//  - ScalarCsrPlan runs on rocSPARSE instead of cuSPARSE, and GroupedGemmPlan
//    on rocBLAS (one batched GEMM per slot and block shape) instead of
//    cuBLAS grouped GEMM; the one-shot helpers keep the reference's names
//    (cusparse_scalar_baseline runs the rocSPARSE plan).
//  - Distribution gains Bimodal8or64 and Tied8to64; GeneratorOptions gains
//    clamp_local_columns (clamped instead of cyclic local columns).
//  - launch_row_owned takes the matrix's row schedule instead of the
//    reference's row_shape_order and h <= 16 partition counts.
//  - Kernel::SplitRow, reserved and rejected in the reference, selects the
//    split-row path (also reachable as launch_split_row).  Kernel::Auto runs
//    the row-owned kernel, as the reference's does; split_row_advised says
//    when the split would pay.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include <vbsr.h>

namespace vbsr {

namespace detail {
inline void check(int status) {
  if (status == VBSR_OK) return;
  if (status == VBSR_INVALID_ARGUMENT) throw std::invalid_argument(vbsr_last_error());
  throw std::runtime_error(vbsr_last_error());
}
}  // namespace detail

/** Host-side variable-block sparse-row matrix (reference vbsr.hpp:16-29). */
struct HostMatrix {
  int block_rows{}, block_cols{};
  std::vector<int32_t> row_ptr, block_col, row_size, col_size;
  std::vector<int64_t> row_scalar_off, col_scalar_off, value_off;
  std::vector<float> values;
  int64_t scalar_rows() const { return row_scalar_off.empty() ? 0 : row_scalar_off.back(); }
  int64_t scalar_cols() const { return col_scalar_off.empty() ? 0 : col_scalar_off.back(); }

  vbsr_host_view view() const {
    vbsr_host_view v{};
    v.block_rows = block_rows;
    v.block_cols = block_cols;
    v.row_ptr = row_ptr.data();
    v.row_ptr_len = int64_t(row_ptr.size());
    v.block_col = block_col.data();
    v.block_col_len = int64_t(block_col.size());
    v.row_size = row_size.data();
    v.row_size_len = int64_t(row_size.size());
    v.col_size = col_size.data();
    v.col_size_len = int64_t(col_size.size());
    v.row_scalar_off = row_scalar_off.data();
    v.row_scalar_off_len = int64_t(row_scalar_off.size());
    v.col_scalar_off = col_scalar_off.data();
    v.col_scalar_off_len = int64_t(col_scalar_off.size());
    v.value_off = value_off.data();
    v.value_off_len = int64_t(value_off.size());
    v.values = values.data();
    v.values_len = int64_t(values.size());
    return v;
  }

  /** Throws std::invalid_argument if metadata or packed values are inconsistent. */
  void validate() const {
    const vbsr_host_view v = view();
    detail::check(vbsr_validate(&v));
  }
};

/** Non-owning device view (reference vbsr.hpp:32-38). */
using DeviceMatrix = vbsr_device_view;

/** Owns an immutable copy of a validated matrix in device memory (reference vbsr.hpp:41-64). */
class Matrix {
public:
  /** Copies `host` and all of its metadata to the current HIP device. */
  explicit Matrix(const HostMatrix& host) {
    const vbsr_host_view v = host.view();
    vbsr_matrix* handle = nullptr;
    detail::check(vbsr_matrix_create(&v, &handle));
    handle_ = handle;
  }
  ~Matrix() { vbsr_matrix_destroy(handle_); }
  Matrix(const Matrix&) = delete;
  Matrix& operator=(const Matrix&) = delete;
  Matrix(Matrix&& other) noexcept : handle_(std::exchange(other.handle_, nullptr)) {}
  Matrix& operator=(Matrix&& other) noexcept {
    if (this != &other) {
      vbsr_matrix_destroy(handle_);
      handle_ = std::exchange(other.handle_, nullptr);
    }
    return *this;
  }
  /** Returns a non-owning view valid for this object's lifetime. */
  DeviceMatrix device_view() const {
    DeviceMatrix v{};
    detail::check(vbsr_matrix_device_view(handle_, &v));
    return v;
  }
  int64_t scalar_rows() const { return vbsr_matrix_scalar_rows(handle_); }
  int64_t scalar_cols() const { return vbsr_matrix_scalar_cols(handle_); }
  /** The row schedule that Plan passes to launch_row_owned. */
  vbsr_row_schedule row_schedule() const {
    vbsr_row_schedule schedule{};
    detail::check(vbsr_matrix_row_schedule(handle_, &schedule));
    return schedule;
  }
  const vbsr_matrix* handle() const { return handle_; }

private:
  vbsr_matrix* handle_{};
};

/** Distribution of block heights and widths (reference vbsr.hpp:67, plus two extensions). */
enum class Distribution { Uniform, LowVariance, HighVariance, Bimodal, Bimodal8or64, Tied8to64 };

/** Parameters for deterministic synthetic generation (reference vbsr.hpp:70-76). */
struct GeneratorOptions {
  int block_rows = 1024, block_cols = 1024, degree = 4;
  int rhs_width = 32;
  Distribution distribution = Distribution::HighVariance;
  bool local_columns = true;
  bool clamp_local_columns = false;
  uint64_t seed = 1;
};

/** Generates a validated matrix from `options`; equal seeds give equal matrices. */
inline HostMatrix generate(const GeneratorOptions& o) {
  vbsr_generator_options c{};
  c.block_rows = o.block_rows;
  c.block_cols = o.block_cols;
  c.degree = o.degree;
  c.rhs_width = o.rhs_width;
  c.distribution = int32_t(o.distribution);
  c.locality = !o.local_columns ? VBSR_LOCALITY_RANDOM
                                : (o.clamp_local_columns ? VBSR_LOCALITY_LOCAL_CLAMPED : VBSR_LOCALITY_LOCAL);
  c.seed = o.seed;
  vbsr_host_matrix* handle = nullptr;
  detail::check(vbsr_generate(&c, &handle));
  std::unique_ptr<vbsr_host_matrix, void (*)(vbsr_host_matrix*)> owner(handle, vbsr_host_matrix_destroy);
  vbsr_host_view v{};
  detail::check(vbsr_host_matrix_view(handle, &v));
  HostMatrix m;
  m.block_rows = v.block_rows;
  m.block_cols = v.block_cols;
  m.row_ptr.assign(v.row_ptr, v.row_ptr + v.row_ptr_len);
  m.block_col.assign(v.block_col, v.block_col + v.block_col_len);
  m.row_size.assign(v.row_size, v.row_size + v.row_size_len);
  m.col_size.assign(v.col_size, v.col_size + v.col_size_len);
  m.row_scalar_off.assign(v.row_scalar_off, v.row_scalar_off + v.row_scalar_off_len);
  m.col_scalar_off.assign(v.col_scalar_off, v.col_scalar_off + v.col_scalar_off_len);
  m.value_off.assign(v.value_off, v.value_off + v.value_off_len);
  m.values.assign(v.values, v.values + v.values_len);
  return m;
}

/** Computes `C = A * B` on the CPU with double-precision accumulation
 * (reference vbsr.hpp:82-87): the reference's arithmetic, so the result is
 * bit-identical to the reference's.  `B` and the returned `C` are
 * column-major; `B` must hold `matrix.scalar_cols() * rhs` elements
 * (std::invalid_argument "B size" otherwise).  The matrix is validated first. */
inline std::vector<float> cpu_reference(const HostMatrix& matrix, const std::vector<float>& B, int rhs) {
  const vbsr_host_view v = matrix.view();
  std::vector<float> C;
  int64_t c_len = 0;
  if (rhs > 0 && !__builtin_mul_overflow(matrix.scalar_rows(), int64_t(rhs), &c_len) && c_len > 0) C.resize(size_t(c_len));
  detail::check(vbsr_cpu_reference(&v, B.data(), int64_t(B.size()), rhs, C.data(), int64_t(C.size())));
  return C;
}

/** Kernel selection (reference vbsr.hpp:91).  Auto and RowOwned run the
 * row-owned kernel (no workspace; a plan may execute on several streams at
 * once), as in the reference.  SplitRow, reserved in the reference, is the
 * split-row path here: two launches and a plan-owned workspace, so one such
 * plan (or a copy of it, which shares the workspace) must not execute on two
 * streams at once, and must outlive any HIP graph captured from it. */
enum class Kernel { Auto, RowOwned, SplitRow };

/** Configuration for a reusable execution plan (reference vbsr.hpp:94-97). */
struct PlanOptions {
  int rhs_width = 32;
  Kernel kernel = Kernel::Auto;
};

/** Execution plan (reference vbsr.hpp:104-119).  The Matrix must outlive the plan;
 * execute enqueues asynchronously on the given stream. */
class Plan {
public:
  Plan(const Matrix& matrix, PlanOptions options) {
    const vbsr_plan_options c{options.rhs_width, int32_t(options.kernel)};
    vbsr_plan* handle = nullptr;
    detail::check(vbsr_plan_create(matrix.handle(), &c, &handle));
    plan_.reset(handle, vbsr_plan_destroy);
  }
  /** Enqueues C = A * B; both dense matrices are column-major device buffers. */
  void execute(const float* B, float* C, hipStream_t stream = 0) const {
    detail::check(vbsr_plan_execute(plan_.get(), B, C, stream));
  }
  /** Returns the number of kernel launches used by one execution. */
  int launch_count() const { return vbsr_plan_launch_count(plan_.get()); }

private:
  std::shared_ptr<vbsr_plan> plan_;
};

/** Persistent rocSPARSE baseline on an expanded scalar CSR copy of the
 * matrix (reference ScalarCsrPlan, vbsr.hpp:121-136).  Not thread-safe. */
class ScalarCsrPlan {
public:
  ScalarCsrPlan(const HostMatrix& matrix, int rhs_width) {
    const vbsr_host_view v = matrix.view();
    vbsr_csr_plan* handle = nullptr;
    detail::check(vbsr_csr_plan_create(&v, rhs_width, &handle));
    plan_.reset(handle);
  }
  ScalarCsrPlan(const ScalarCsrPlan&) = delete;
  ScalarCsrPlan& operator=(const ScalarCsrPlan&) = delete;
  /** Enqueues the baseline multiplication on `stream`. */
  void execute(const float* B, float* C, hipStream_t stream = 0) {
    detail::check(vbsr_csr_plan_execute(plan_.get(), B, C, stream));
  }
  /** Returns persistent temporary storage allocated after the first execution. */
  size_t workspace_bytes() const { return size_t(vbsr_csr_plan_workspace_bytes(plan_.get())); }

private:
  struct Destroy {
    void operator()(vbsr_csr_plan* p) const { vbsr_csr_plan_destroy(p); }
  };
  std::unique_ptr<vbsr_csr_plan, Destroy> plan_;
};

/** Persistent rocBLAS baseline that groups equally shaped blocks of each
 * block slot into batched GEMMs (reference GroupedGemmPlan, vbsr.hpp:138-152).
 * Not thread-safe. */
class GroupedGemmPlan {
public:
  GroupedGemmPlan(const HostMatrix& matrix, int rhs_width) {
    const vbsr_host_view v = matrix.view();
    vbsr_gemm_plan* handle = nullptr;
    detail::check(vbsr_gemm_plan_create(&v, rhs_width, &handle));
    plan_.reset(handle);
  }
  GroupedGemmPlan(const GroupedGemmPlan&) = delete;
  GroupedGemmPlan& operator=(const GroupedGemmPlan&) = delete;
  /** Enqueues all grouped GEMM batches on `stream`. */
  void execute(const float* B, float* C, hipStream_t stream = 0) {
    detail::check(vbsr_gemm_plan_execute(plan_.get(), B, C, stream));
  }
  /** Returns the number of sequential block slots. */
  int launch_count() const { return vbsr_gemm_plan_launch_count(plan_.get()); }
  size_t workspace_bytes() const { return 0; }

private:
  struct Destroy {
    void operator()(vbsr_gemm_plan* p) const { vbsr_gemm_plan_destroy(p); }
  };
  std::unique_ptr<vbsr_gemm_plan, Destroy> plan_;
};

/** The tuned row-owned kernels (reference vbsr.hpp:158-159). */
inline void launch_row_owned(DeviceMatrix matrix, const vbsr_row_schedule& schedule, const float* B, float* C,
                             int rhs, hipStream_t stream) {
  detail::check(vbsr_launch_row_owned(&matrix, &schedule, B, C, rhs, stream));
}

/** Bytes of workspace the split-row path needs for `matrix` at `rhs`. */
inline int64_t split_row_workspace_bytes(const Matrix& matrix, int rhs) {
  int64_t bytes = 0;
  detail::check(vbsr_split_row_workspace_bytes(matrix.handle(), rhs, &bytes));
  return bytes;
}

/** Whether the split-row path is expected to beat the row-owned kernel for
 * `matrix` at `rhs` (few row-owned workgroups, long rows, rhs >= 16).  No
 * counterpart in the reference; no plan acts on it by itself. */
inline bool split_row_advised(const Matrix& matrix, int rhs) {
  int32_t advised = 0;
  detail::check(vbsr_matrix_split_row_advised(matrix.handle(), rhs, &advised));
  return advised != 0;
}

/** The split-row path (the reference's reserved Kernel::SplitRow) with a
 * caller-owned device workspace of split_row_workspace_bytes(matrix, rhs). */
inline void launch_split_row(const Matrix& matrix, const float* B, float* C, int rhs, void* workspace,
                             int64_t workspace_bytes, hipStream_t stream) {
  detail::check(vbsr_launch_split_row(matrix.handle(), B, C, rhs, workspace, workspace_bytes, stream));
}

/** One-shot, synchronizing library baseline (reference vbsr.hpp:163-165):
 * the rocSPARSE ScalarCsrPlan built, executed and released.  Prefer
 * `ScalarCsrPlan` for repeated work. */
inline void cusparse_scalar_baseline(const HostMatrix& matrix, const float* dB, float* dC, int rhs,
                                     hipStream_t stream) {
  const vbsr_host_view v = matrix.view();
  detail::check(vbsr_scalar_csr_baseline(&v, dB, dC, rhs, stream));
}

/** One-shot, synchronizing grouped baseline (reference vbsr.hpp:166-168):
 * the rocBLAS GroupedGemmPlan built, executed and released.  Prefer
 * `GroupedGemmPlan` for reuse. */
inline void slot_split_baseline(const HostMatrix& matrix, const float* dB, float* dC, int rhs, hipStream_t stream) {
  const vbsr_host_view v = matrix.view();
  detail::check(vbsr_slot_split_baseline(&v, dB, dC, rhs, stream));
}

/** The reference-order kernel (reference vbsr.hpp:161). */
inline void launch_row_owned_scalar(DeviceMatrix matrix, const float* B, float* C, int rhs, hipStream_t stream) {
  detail::check(vbsr_launch_row_owned_scalar(&matrix, B, C, rhs, stream));
}

}  // namespace vbsr
