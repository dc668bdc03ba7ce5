// ScalarCsrPlan: the counterpart of the reference's cuSPARSE baseline
// (src/baseline/cusparse_baseline.cu:35-188, declared at
// include/varblockspmm/vbsr.hpp:121-136), on rocSPARSE.
//
// The VBSR matrix is expanded once, on the host, to scalar CSR: scalar rows
// in order, and within a row the blocks in row_ptr order, each block's
// columns ascending (cusparse_baseline.cu:35-64).  Execution is rocSPARSE's
// generic SpMM (rocsparse_spmm, default algorithm) with column-major dense
// descriptors, alpha = 1 and beta = 0.  As in the reference, the dense
// descriptors and the workspace are created at the first execute and reused
// afterwards (cusparse_baseline.cu:167-181); the plan is not thread-safe.
#include <algorithm>
#include <cstring>

#include <hip/hip_runtime_api.h>
#include <rocsparse/rocsparse.h>

#include "internal.hpp"

namespace vbsr_amd {
namespace {

void check_rocsparse(rocsparse_status status, const char* what) {
  if (status != rocsparse_status_success)
    throw std::runtime_error(std::string("rocSPARSE failure in ") + what + ": " + std::to_string(int(status)));
}

template <class T>
T* upload(const std::vector<T>& source) {
  T* destination = nullptr;
  const size_t bytes = std::max<size_t>(source.size(), 1) * sizeof(T);
  check_hip(hipMalloc(reinterpret_cast<void**>(&destination), bytes), "hipMalloc");
  if (!source.empty()) {
    const hipError_t status = hipMemcpy(destination, source.data(), source.size() * sizeof(T), hipMemcpyHostToDevice);
    if (status != hipSuccess) {
      (void)hipFree(destination);
      check_hip(status, "hipMemcpy");
    }
  }
  return destination;
}

}  // namespace

ScalarCsr expand_to_scalar_csr(const vbsr_host_view& m) {
  const int64_t rows = m.row_scalar_off[m.block_rows];
  if (m.values_len > int64_t(INT32_MAX))
    throw std::invalid_argument("scalar CSR needs fewer than 2^31 stored values");
  ScalarCsr csr;
  csr.row_offsets.resize(static_cast<size_t>(rows) + 1);
  csr.columns.reserve(static_cast<size_t>(m.values_len));
  csr.values.reserve(static_cast<size_t>(m.values_len));
  for (int32_t i = 0; i < m.block_rows; ++i) {
    const int32_t h = m.row_size[i];
    for (int32_t r = 0; r < h; ++r) {
      csr.row_offsets[static_cast<size_t>(m.row_scalar_off[i] + r)] = int32_t(csr.values.size());
      for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) {
        const int32_t col = m.block_col[blk];
        const int32_t w = m.col_size[col];
        const float* block = m.values + m.value_off[blk];
        for (int32_t k = 0; k < w; ++k) {
          csr.columns.push_back(int32_t(m.col_scalar_off[col] + k));
          csr.values.push_back(block[r + int64_t(k) * h]);
        }
      }
    }
  }
  csr.row_offsets.back() = int32_t(csr.values.size());
  return csr;
}

CsrPlan::CsrPlan(const vbsr_host_view& host, int rhs) : rhs_(rhs) {
  validate(host);
  if (!supported_rhs(rhs)) throw std::invalid_argument("rhs_width must be 8,16,32,64");
  if (host.row_scalar_off[0] != 0 || host.col_scalar_off[0] != 0)
    throw std::invalid_argument("scalar offsets must start at 0");
  const ScalarCsr csr = expand_to_scalar_csr(host);
  rows_ = host.row_scalar_off[host.block_rows];
  cols_ = host.col_scalar_off[host.block_cols];
  nnz_ = int64_t(csr.values.size());
  try {
    row_offsets_ = upload(csr.row_offsets);
    columns_ = upload(csr.columns);
    values_ = upload(csr.values);
    check_rocsparse(rocsparse_create_handle(&handle_), "rocsparse_create_handle");
    check_rocsparse(rocsparse_create_csr_descr(&matrix_, rows_, cols_, nnz_, row_offsets_, columns_, values_,
                                               rocsparse_indextype_i32, rocsparse_indextype_i32,
                                               rocsparse_index_base_zero, rocsparse_datatype_f32_r),
                    "rocsparse_create_csr_descr");
  } catch (...) {
    release();
    throw;
  }
}

void CsrPlan::release() noexcept {
  if (input_) (void)rocsparse_destroy_dnmat_descr(input_);
  if (output_) (void)rocsparse_destroy_dnmat_descr(output_);
  if (matrix_) (void)rocsparse_destroy_spmat_descr(matrix_);
  if (handle_) (void)rocsparse_destroy_handle(handle_);
  (void)hipFree(workspace_);
  (void)hipFree(row_offsets_);
  (void)hipFree(columns_);
  (void)hipFree(values_);
  input_ = output_ = nullptr;
  matrix_ = nullptr;
  handle_ = nullptr;
  workspace_ = nullptr;
  row_offsets_ = columns_ = nullptr;
  values_ = nullptr;
}

CsrPlan::~CsrPlan() { release(); }

void CsrPlan::execute(const float* b, float* c, hipStream_t stream) {
  check_panels(rows_, cols_, b, c, rhs_);
  check_rocsparse(rocsparse_set_stream(handle_, stream), "rocsparse_set_stream");
  const float one = 1.0f, zero = 0.0f;
  auto spmm = [&](rocsparse_spmm_stage stage, size_t* bytes, void* buffer) {
    check_rocsparse(rocsparse_spmm(handle_, rocsparse_operation_none, rocsparse_operation_none, &one, matrix_, input_,
                                   &zero, output_, rocsparse_datatype_f32_r, rocsparse_spmm_alg_default, stage,
                                   bytes, buffer),
                    "rocsparse_spmm");
  };
  if (input_ == nullptr) {
    check_rocsparse(rocsparse_create_dnmat_descr(&input_, cols_, rhs_, cols_, const_cast<float*>(b),
                                                 rocsparse_datatype_f32_r, rocsparse_order_column),
                    "rocsparse_create_dnmat_descr");
    check_rocsparse(rocsparse_create_dnmat_descr(&output_, rows_, rhs_, rows_, c, rocsparse_datatype_f32_r,
                                                 rocsparse_order_column),
                    "rocsparse_create_dnmat_descr");
    size_t bytes = 0;
    spmm(rocsparse_spmm_stage_buffer_size, &bytes, nullptr);
    if (bytes > 0) check_hip(hipMalloc(&workspace_, bytes), "hipMalloc workspace");
    workspace_bytes_ = bytes;
    spmm(rocsparse_spmm_stage_preprocess, &bytes, workspace_);
  } else {
    check_rocsparse(rocsparse_dnmat_set_values(input_, const_cast<float*>(b)), "rocsparse_dnmat_set_values");
    check_rocsparse(rocsparse_dnmat_set_values(output_, c), "rocsparse_dnmat_set_values");
  }
  size_t bytes = workspace_bytes_;
  spmm(rocsparse_spmm_stage_compute, &bytes, workspace_);
}

}  // namespace vbsr_amd
