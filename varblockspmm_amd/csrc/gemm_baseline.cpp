// GroupedGemmPlan: the counterpart of the reference's slot-grouped cuBLAS
// baseline (src/baseline/slot_split.cu:22-145, declared at
// include/varblockspmm/vbsr.hpp:138-152), on rocBLAS.
//
// Slot s holds the s-th block of every block row that has one; within a
// slot, blocks are grouped by (h, w) (slot_split.cu:72-95).  Execute zeroes
// C, then runs the slots in order: each group is one rocblas_sgemm_batched
// call, C_i = A_b * B_c (+ C_i after the first slot), with A h x w (ld h),
// B's w x rhs slice (ld K) and C's h x rhs slab (ld M).  Blocks of one slot
// come from distinct rows, so the GEMMs of a slot never write the same C.
// rocBLAS has no grouped-batched GEMM, so a slot takes one call per (h, w)
// group instead of the reference's one grouped call.  The A pointers are
// made once; the B and C pointers of each call are written on the device
// (batch_pointers.hip).  Not thread-safe, like the reference's.
#include <algorithm>
#include <map>

#include <hip/hip_runtime_api.h>
#include <rocblas/rocblas.h>

#include "internal.hpp"

namespace vbsr_amd {
namespace {

void check_rocblas(rocblas_status status, const char* what) {
  if (status != rocblas_status_success)
    throw std::runtime_error(std::string("rocBLAS failure in ") + what + ": " + std::to_string(int(status)));
}

template <class T>
T* upload(const T* source, size_t count) {
  T* destination = nullptr;
  check_hip(hipMalloc(reinterpret_cast<void**>(&destination), std::max<size_t>(count, 1) * sizeof(T)), "hipMalloc");
  if (count > 0) {
    const hipError_t status = hipMemcpy(destination, source, count * sizeof(T), hipMemcpyHostToDevice);
    if (status != hipSuccess) {
      (void)hipFree(destination);
      check_hip(status, "hipMemcpy");
    }
  }
  return destination;
}

template <class T>
T* upload(const std::vector<T>& source) {
  return upload(source.data(), source.size());
}

}  // namespace

GemmPlan::GemmPlan(const vbsr_host_view& host, int rhs) : rhs_(rhs) {
  validate(host);
  if (!supported_rhs(rhs)) throw std::invalid_argument("rhs_width must be 8,16,32,64");
  if (host.row_scalar_off[0] != 0 || host.col_scalar_off[0] != 0)
    throw std::invalid_argument("scalar offsets must start at 0");
  rows_ = host.row_scalar_off[host.block_rows];
  cols_ = host.col_scalar_off[host.block_cols];
  if (rows_ > int64_t(INT32_MAX) || cols_ > int64_t(INT32_MAX))
    throw std::invalid_argument("rocBLAS leading dimensions must fit in 32 bits");

  int32_t max_degree = 0;
  for (int32_t i = 0; i < host.block_rows; ++i) max_degree = std::max(max_degree, host.row_ptr[i + 1] - host.row_ptr[i]);
  std::vector<int64_t> a_offset, b_offset, c_offset;
  for (int32_t slot = 0; slot < max_degree; ++slot) {
    std::map<std::pair<int32_t, int32_t>, std::vector<int32_t>> groups;  // (h, w) -> block indices, rows ascending
    for (int32_t i = 0; i < host.block_rows; ++i) {
      const int32_t blk = host.row_ptr[i] + slot;
      if (blk < host.row_ptr[i + 1]) groups[{host.row_size[i], host.col_size[host.block_col[blk]]}].push_back(i);
    }
    std::vector<Group> slot_groups;
    for (const auto& [shape, members] : groups) {
      Group g{};
      g.h = shape.first;
      g.w = shape.second;
      g.first = int64_t(a_offset.size());
      g.count = int32_t(members.size());
      for (const int32_t i : members) {
        const int32_t blk = host.row_ptr[i] + slot;
        a_offset.push_back(host.value_off[blk]);
        b_offset.push_back(host.col_scalar_off[host.block_col[blk]]);
        c_offset.push_back(host.row_scalar_off[i]);
      }
      slot_groups.push_back(g);
    }
    slots_.push_back(std::move(slot_groups));
  }
  entries_ = int64_t(a_offset.size());

  try {
    values_ = upload(host.values, size_t(host.values_len));
    std::vector<const float*> a_pointers(a_offset.size());
    for (size_t e = 0; e < a_offset.size(); ++e) a_pointers[e] = values_ + a_offset[e];
    a_pointers_ = upload(a_pointers);
    b_offset_ = upload(b_offset);
    c_offset_ = upload(c_offset);
    check_hip(hipMalloc(reinterpret_cast<void**>(&b_pointers_), std::max<size_t>(a_offset.size(), 1) * sizeof(float*)),
              "hipMalloc");
    check_hip(hipMalloc(reinterpret_cast<void**>(&c_pointers_), std::max<size_t>(a_offset.size(), 1) * sizeof(float*)),
              "hipMalloc");
    check_rocblas(rocblas_create_handle(&handle_), "rocblas_create_handle");
    check_rocblas(rocblas_set_pointer_mode(handle_, rocblas_pointer_mode_host), "rocblas_set_pointer_mode");
  } catch (...) {
    release();
    throw;
  }
}

void GemmPlan::release() noexcept {
  if (handle_) (void)rocblas_destroy_handle(handle_);
  handle_ = nullptr;
  for (void* p : {static_cast<void*>(values_), static_cast<void*>(a_pointers_), static_cast<void*>(b_offset_),
                  static_cast<void*>(c_offset_), static_cast<void*>(b_pointers_), static_cast<void*>(c_pointers_)})
    (void)hipFree(p);
  values_ = nullptr;
  a_pointers_ = nullptr;
  b_offset_ = c_offset_ = nullptr;
  b_pointers_ = nullptr;
  c_pointers_ = nullptr;
}

GemmPlan::~GemmPlan() { release(); }

void GemmPlan::execute(const float* b, float* c, hipStream_t stream) {
  check_panels(rows_, cols_, b, c, rhs_);
  check_rocblas(rocblas_set_stream(handle_, stream), "rocblas_set_stream");
  check_hip(hipMemsetAsync(c, 0, size_t(rows_) * size_t(rhs_) * sizeof(float), stream), "hipMemsetAsync");
  fill_batch_pointers(b_offset_, c_offset_, entries_, b, c, b_pointers_, c_pointers_, stream);
  const float one = 1.0f, zero = 0.0f;
  for (size_t slot = 0; slot < slots_.size(); ++slot) {
    for (const Group& g : slots_[slot]) {
      check_rocblas(rocblas_sgemm_batched(handle_, rocblas_operation_none, rocblas_operation_none, g.h, rhs_, g.w, &one,
                                          a_pointers_ + g.first, g.h, b_pointers_ + g.first, rocblas_int(cols_),
                                          slot == 0 ? &zero : &one, c_pointers_ + g.first, rocblas_int(rows_),
                                          g.count),
                    "rocblas_sgemm_batched");
    }
  }
}

}  // namespace vbsr_amd
