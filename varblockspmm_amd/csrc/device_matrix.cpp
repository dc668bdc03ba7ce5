// Owning device format: the counterpart of the reference Matrix
// (src/format/vbsr.cpp:84-166).  Arrays are copied verbatim (same packed
// column-major block payload, same 64-bit scalar/value offsets), so the
// device view has exactly the reference DeviceMatrix semantics.  The only
// plan-private array is the row schedule.
#include <algorithm>
#include <numeric>

#include <hip/hip_runtime_api.h>

#include "internal.hpp"

namespace vbsr_amd {

void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

std::vector<int32_t> build_row_schedule(const vbsr_host_view& m) {
  // Work of a block row in the MFMA kernels is proportional to its number of
  // 16-row tiles times its total block width; heavy rows go first so that the
  // hardware dispatcher packs the light ones into the tail.
  std::vector<int64_t> work(size_t(m.block_rows), 0);
  for (int32_t i = 0; i < m.block_rows; ++i) {
    int64_t width = 0;
    for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) width += m.col_size[m.block_col[blk]];
    work[size_t(i)] = int64_t((m.row_size[i] + 15) / 16) * (width + 16);
  }
  std::vector<int32_t> order(size_t(m.block_rows));
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(),
                   [&](int32_t x, int32_t y) { return work[size_t(x)] > work[size_t(y)]; });
  return order;
}

namespace {

template <class T>
T* upload(const T* source, int64_t count, std::vector<void*>& owned) {
  T* destination = nullptr;
  // A zero-length array still gets a (tiny) allocation so that every view
  // pointer is a valid device pointer.
  const size_t bytes = size_t(std::max<int64_t>(count, 1)) * sizeof(T);
  check_hip(hipMalloc(reinterpret_cast<void**>(&destination), bytes), "hipMalloc");
  owned.push_back(destination);
  if (count > 0)
    check_hip(hipMemcpy(destination, source, size_t(count) * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
  return destination;
}

}  // namespace

DeviceMatrix::DeviceMatrix(const vbsr_host_view& host) {
  validate(host);
  // Stricter than the reference: offsets must start at 0 so that every row
  // of C is written and every access stays inside B and C.
  if (host.row_scalar_off[0] != 0 || host.col_scalar_off[0] != 0)
    throw std::invalid_argument("scalar offsets must start at 0");

  const std::vector<int32_t> order = build_row_schedule(host);
  try {
    view_.block_rows = host.block_rows;
    view_.block_cols = host.block_cols;
    view_.nnzb = int32_t(host.block_col_len);
    view_.scalar_rows = host.row_scalar_off[host.block_rows];
    view_.scalar_cols = host.col_scalar_off[host.block_cols];
    view_.row_ptr = upload(host.row_ptr, host.row_ptr_len, allocations_);
    view_.block_col = upload(host.block_col, host.block_col_len, allocations_);
    view_.row_size = upload(host.row_size, host.row_size_len, allocations_);
    view_.col_size = upload(host.col_size, host.col_size_len, allocations_);
    view_.row_scalar_off = upload(host.row_scalar_off, host.row_scalar_off_len, allocations_);
    view_.col_scalar_off = upload(host.col_scalar_off, host.col_scalar_off_len, allocations_);
    view_.value_off = upload(host.value_off, host.value_off_len, allocations_);
    view_.values = upload(host.values, host.values_len, allocations_);
    row_order_ = upload(order.data(), int64_t(order.size()), allocations_);
  } catch (...) {
    release();
    throw;
  }
}

void DeviceMatrix::release() noexcept {
  for (void* p : allocations_) (void)hipFree(p);
  allocations_.clear();
  view_ = vbsr_device_view{};
  row_order_ = nullptr;
}

DeviceMatrix::~DeviceMatrix() { release(); }

}  // namespace vbsr_amd
