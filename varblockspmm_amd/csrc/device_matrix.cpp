// Owning device format: the counterpart of the reference Matrix
// (src/format/vbsr.cpp:84-166).  Arrays are copied verbatim (same packed
// column-major block payload, same 64-bit scalar/value offsets), so the
// device view has exactly the reference DeviceMatrix semantics.  The only
// plan-private arrays are the row schedule and the split-row schedule
// (schedule.cpp).
#include <algorithm>

#include <hip/hip_runtime_api.h>

#include "internal.hpp"

namespace vbsr_amd {

void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
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

  const HostSchedule schedule = build_schedule(host);
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
    schedule_.steps = upload(schedule.steps.data(), int64_t(schedule.steps.size()), allocations_);
    schedule_.rows = upload(schedule.rows.data(), int64_t(schedule.rows.size()), allocations_);
    schedule_.rows_wide = upload(schedule.rows_wide.data(), int64_t(schedule.rows_wide.size()), allocations_);
    schedule_.groups = schedule.groups;
    schedule_.rows_rhs64 = upload(schedule.rows_rhs64.data(), int64_t(schedule.rows_rhs64.size()), allocations_);
    schedule_.groups_rhs64 = schedule.groups_rhs64;
    schedule_.rows_tile = upload(schedule.rows_tile.data(), int64_t(schedule.rows_tile.size()), allocations_);
    schedule_.groups_tile = schedule.groups_tile;
    schedule_.rhs64_tiles = schedule.rhs64_tiles ? 1 : 0;
    schedule_.step_limit = int32_t(std::max<size_t>(schedule.steps.size(), 1) - 1);
    split_.items = upload(schedule.split.items.data(), int64_t(schedule.split.items.size()), allocations_);
    split_.rows = upload(schedule.split.rows.data(), int64_t(schedule.split.rows.size()), allocations_);
    split_.groups = schedule.split.groups;
    split_.virtual_rows = schedule.split.virtual_rows;
    split_.preferred = schedule.split_preferred;
  } catch (...) {
    release();
    throw;
  }
}

void DeviceMatrix::release() noexcept {
  for (void* p : allocations_) (void)hipFree(p);
  allocations_.clear();
  view_ = vbsr_device_view{};
  schedule_ = vbsr_row_schedule{};
  split_ = Split{};
}

DeviceMatrix::~DeviceMatrix() { release(); }

}  // namespace vbsr_amd
