// Internal declarations of libvarblockspmm_amd.  The public boundary is the
// C ABI in include/vbsr.h; everything here may throw std::invalid_argument or
// std::runtime_error, which capi.cpp maps to status codes.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "vbsr.h"

namespace vbsr_amd {

// Throws std::runtime_error carrying the HIP error string on failure.
void check_hip(hipError_t status, const char* what);

// ---- host format (host_format.cpp) --------------------------------------

// HostMatrix::validate (vbsr.cpp:29-82): same checks, same order.
void validate(const vbsr_host_view& host);

// Owning host matrix with the reference HostMatrix fields (vbsr.hpp:16-29).
struct HostMatrix {
  int32_t block_rows{}, block_cols{};
  std::vector<int32_t> row_ptr, block_col, row_size, col_size;
  std::vector<int64_t> row_scalar_off, col_scalar_off, value_off;
  std::vector<float> values;
  vbsr_host_view view() const;
};

// generate (generator.cpp:7-88) plus the extension distributions/localities.
HostMatrix generate(const vbsr_generator_options& options);

// make_random_input (tests/test_main.cpp:42-51).
void make_random_input(int64_t count, uint64_t seed, float* out);

// ---- device format (device_matrix.cpp) ----------------------------------

// Matrix (vbsr.hpp:41-64): owns device copies of every array plus the row
// schedule.  Immutable after construction.
class DeviceMatrix {
public:
  explicit DeviceMatrix(const vbsr_host_view& host);
  ~DeviceMatrix();
  DeviceMatrix(const DeviceMatrix&) = delete;
  DeviceMatrix& operator=(const DeviceMatrix&) = delete;

  const vbsr_device_view& view() const { return view_; }
  const int32_t* row_order() const { return row_order_; }

private:
  vbsr_device_view view_{};
  int32_t* row_order_{};
  std::vector<void*> allocations_;
  void release() noexcept;
};

// Host-side construction of the row schedule: block rows sorted by decreasing
// estimated work (ties keep ascending row index).
std::vector<int32_t> build_row_schedule(const vbsr_host_view& host);

// ---- kernels -------------------------------------------------------------

// True for the RHS widths the reference supports (plan.cpp:9-12).
inline bool supported_rhs(int rhs) { return rhs == 8 || rhs == 16 || rhs == 32 || rhs == 64; }

// Order-preserving kernel (row_owned_scalar.hip).
void launch_scalar(const vbsr_device_view& a, const float* b, float* c, int rhs, hipStream_t stream);

// MFMA row-owned kernels (row_owned_mfma.hip).  Launch count: 1.
void launch_mfma(const vbsr_device_view& a, const int32_t* row_order, const float* b, float* c,
                 int rhs, hipStream_t stream);

// ---- plan (plan.cpp) -------------------------------------------------------

struct Plan {
  vbsr_device_view a{};
  const int32_t* row_order{};
  vbsr_plan_options options{};
  Plan(const DeviceMatrix& matrix, const vbsr_plan_options& options);
  void execute(const float* b, float* c, hipStream_t stream) const;
  int launch_count() const;
};

}  // namespace vbsr_amd
