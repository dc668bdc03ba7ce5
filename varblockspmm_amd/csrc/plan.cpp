// Plan: the counterpart of the reference Plan (src/plan/plan.cpp:5-31).
//
// The reference splits RHS-32 rows at h <= 16 into two CUDA launches and
// picks a different CUDA kernel per width (row_owned.cu:333-358, 397-423).
// On MI355X every width runs one launch of the MFMA row-owned kernel: one
// wave64 owns one block row at a time and covers the row's h x rhs output in
// 16x16 MFMA tiles, so the row-height split has no counterpart; the block
// rows are ordered by decreasing work at Matrix construction instead.
#include "internal.hpp"

namespace vbsr_amd {

Plan::Plan(const DeviceMatrix& matrix, const vbsr_plan_options& o)
    : a(matrix.view()), row_order(matrix.row_order()), options(o) {
  if (!supported_rhs(o.rhs_width)) throw std::invalid_argument("rhs_width must be 8,16,32,64");
  if (o.kernel == VBSR_KERNEL_SPLIT_ROW)
    throw std::invalid_argument("split-row is reserved and not provided; use RowOwned");
  if (o.kernel != VBSR_KERNEL_AUTO && o.kernel != VBSR_KERNEL_ROW_OWNED)
    throw std::invalid_argument("unknown kernel selection");
}

void Plan::execute(const float* b, float* c, hipStream_t stream) const {
  launch_mfma(a, row_order, b, c, options.rhs_width, stream);
}

int Plan::launch_count() const { return a.block_rows > 0 ? 1 : 0; }

}  // namespace vbsr_amd
