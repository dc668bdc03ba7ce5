// Plan: the counterpart of the reference Plan (src/plan/plan.cpp:5-31).
//
// The reference splits RHS-32 rows at h <= 16 into two CUDA launches and
// picks a different CUDA kernel per width (row_owned.cu:333-358, 397-423).
// On MI355X every width runs one launch of the row-owned MFMA kernel: a
// workgroup owns a block row, its four waves share the row's k steps and
// reduce their partial tiles in LDS, so the row height no longer decides the
// kernel and the height split has no counterpart.  The matrix's row schedule
// (schedule.cpp) orders and places the rows instead.
//
// Matrices with more scalar columns than the MFMA kernel's 32-bit B offsets
// reach (K > 153,391,684 at RHS 8, K > 71,582,785 otherwise) go to the
// order-preserving kernel, which has no such limit.  Any float-aligned B and C panels stay on the MFMA kernel.
#include "internal.hpp"

namespace vbsr_amd {

Plan::Plan(const DeviceMatrix& matrix, const vbsr_plan_options& o)
    : a(matrix.view()), schedule(matrix.schedule()), options(o) {
  if (!supported_rhs(o.rhs_width)) throw std::invalid_argument("rhs_width must be 8,16,32,64");
  if (o.kernel == VBSR_KERNEL_SPLIT_ROW)
    throw std::invalid_argument("split-row is reserved and not provided; use RowOwned");
  if (o.kernel != VBSR_KERNEL_AUTO && o.kernel != VBSR_KERNEL_ROW_OWNED)
    throw std::invalid_argument("unknown kernel selection");
}

void Plan::execute(const float* b, float* c, hipStream_t stream) const {
  if (row_owned_supported(a, b, c, options.rhs_width))
    launch_row_owned(a, schedule, b, c, options.rhs_width, stream);
  else
    launch_scalar(a, b, c, options.rhs_width, stream);
}

int Plan::launch_count() const { return schedule.groups > 0 ? 1 : 0; }

}  // namespace vbsr_amd
