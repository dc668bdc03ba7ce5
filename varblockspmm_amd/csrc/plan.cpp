// Plan: the counterpart of the reference Plan (src/plan/plan.cpp:5-31).
//
// The reference splits RHS-32 rows at h <= 16 into two CUDA launches and
// picks a different CUDA kernel per width (row_owned.cu:333-358, 397-423).
// On MI355X every width runs one launch of the row-owned MFMA kernel: a
// workgroup owns a block row (or four light ones, one per wave), its waves
// share the row's k steps and reduce their partial tiles in LDS, so the row
// height no longer decides the kernel and the height split has no
// counterpart.  The matrix's row schedule (schedule.cpp) orders and places
// the rows instead.
//
// Kernel::Auto and Kernel::RowOwned both run the row-owned kernel, as in the
// reference (docs/design.md:15,17): the plan views the matrix, owns nothing,
// and its executes may run concurrently on any streams.
//
// Kernel::SplitRow, reserved in the reference (plan.cpp:13-17), is the
// split-row path here, taken only on request: each row's k steps are cut
// into parts computed by the same kernel into a plan-owned workspace, and a
// second launch sums each row's parts in a fixed order.  Such a plan's
// executes share that workspace.  The matrix reports whether the split pays
// for a given width (vbsr_matrix_split_row_advised); the plan never switches
// by itself.
//
// Every K stays on the MFMA kernel: past the reach of its 32-bit B offsets
// (K > 153,391,684 at RHS 8, K > 71,582,785 otherwise) it addresses B with
// 64-bit lane pointers instead.
#include <hip/hip_runtime_api.h>

#include "internal.hpp"

namespace vbsr_amd {

Plan::Plan(const DeviceMatrix& matrix, const vbsr_plan_options& o)
    : a_(matrix.view()), schedule_(matrix.schedule()), split_(matrix.split()), options_(o) {
  if (!supported_rhs(o.rhs_width)) throw std::invalid_argument("rhs_width must be 8,16,32,64");
  if (o.kernel != VBSR_KERNEL_AUTO && o.kernel != VBSR_KERNEL_ROW_OWNED && o.kernel != VBSR_KERNEL_SPLIT_ROW)
    throw std::invalid_argument("unknown kernel selection");
  split_row_ = o.kernel == VBSR_KERNEL_SPLIT_ROW;
  if (split_row_) {
    workspace_floats_ = split_workspace_floats(split_, o.rhs_width);
    if (workspace_floats_ > 0)
      check_hip(hipMalloc(reinterpret_cast<void**>(&workspace_), size_t(workspace_floats_) * sizeof(float)),
                "hipMalloc (split-row workspace)");
  }
}

Plan::~Plan() {
  if (workspace_ != nullptr) (void)hipFree(workspace_);
}

void Plan::execute(const float* b, float* c, hipStream_t stream) const {
  if (split_row_)
    launch_split_row(a_, schedule_, split_, b, c, options_.rhs_width, workspace_, workspace_floats_, stream);
  else
    launch_row_owned(a_, schedule_, b, c, options_.rhs_width, stream);
}

int Plan::launch_count() const {
  if (a_.block_rows <= 0) return 0;
  if (split_row_) return 2;
  return schedule_.groups > 0 ? 1 : 0;
}

}  // namespace vbsr_amd
