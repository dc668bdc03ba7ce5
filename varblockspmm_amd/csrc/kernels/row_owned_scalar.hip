// Order-preserving row-owned kernel: the counterpart of the reference's
// launch_row_owned_scalar (src/kernels/row_owned.cu:11-45, 312-318, 376-395).
//
// Every output C[r, n] is one fmaf chain: acc = 0, then for each block of the
// row in row_ptr order and k ascending, acc = fmaf(A[r, k], B[k, n], acc).
// That is the order every reference kernel uses, so this kernel's results
// are bit-identical to the reference's.  It is the GPU-side order oracle and
// the profiling baseline, not the fast path.
//
// Mapping: one workgroup (256 lanes = 4 waves) per block row; lanes stride
// over the row's h x rhs outputs with the local row fastest, so a wave's A
// loads for one k are consecutive floats of one block column.
#include <hip/hip_runtime.h>

#include "../internal.hpp"

namespace vbsr_amd {
namespace {

constexpr int kScalarThreads = 256;

template <int RHS>
__global__ __launch_bounds__(kScalarThreads) void row_owned_scalar_kernel(vbsr_device_view a,
                                                                          const float* __restrict__ b,
                                                                          float* __restrict__ c) {
  const int row = blockIdx.x;
  const int h = a.row_size[row];
  const int first = a.row_ptr[row];
  const int last = a.row_ptr[row + 1];
  const int64_t out_base = a.row_scalar_off[row];

  for (int item = threadIdx.x; item < h * RHS; item += kScalarThreads) {
    const int r = item % h;
    const int n = item / h;
    float acc = 0.0f;
    for (int blk = first; blk < last; ++blk) {
      const int col = a.block_col[blk];
      const int w = a.col_size[col];
      const float* a_col = a.values + a.value_off[blk] + r;
      const float* b_col = b + a.col_scalar_off[col] + int64_t(n) * a.scalar_cols;
      for (int k = 0; k < w; ++k) acc = __builtin_fmaf(a_col[int64_t(k) * h], b_col[k], acc);
    }
    c[out_base + r + int64_t(n) * a.scalar_rows] = acc;
  }
}

template <int RHS>
void launch(const vbsr_device_view& a, const float* b, float* c, hipStream_t stream) {
  row_owned_scalar_kernel<RHS><<<dim3(unsigned(a.block_rows)), dim3(kScalarThreads), 0, stream>>>(a, b, c);
}

}  // namespace

void launch_scalar(const vbsr_device_view& a, const float* b, float* c, int rhs, hipStream_t stream) {
  if (!supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
  check_panels(a, b, c, rhs);
  if (a.block_rows <= 0) return;
  switch (rhs) {
  case 8: launch<8>(a, b, c, stream); break;
  case 16: launch<16>(a, b, c, stream); break;
  case 32: launch<32>(a, b, c, stream); break;
  default: launch<64>(a, b, c, stream); break;
  }
  check_hip(hipGetLastError(), "row_owned_scalar launch");
}

}  // namespace vbsr_amd
