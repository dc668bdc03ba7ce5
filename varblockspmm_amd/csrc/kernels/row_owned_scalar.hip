// Order-preserving row-owned kernel: the counterpart of the reference's
// launch_row_owned_scalar (src/kernels/row_owned.cu:11-45, 312-318, 376-395).
//
// Every output C[r, n] is one fmaf chain: acc = 0, then for each block of the
// row in row_ptr order and k ascending, acc = fmaf(A[r, k], B[k, n], acc).
// That is the order every reference kernel uses, so this kernel's results
// are bit-identical to the reference's.  It is the GPU-side order oracle and
// the profiling baseline, not the fast path.
//
// Mapping: one workgroup per block row.  Lane (r, g) owns local row r and
// the adjacent output columns of group g: 4 groups of RHS/4 columns (256
// lanes), or 8 groups of 8 at RHS 64 (512 lanes), so gh lanes cover the row
// in one pass and each A value a lane loads feeds RHS/groups fmaf chains.
// Each block's B slice (w x RHS floats) is staged once per workgroup in LDS,
// double-buffered with one barrier per block, stored k-major with a padded
// row (RHS + 4 floats) so a lane's columns are one 8- to 64-byte read.
#include <hip/hip_runtime.h>

#include "../internal.hpp"

namespace vbsr_amd {
namespace {

constexpr int kMaxBlockDim = 64;  // largest block height and width

// Column groups per local row, and the workgroup that covers 64 rows of them.
template <int RHS>
constexpr int scalar_groups() {
  return RHS >= 32 ? 8 : 4;
}
template <int RHS>
constexpr int scalar_threads() {
  return scalar_groups<RHS>() * kMaxBlockDim;
}

template <int RHS>
__global__ __launch_bounds__(scalar_threads<RHS>()) void row_owned_scalar_kernel(vbsr_device_view a,
                                                                          const float* __restrict__ b,
                                                                          float* __restrict__ c) {
  constexpr int kGroups = scalar_groups<RHS>();
  constexpr int kThreads = scalar_threads<RHS>();
  constexpr int kCols = RHS / kGroups;  // output columns per lane
  constexpr int kLd = RHS + 4;          // LDS row of one k of a B slice
  __shared__ __attribute__((aligned(16))) float slice[2][kMaxBlockDim * kLd];

  const int row = blockIdx.x;
  const int tid = int(threadIdx.x);
  const int h = a.row_size[row];
  const int first = a.row_ptr[row];
  const int last = a.row_ptr[row + 1];
  const int r = tid % h;
  const int g = tid / h;
  const bool owner = g < kGroups;  // kGroups * h lanes own outputs; the rest only stage B

  // Stages block blk's B slice: B[col0 + k, n] for k < w, n < RHS at k * kLd + n.
  auto stage = [&](int blk, float* dst) {
    const int col = a.block_col[blk];
    const int w = a.col_size[col];
    const float* src = b + a.col_scalar_off[col];
    const int k = tid % kMaxBlockDim;
    if (k < w)
      for (int n = tid / kMaxBlockDim; n < RHS; n += kThreads / kMaxBlockDim)
        dst[k * kLd + n] = src[k + int64_t(n) * a.scalar_cols];
  };

  float acc[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc[j] = 0.0f;

  if (first < last) stage(first, slice[0]);
  __syncthreads();
  for (int blk = first; blk < last; ++blk) {
    const int buf = (blk - first) & 1;
    if (blk + 1 < last) stage(blk + 1, slice[buf ^ 1]);
    if (owner) {
      const int w = a.col_size[a.block_col[blk]];
      const float* a_col = a.values + a.value_off[blk] + r;
      const float* bs = slice[buf] + g * kCols;
      // w is a multiple of 8: eight A loads in flight, then their fmafs in
      // k order.
      for (int k0 = 0; k0 < w; k0 += 8) {
        float av[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) av[i] = a_col[int64_t(k0 + i) * h];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float* bk = bs + (k0 + i) * kLd;
#pragma unroll
          for (int j = 0; j < kCols; ++j) acc[j] = __builtin_fmaf(av[i], bk[j], acc[j]);
        }
      }
    }
    __syncthreads();
  }
  if (owner) {
    float* c_row = c + a.row_scalar_off[row] + r;
#pragma unroll
    for (int j = 0; j < kCols; ++j) c_row[int64_t(g * kCols + j) * a.scalar_rows] = acc[j];
  }
}

template <int RHS>
void launch(const vbsr_device_view& a, const float* b, float* c, hipStream_t stream) {
  row_owned_scalar_kernel<RHS><<<dim3(unsigned(a.block_rows)), dim3(scalar_threads<RHS>()), 0, stream>>>(a, b, c);
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
