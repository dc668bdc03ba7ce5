// cpu_reference (reference include/varblockspmm/vbsr.hpp:82-87,
// src/format/vbsr.cpp:167-201): C = A * B on the host, single-threaded, as
// the reference library exports it for its callers' checks.
//
// Arithmetic, which fixes every output bit: each block contributes, to each
// (local row r, rhs column n), one double sum of double(A[r, k]) * B[k, n]
// over k ascending from 0, rounded once to float and added to C in FP32;
// blocks are added in row_ptr order and C starts at zero.  Products of two
// floats are exact in double, so contraction into fused multiply-adds cannot
// change a sum either.
//
// The loop runs the k sums of all h rows of a block side by side (one double
// accumulator per row) so that A is read in its stored order; each row's sum
// still takes its terms in k order.
#include <array>

#include "internal.hpp"

namespace vbsr_amd {

void cpu_reference(const vbsr_host_view& m, const float* b, int64_t b_len, int rhs, float* c, int64_t c_len) {
  validate(m);
  if (m.row_scalar_off[0] < 0 || m.col_scalar_off[0] < 0)
    throw std::invalid_argument("scalar offsets must not be negative");
  if (rhs < 0) throw std::invalid_argument("B size");
  const int64_t rows = m.row_scalar_off[m.row_scalar_off_len - 1];
  const int64_t cols = m.col_scalar_off[m.col_scalar_off_len - 1];
  int64_t b_size = 0, c_size = 0;
  if (__builtin_mul_overflow(cols, int64_t(rhs), &b_size) || b_len != b_size) throw std::invalid_argument("B size");
  if (__builtin_mul_overflow(rows, int64_t(rhs), &c_size) || c_len != c_size) throw std::invalid_argument("C size");
  if ((b_len > 0 && b == nullptr) || (c_len > 0 && c == nullptr)) throw std::invalid_argument("null B or C");

  for (int64_t i = 0; i < c_len; ++i) c[i] = 0.0f;
  std::array<double, 64> sum{};
  for (int32_t i = 0; i < m.block_rows; ++i) {
    const int32_t h = m.row_size[i];
    float* c_rows = c + m.row_scalar_off[i];
    for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) {
      const int32_t col = m.block_col[blk];
      const int32_t w = m.col_size[col];
      const float* a = m.values + m.value_off[blk];
      const float* b_rows = b + m.col_scalar_off[col];
      for (int n = 0; n < rhs; ++n) {
        const float* bn = b_rows + int64_t(n) * cols;
        for (int32_t r = 0; r < h; ++r) sum[size_t(r)] = 0.0;
        for (int32_t k = 0; k < w; ++k) {
          const double bk = double(bn[k]);
          const float* ak = a + int64_t(k) * h;
          for (int32_t r = 0; r < h; ++r) sum[size_t(r)] += double(ak[r]) * bk;
        }
        float* cn = c_rows + int64_t(n) * rows;
        for (int32_t r = 0; r < h; ++r) cn[r] += float(sum[size_t(r)]);
      }
    }
  }
}

}  // namespace vbsr_amd
