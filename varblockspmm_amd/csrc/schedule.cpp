// Row schedule: the plan-private metadata of the row-owned kernel, built once
// per matrix.  It replaces the reference's row_shape_order partition
// (src/format/vbsr.cpp:96-102) and its two-launch height split
// (src/kernels/row_owned.cu:333-358) with a single-launch layout derived from
// the MI355X execution model:
//
//  * one record per k step (16 columns of a block, or the 8 that end a block
//    of width 8 mod 16) holds where the step's A columns and B rows start, so
//    the kernel never walks block metadata: a wave loads the records of all
//    its steps of a row with one load;
//  * one workgroup owns one block row;
//  * workgroups are dispatched to the 8 XCDs round-robin by index, so the
//    block rows are cut into 8 contiguous bands and band x is placed at
//    indices x, x + 8, x + 16, ...: each XCD works through one band, and the
//    B slices of a band stay in that XCD's L2 when columns are local;
//  * within a band, heavier rows are dispatched first, so the light ones fill
//    the tail of the launch.
#include <algorithm>
#include <numeric>

#include "internal.hpp"

namespace vbsr_amd {

HostSchedule build_schedule(const vbsr_host_view& m) {
  HostSchedule out;
  const int32_t rows = m.block_rows;
  std::vector<int32_t> step_first(static_cast<size_t>(rows) + 1, 0);
  for (int32_t i = 0; i < rows; ++i) {
    const int32_t h = m.row_size[i];
    for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) {
      const int32_t col = m.block_col[blk];
      const int32_t w = m.col_size[col];
      for (int32_t k0 = 0; k0 < w; k0 += (w - k0 == 8) ? 8 : 16) {
        StepRec step{};
        step.a_off = m.value_off[blk] + int64_t(k0) * h;
        step.b_off = (m.col_scalar_off[col] + k0) | ((w - k0 == 8) ? kHalfStep : 0);
        out.steps.push_back(step);
      }
    }
    if (out.steps.size() > size_t(INT32_MAX)) throw std::invalid_argument("too many k steps for one matrix");
    step_first[size_t(i) + 1] = int32_t(out.steps.size());
  }

  // Cost of a row: its 16-row tiles times its k steps, plus a fixed per-row
  // overhead (in units of one 16 x 16 x 16 MFMA step).
  std::vector<int64_t> work(static_cast<size_t>(rows));
  for (int32_t i = 0; i < rows; ++i)
    work[size_t(i)] = int64_t((m.row_size[i] + 15) / 16) * (step_first[size_t(i) + 1] - step_first[size_t(i)]) + 8;

  const int64_t per_xcd = (int64_t(rows) + kXcds - 1) / kXcds;
  out.groups = per_xcd * kXcds;
  RowItem padding{};
  padding.step_count = -1;
  padding.row = -1;
  out.rows.assign(size_t(out.groups), padding);
  std::vector<int32_t> band;
  for (int xcd = 0; xcd < kXcds; ++xcd) {
    const int64_t lo = std::min<int64_t>(rows, xcd * per_xcd);
    const int64_t hi = std::min<int64_t>(rows, lo + per_xcd);
    band.resize(size_t(hi - lo));
    std::iota(band.begin(), band.end(), int32_t(lo));
    std::stable_sort(band.begin(), band.end(),
                     [&](int32_t x, int32_t y) { return work[size_t(x)] > work[size_t(y)]; });
    for (int64_t pos = 0; pos < hi - lo; ++pos) {
      const int32_t i = band[size_t(pos)];
      RowItem& item = out.rows[size_t(pos * kXcds + xcd)];
      item.c_off = m.row_scalar_off[i];
      item.step_first = step_first[size_t(i)];
      item.step_count = step_first[size_t(i) + 1] - step_first[size_t(i)];
      item.h = m.row_size[i];
      item.row = i;
    }
  }
  return out;
}

}  // namespace vbsr_amd
