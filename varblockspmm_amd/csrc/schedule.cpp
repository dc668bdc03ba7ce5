// Row schedule: the plan-private metadata of the row-owned kernel, built once
// per matrix.  It replaces the reference's row_shape_order partition
// (src/format/vbsr.cpp:96-102) and its two-launch height split
// (src/kernels/row_owned.cu:333-358) with a single-launch order derived from
// the MI355X execution model:
//
//  * one workgroup owns one block row, so every row is one unit of work;
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
  const int64_t nnzb = m.block_col_len;
  out.blocks.resize(size_t(nnzb));
  for (int64_t blk = 0; blk < nnzb; ++blk) {
    const int32_t col = m.block_col[blk];
    const int64_t w = m.col_size[col];
    out.blocks[size_t(blk)].a_off = m.value_off[blk];
    out.blocks[size_t(blk)].b_off = m.col_scalar_off[col] | (w << kWidthShift);
  }

  // Cost of a row: its 16-row tiles times its k steps, plus fixed per-block
  // and per-row overheads (all in units of one 16 x 16 x 16 MFMA step).
  const int32_t rows = m.block_rows;
  std::vector<int64_t> work(static_cast<size_t>(rows));
  for (int32_t i = 0; i < rows; ++i) {
    int64_t steps = 0;
    for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) steps += (m.col_size[m.block_col[blk]] + 8) / 16;
    const int64_t tiles = (m.row_size[i] + 15) / 16;
    work[size_t(i)] = tiles * steps + (m.row_ptr[i + 1] - m.row_ptr[i]) + 8;
  }

  const int64_t per_xcd = (int64_t(rows) + kXcds - 1) / kXcds;
  out.groups = per_xcd * kXcds;
  RowItem padding{};
  padding.nblocks = -1;
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
      item.first = m.row_ptr[i];
      item.nblocks = m.row_ptr[i + 1] - m.row_ptr[i];
      item.h = m.row_size[i];
      item.row = i;
    }
  }
  return out;
}

}  // namespace vbsr_amd
