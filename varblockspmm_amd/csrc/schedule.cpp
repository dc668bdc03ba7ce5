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
//  * one workgroup owns one block row, or up to four light rows (at most
//    kPackSteps k steps each; kPackStepsRhs64 in the RHS 64 order, whose
//    steps cost twice as much), one per wave, so that rows too short to
//    keep four waves busy do not leave three of them idle;
//  * workgroups are dispatched to the 8 XCDs round-robin by index, so each
//    XCD's rows (its band) are placed at indices x, x + 8, x + 16, ...;
//  * a block row goes to the XCD whose eighth of the block columns holds the
//    largest share of the row's block widths, as long as that XCD holds less
//    than an eighth of the total work (else to its next best eighth): the B
//    slices an XCD reads then concentrate in one eighth of B, which its L2
//    keeps; rows with the most concentrated columns are placed first, and
//    equal work per XCD keeps any XCD from finishing late.  With local
//    columns this gives contiguous bands of rows;
//  * within a band, two launch orders are kept.  For RHS 8 and 16 heavier
//    rows are dispatched first, so the light ones fill the tail of the launch.
//    For RHS 32 and 64, where B is most of the traffic, the workgroups among
//    the heavier three quarters of the band are chained so that each follows
//    the workgroups it shares block columns (or neighbouring block columns,
//    which share B's 128-byte lines) with; the lightest quarter follows,
//    heaviest first.  Chaining cuts the XCD's B line misses; keeping a light
//    tail bounds the imbalance it costs.  It pays only when an XCD runs its
//    workgroups in more than about one and a half rounds of its workgroup
//    slots (128 at RHS 32, 96 at RHS 64), so matrices of at most
//    kChainMinUnits workgroups per XCD (few rows, or degree 1) keep the
//    heaviest-first order at RHS 32 and 64 too.  On RHS 8 and 16, where A
//    dominates, the imbalance always outweighs the saving.
#include <algorithm>
#include <array>
#include <numeric>
#include <queue>

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
  auto steps_of = [&](int32_t i) { return step_first[size_t(i) + 1] - step_first[size_t(i)]; };

  // Cost of a row: its 16-row tiles times its k steps (in units of one
  // 16 x 16 x 16 MFMA step).
  std::vector<int64_t> row_work(static_cast<size_t>(rows));
  for (int32_t i = 0; i < rows; ++i) row_work[size_t(i)] = int64_t((m.row_size[i] + 15) / 16) * steps_of(i);

  // The workgroups of one launch, for rows of at most pack_steps steps
  // packed kRowWaves to a workgroup, in the heaviest-first order (if asked
  // for) and in the wide order; returns the launch's workgroup count.
  auto launch_orders = [&](int32_t pack_steps, std::vector<WaveItem>* heaviest, std::vector<WaveItem>* chained_items,
                           size_t* units_out) -> int64_t {
    // Workgroups ("units"): every row of more than pack_steps steps alone;
    // the light rows, heaviest first, kRowWaves at a time.  A unit's cost is
    // its rows' work plus a fixed per-workgroup overhead.
    std::vector<std::vector<int32_t>> units;
    std::vector<int32_t> light;
    for (int32_t i = 0; i < rows; ++i) {
      if (steps_of(i) > pack_steps)
        units.push_back({i});
      else
        light.push_back(i);
    }
    std::stable_sort(light.begin(), light.end(),
                     [&](int32_t x, int32_t y) { return row_work[size_t(x)] > row_work[size_t(y)]; });
    for (size_t q = 0; q < light.size(); q += kRowWaves)
      units.emplace_back(light.begin() + std::ptrdiff_t(q),
                         light.begin() + std::ptrdiff_t(std::min(light.size(), q + size_t(kRowWaves))));
    const size_t n_units = units.size();
    std::vector<int64_t> work(n_units, 8);
    for (size_t u = 0; u < n_units; ++u)
      for (const int32_t i : units[u]) work[u] += row_work[size_t(i)];

    // Home eighth of each unit: the eighth of the block columns holding the
    // largest share of its rows' block widths.
    const int32_t cols = m.block_cols;
    std::vector<std::array<int64_t, kXcds>> share(n_units);
    for (size_t u = 0; u < n_units; ++u) {
      share[u].fill(0);
      for (const int32_t i : units[u])
        for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) {
          const int32_t c = m.block_col[blk];
          share[u][size_t(std::min<int64_t>(kXcds - 1, int64_t(c) * kXcds / cols))] += m.col_size[c];
        }
    }
    auto top_share = [&](size_t u) { return *std::max_element(share[u].begin(), share[u].end()); };
    std::vector<size_t> order(n_units);
    std::iota(order.begin(), order.end(), size_t(0));
    std::stable_sort(order.begin(), order.end(), [&](size_t x, size_t y) { return top_share(x) > top_share(y); });

    const int64_t total = std::accumulate(work.begin(), work.end(), int64_t(0));
    const int64_t cap = total / kXcds + 1;
    std::array<int64_t, kXcds> load{};
    std::vector<std::vector<size_t>> bands(kXcds);
    for (const size_t u : order) {
      std::array<int, kXcds> rank{};
      std::iota(rank.begin(), rank.end(), 0);
      std::stable_sort(rank.begin(), rank.end(), [&](int x, int y) { return share[u][size_t(x)] > share[u][size_t(y)]; });
      int chosen = -1;
      for (const int x : rank)
        if (load[size_t(x)] + work[u] <= cap) {
          chosen = x;
          break;
        }
      if (chosen < 0) chosen = int(std::min_element(load.begin(), load.end()) - load.begin());
      bands[size_t(chosen)].push_back(u);
      load[size_t(chosen)] += work[u];
    }

    int64_t per_xcd = 0;
    for (auto& band : bands) {
      std::stable_sort(band.begin(), band.end(), [&](size_t x, size_t y) { return work[x] > work[y]; });
      per_xcd = std::max<int64_t>(per_xcd, int64_t(band.size()));
    }
    const int64_t groups = per_xcd * kXcds;
    if (units_out != nullptr) *units_out = n_units;

    // Lays the bands out in launch order: the unit at position pos of XCD x's
    // band is workgroup pos * 8 + x; missing positions are padding
    // workgroups, all of whose waves are idle.
    auto emit = [&](const std::vector<std::vector<size_t>>& ordered, std::vector<WaveItem>& items) {
      WaveItem idle{};
      idle.step_count = -1;
      idle.row = -1;
      idle.group = 1;
      items.assign(size_t(groups) * kRowWaves, idle);
      for (int xcd = 0; xcd < kXcds; ++xcd) {
        const auto& band = ordered[size_t(xcd)];
        for (size_t pos = 0; pos < band.size(); ++pos) {
          const auto& unit = units[band[pos]];
          WaveItem* wg = &items[(pos * kXcds + size_t(xcd)) * kRowWaves];
          const bool shared = steps_of(unit[0]) > pack_steps;
          for (int w = 0; w < kRowWaves; ++w) {
            if (!shared && size_t(w) >= unit.size()) continue;
            const int32_t i = shared ? unit[0] : unit[size_t(w)];
            WaveItem& item = wg[w];
            item.c_off = m.row_scalar_off[i];
            item.step_first = step_first[size_t(i)];
            item.step_count = steps_of(i);
            item.h = m.row_size[i];
            item.row = i;
            item.group = shared ? kRowWaves : 1;
            item.lead = shared ? w : 0;
            const int32_t first = shared ? kStepRun * w : 0;
            if (first < item.step_count) item.first = out.steps[size_t(item.step_first + first)];
          }
        }
      }
    };
    if (heaviest != nullptr) emit(bands, *heaviest);

    // Chained order of each band for RHS 32 and 64.  A unit's affinity to the
    // units already placed counts 2 per shared block column and 1 per
    // neighbouring one; the next unit is the unplaced one of highest affinity,
    // ties to the heavier (then earlier) unit.  Affinities only grow, so a
    // max-heap with stale entries skipped finds it.  A block column used by
    // more than kMaxUsers units of the band adds no affinity: it says little
    // about which units belong together, and skipping it bounds the work by
    // 3 * kMaxUsers updates per block instead of growing with the square of
    // the units that share a column.
    constexpr size_t kMaxUsers = 64;
    // Chaining needs more than kChainMinUnits workgroups per XCD on average.
    // Heaviest first instead of chaining, measured at RHS 32 / 64: 512 block
    // rows of degree 8 -6% / -8%, 1024 rows -6% / +3%, 4096 rows of degree 1
    // (every workgroup packed) -5% at RHS 32; from 2048 rows of degree 4 on
    // chaining is as fast or faster (degree 2 at 4096 rows: -3% to -6%).
    constexpr size_t kChainMinUnits = 192;
    const bool chain = n_units > size_t(kXcds) * kChainMinUnits;
    std::vector<std::vector<int32_t>> users(static_cast<size_t>(cols));
    std::vector<std::vector<size_t>> chained(kXcds);
    for (int xcd = 0; xcd < kXcds; ++xcd) {
      // The chain takes the band's heavier three quarters; the lightest
      // quarter follows it in band order, heaviest first.
      const auto& sorted = bands[size_t(xcd)];
      const size_t n = sorted.size();
      const size_t head = chain ? n - n / 4 : 0;  // units chained
      std::vector<size_t> band(sorted.begin(), sorted.end());
      for (auto& u : users) u.clear();
      auto for_each_col = [&](size_t unit, auto&& f) {
        for (const int32_t i : units[unit])
          for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) f(m.block_col[blk]);
      };
      for (size_t q = 0; q < head; ++q) for_each_col(band[q], [&](int32_t c) { users[size_t(c)].push_back(int32_t(q)); });
      // Heap keys: affinity in the high word, then the lower position (the
      // band is sorted heaviest first, so that is the heavier unit).
      auto key = [](uint64_t affinity, size_t q) { return (affinity << 32) | (0xffffffffu - uint32_t(q)); };
      std::vector<uint32_t> affinity(head, 0), gain(head, 0);
      std::vector<char> placed(head, 0);
      std::vector<int32_t> touched;
      std::priority_queue<uint64_t> heap;
      for (size_t q = 0; q < head; ++q) heap.push(key(0, q));
      auto& order_out = chained[size_t(xcd)];
      while (!heap.empty()) {
        const uint64_t top = heap.top();
        heap.pop();
        const size_t q = 0xffffffffu - uint32_t(top);
        if (placed[q] || (top >> 32) != affinity[q]) continue;  // placed, or a stale entry
        placed[q] = 1;
        order_out.push_back(band[q]);
        // Gains of the units this placement touches, summed first so that each
        // touched unit is pushed once.
        touched.clear();
        for_each_col(band[q], [&](int32_t c) {
          for (int32_t d = -1; d <= 1; ++d) {
            if (c + d < 0 || c + d >= cols || users[size_t(c + d)].size() > kMaxUsers) continue;
            for (const int32_t r : users[size_t(c + d)]) {
              if (placed[size_t(r)]) continue;
              if (gain[size_t(r)] == 0) touched.push_back(r);
              gain[size_t(r)] += d == 0 ? 2 : 1;
            }
          }
        });
        for (const int32_t r : touched) {
          affinity[size_t(r)] += gain[size_t(r)];
          gain[size_t(r)] = 0;
          heap.push(key(affinity[size_t(r)], size_t(r)));
        }
      }
      order_out.insert(order_out.end(), band.begin() + std::ptrdiff_t(head), band.end());
    }
    emit(chained, *chained_items);
    return groups;
  };
  size_t n_units = 0;
  out.groups = launch_orders(kPackSteps, &out.rows, &out.rows_wide, &n_units);
  out.groups_rhs64 = launch_orders(kPackStepsRhs64, nullptr, &out.rows_rhs64, nullptr);

  // The tile-split kernel's order: pack_steps 0 gives every row with k steps
  // a workgroup of its own.
  out.groups_tile = launch_orders(0, nullptr, &out.rows_tile, nullptr);

  // RHS 64 kernel choice.  The tile-split kernel runs a row's steps one after
  // another on one workgroup (all four waves on each step), so its launch
  // lasts at least the longest row's steps.  It is taken when those stay
  // within kTileSpanLimit times the mean steps per workgroup slot (6
  // workgroups on each of the 256 CUs).  Measured against the split-k kernel
  // at RHS 64 (cold, alternating on one box): 4096 block rows of degree 1, 2,
  // 4, 8 and 16 and 1024-2048 rows of degree 8 and 16 (span ratio up to 2.2),
  // 2-15% faster; 512 and 256 rows of degree 16 (ratio 3.9 and 7.8) 8% and
  // 22% slower.
  {
    constexpr int64_t kTileSlots = 256 * 6;
    constexpr int64_t kTileSpanLimit = 3;
    int64_t longest = 0;
    for (int32_t i = 0; i < rows; ++i) longest = std::max<int64_t>(longest, steps_of(i));
    const int64_t total = int64_t(out.steps.size());
    out.rhs64_tiles = rows > 0 && longest * kTileSlots <= kTileSpanLimit * total;
  }

  // Split-row schedule.  Parts of a row hold part_steps consecutive steps (a
  // multiple of one run per wave, sized so that the parts of the whole
  // matrix fill about kSplitTargetGroups workgroups); the row's last part
  // holds the rest.  A part of more than kPackSteps steps gets a workgroup of
  // its own, shorter parts are packed kRowWaves to a workgroup.  Workgroups
  // run heaviest first, dealt to the XCDs in turn.
  constexpr int64_t kSplitTargetGroups = 2048;
  constexpr size_t kSplitBelowGroups = 160;
  constexpr int32_t kRunSteps = kRowWaves * kStepRun;
  HostSplitSchedule& sp = out.split;
  const int64_t total_steps = int64_t(out.steps.size());
  sp.part_steps = int32_t(kRunSteps * std::max<int64_t>(1, (total_steps + kRunSteps * kSplitTargetGroups - 1) /
                                                                (kRunSteps * kSplitTargetGroups)));
  struct Part {
    int32_t row, step_first, step_count;
    int64_t w_off;
  };
  std::vector<Part> parts;
  sp.rows.resize(static_cast<size_t>(rows));
  int64_t virtual_rows = 0;
  for (int32_t i = 0; i < rows; ++i) {
    const int32_t n = steps_of(i);
    const int32_t count = std::max<int32_t>(1, (n + sp.part_steps - 1) / sp.part_steps);
    SplitRowRec& rec = sp.rows[size_t(i)];
    rec.c_off = m.row_scalar_off[i];
    rec.w_off = virtual_rows;
    rec.h = m.row_size[i];
    rec.parts = count;
    rec.row = i;
    for (int32_t q = 0; q < count; ++q) {
      const int32_t first = q * sp.part_steps;
      parts.push_back({i, step_first[size_t(i)] + first, std::min(sp.part_steps, n - first), virtual_rows});
      virtual_rows += m.row_size[i];
    }
  }
  sp.virtual_rows = virtual_rows;
  auto part_work = [&](const Part& p) { return int64_t((m.row_size[p.row] + 15) / 16) * p.step_count; };
  std::vector<std::vector<size_t>> split_units;
  std::vector<size_t> short_parts;
  for (size_t q = 0; q < parts.size(); ++q) {
    if (parts[q].step_count > kPackSteps)
      split_units.push_back({q});
    else
      short_parts.push_back(q);
  }
  std::stable_sort(short_parts.begin(), short_parts.end(),
                   [&](size_t x, size_t y) { return part_work(parts[x]) > part_work(parts[y]); });
  for (size_t q = 0; q < short_parts.size(); q += kRowWaves)
    split_units.emplace_back(short_parts.begin() + std::ptrdiff_t(q),
                             short_parts.begin() + std::ptrdiff_t(std::min(short_parts.size(), q + size_t(kRowWaves))));
  auto unit_work = [&](const std::vector<size_t>& u) {
    int64_t w = 0;
    for (const size_t q : u) w += part_work(parts[q]);
    return w;
  };
  std::stable_sort(split_units.begin(), split_units.end(),
                   [&](const auto& x, const auto& y) { return unit_work(x) > unit_work(y); });
  sp.groups = int64_t((split_units.size() + kXcds - 1) / kXcds) * kXcds;
  WaveItem idle{};
  idle.step_count = -1;
  idle.row = -1;
  idle.group = 1;
  sp.items.assign(size_t(sp.groups) * kRowWaves, idle);
  for (size_t u = 0; u < split_units.size(); ++u) {
    WaveItem* wg = &sp.items[u * kRowWaves];
    const bool shared = parts[split_units[u][0]].step_count > kPackSteps;
    for (int w = 0; w < kRowWaves; ++w) {
      if (!shared && size_t(w) >= split_units[u].size()) continue;
      const Part& p = parts[shared ? split_units[u][0] : split_units[u][size_t(w)]];
      WaveItem& item = wg[w];
      item.c_off = p.w_off;
      item.step_first = p.step_first;
      item.step_count = p.step_count;
      item.h = m.row_size[p.row];
      item.row = p.row;
      item.group = shared ? kRowWaves : 1;
      item.lead = shared ? w : 0;
      const int32_t first = shared ? kStepRun * w : 0;
      if (first < item.step_count) item.first = out.steps[size_t(item.step_first + first)];
    }
  }
  // Automatic choice: the row-owned launch would occupy fewer than 160 of
  // the 256 CUs, and its longest row needs three or more runs per wave.
  // Measured at degree 16 (high sizes, random columns): the split-row path
  // takes 13-35% off at 32 and 64 block rows, 0-12% at 128, and is slower
  // from 256 rows on.
  int32_t longest = 0;
  for (int32_t i = 0; i < rows; ++i) longest = std::max(longest, steps_of(i));
  out.split_preferred = n_units < kSplitBelowGroups && longest > 2 * kRunSteps;
  return out;
}

}  // namespace vbsr_amd
