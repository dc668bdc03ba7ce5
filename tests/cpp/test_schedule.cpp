// CPU checks of the row schedule (varblockspmm_amd/csrc/schedule.cpp), built
// from the library's own sources without a GPU.  For each matrix:
//   * the step records cover every block of every row exactly once, in
//     row_ptr order, with the A and B offsets the kernel reads;
//   * the three launch orders (RHS 8/16, RHS 32, RHS 64) hold every block
//     row once, in workgroups of four wave items: one shared row (rows of
//     more than kPackSteps steps) or up to four packed light rows, one per
//     wave; padding waves have step_count < 0; each item describes its row,
//     including the wave's first step record;
//   * `rows` and `rows_wide` place each row on the same XCD (workgroup index
//     mod 8), as `rows_rhs64` does for its own workgroups (it packs rows of
//     up to kPackStepsRhs64 steps), and no XCD's work exceeds an eighth of
//     the total by more than one row's;
//   * `rows` runs each XCD's workgroups heaviest first; `rows_wide` and
//     `rows_rhs64`, for more than 192 workgroups per XCD, chain the heavier three
//     quarters of each XCD's band and end it with the lightest quarter,
//     heaviest first, and are heaviest first throughout otherwise;
//   * the split-row schedule: each row's parts cover its steps in order and
//     take consecutive virtual rows, every part is in exactly one workgroup,
//     and the automatic choice follows its rule;
//   * building twice gives the same schedule;
//   * matrices whose rows share few block columns (every row on the same 8
//     columns; rows overlapping in 15 of 16 columns) build in seconds: the
//     chained order's work does not grow with the square of a column's users.
// It also checks the launchers' host-side panel check (check_panels) at the
// edges of the B and C ranges, where no address is ever dereferenced.
// Prints one line per check group and exits non-zero if any check fails.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <vector>

#include "internal.hpp"

namespace {

int failures = 0;

#define CHECK(cond)                                                              \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);     \
      ++failures;                                                                \
      return;                                                                    \
    }                                                                            \
  } while (0)

int64_t row_work(const vbsr_amd::WaveItem& item) { return int64_t((item.h + 15) / 16) * item.step_count; }

// Checks one launch order: kRowWaves items per workgroup, each workgroup
// either one shared row (every wave, lead = wave, each wave's first step
// record), or up to kRowWaves packed light rows (one per wave, then idle
// waves), or padding (all idle); every block row exactly once; each row on
// the same XCD in both orders; per-XCD work within an eighth plus one
// workgroup; the order of each XCD's workgroups.
void check_order(const vbsr_host_view& m, const vbsr_amd::HostSchedule& s,
                 const std::vector<vbsr_amd::WaveItem>& items, std::vector<int>& xcd_of_row, bool wide,
                 int64_t groups, int32_t pack_steps) {
  using vbsr_amd::kRowWaves;
  using vbsr_amd::kXcds;
  CHECK(int64_t(items.size()) == groups * kRowWaves);
  CHECK(groups % kXcds == 0);
  std::vector<int> seen(size_t(m.block_rows), 0);
  std::vector<int64_t> load(kXcds, 0);
  std::vector<std::vector<int64_t>> band_work(kXcds);
  bool padding_started[kXcds] = {};
  for (int64_t g = 0; g < groups; ++g) {
    const auto* wg = &items[size_t(g) * kRowWaves];
    const int xcd = int(g % kXcds);
    if (wg[0].step_count < 0) {
      for (int w = 0; w < kRowWaves; ++w) CHECK(wg[w].step_count < 0);
      padding_started[xcd] = true;
      continue;
    }
    CHECK(!padding_started[xcd]);  // padding only after an XCD's last workgroup
    int64_t work = 8;
    const bool shared = wg[0].group == kRowWaves;
    bool idle_seen = false;
    for (int w = 0; w < kRowWaves; ++w) {
      const auto& item = wg[w];
      if (!shared && item.step_count < 0) {
        idle_seen = true;
        continue;
      }
      CHECK(!idle_seen);  // a packed workgroup's idle waves come last
      const int32_t i = item.row;
      CHECK(i >= 0 && i < m.block_rows);
      CHECK(item.c_off == m.row_scalar_off[i]);
      CHECK(item.h == m.row_size[i]);
      int32_t first;
      if (shared) {
        CHECK(item.group == kRowWaves && item.lead == w && item.row == wg[0].row);
        CHECK(item.step_count > pack_steps);
        first = item.step_first + vbsr_amd::kStepRun * w;
      } else {
        CHECK(item.group == 1 && item.lead == 0);
        CHECK(item.step_count <= pack_steps);
        first = item.step_first;
      }
      const bool has = first < item.step_first + item.step_count;
      CHECK(item.first.a_off == (has ? s.steps[size_t(first)].a_off : 0));
      CHECK(item.first.b_off == (has ? s.steps[size_t(first)].b_off : 0));
      if (!shared || w == 0) {
        CHECK(++seen[size_t(i)] == 1);
        work += row_work(item);
        if (xcd_of_row[size_t(i)] < 0) xcd_of_row[size_t(i)] = xcd;
        CHECK(xcd_of_row[size_t(i)] == xcd);
      }
    }
    load[size_t(xcd)] += work;
    band_work[size_t(xcd)].push_back(work);
  }
  for (int32_t i = 0; i < m.block_rows; ++i) CHECK(seen[size_t(i)] == 1);
  int64_t heaviest = 0;
  for (const auto& band : band_work)
    for (const int64_t w : band) heaviest = std::max(heaviest, w);
  // Placement fills an XCD up to an eighth of the work (+1) and only then
  // falls back to the least loaded one.
  int64_t total = 0;
  for (const int64_t l : load) total += l;
  CHECK(*std::max_element(load.begin(), load.end()) <= total / kXcds + 1 + heaviest);
  size_t units = 0;
  for (const auto& band : band_work) units += band.size();
  const bool chained = wide && units > size_t(kXcds) * 192;
  for (int x = 0; x < kXcds; ++x) {
    const auto& band = band_work[size_t(x)];
    // rows_wide, chained: the heavier three quarters in chain order, then
    // the lightest quarter heaviest first; otherwise heaviest first.
    const size_t light = band.size() - band.size() / 4;
    const size_t from = chained ? light : 0;
    for (size_t q = from + 1; q < band.size(); ++q) CHECK(band[q - 1] >= band[q]);
    // The lightest quarter comes last: nothing before it is lighter.
    if (chained && light < band.size()) {
      const int64_t light_max = *std::max_element(band.begin() + std::ptrdiff_t(light), band.end());
      for (size_t q = 0; q < light; ++q) CHECK(band[q] >= light_max);
    }
  }
}

void check_steps(const vbsr_host_view& m, const vbsr_amd::HostSchedule& s) {
  const auto& items = s.rows;
  std::vector<const vbsr_amd::WaveItem*> by_row(size_t(m.block_rows), nullptr);
  for (const auto& item : items)
    if (item.step_count >= 0 && item.lead == 0) by_row[size_t(item.row)] = &item;
  int64_t expected_first = 0;
  for (int32_t i = 0; i < m.block_rows; ++i) {
    const auto* item = by_row[size_t(i)];
    CHECK(item != nullptr);
    CHECK(item->step_first == expected_first);
    int32_t step = item->step_first;
    const int32_t h = m.row_size[i];
    for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) {
      const int32_t col = m.block_col[blk];
      const int32_t w = m.col_size[col];
      int32_t k0 = 0;
      while (k0 < w) {
        CHECK(step < item->step_first + item->step_count);
        const auto& rec = s.steps[size_t(step)];
        const bool half = (rec.b_off & vbsr_amd::kHalfStep) != 0;
        CHECK(half == (w - k0 == 8));
        CHECK(rec.a_off == m.value_off[blk] + int64_t(k0) * h);
        CHECK((rec.b_off & (vbsr_amd::kHalfStep - 1)) == m.col_scalar_off[col] + k0);
        k0 += half ? 8 : 16;
        ++step;
      }
      CHECK(k0 == w);
    }
    CHECK(step == item->step_first + item->step_count);
    expected_first = step;
  }
  CHECK(int64_t(s.steps.size()) == expected_first);
}

// The split-row schedule: every row has at least one part; a row's parts
// take consecutive virtual rows (part q at w_off + q * h) and, in order, its
// consecutive steps, each part at most part_steps long; the workgroups hold
// every part once (a part of more than kPackSteps steps shared by all waves,
// shorter ones packed one per wave, idle waves last); the automatic choice
// follows its rule.
void check_split(const vbsr_host_view& m, const vbsr_amd::HostSchedule& s) {
  using vbsr_amd::kPackSteps;
  using vbsr_amd::kRowWaves;
  const auto& sp = s.split;
  CHECK(int64_t(sp.rows.size()) == m.block_rows);
  CHECK(sp.part_steps > 0 && sp.part_steps % (kRowWaves * vbsr_amd::kStepRun) == 0);
  CHECK(int64_t(sp.items.size()) == sp.groups * kRowWaves && sp.groups % vbsr_amd::kXcds == 0);
  // step_first of each row from the row items (the lead wave of each row)
  std::vector<int32_t> row_first(size_t(m.block_rows), -1), row_count(size_t(m.block_rows), -1);
  for (const auto& item : s.rows)
    if (item.step_count >= 0 && item.lead == 0) {
      row_first[size_t(item.row)] = item.step_first;
      row_count[size_t(item.row)] = item.step_count;
    }
  int64_t virtual_rows = 0;
  std::map<int64_t, const vbsr_amd::WaveItem*> by_offset;  // a part's first virtual row -> its item
  for (int64_t g = 0; g < sp.groups; ++g) {
    const auto* wg = &sp.items[size_t(g) * kRowWaves];
    const bool shared = wg[0].step_count >= 0 && wg[0].group == kRowWaves;
    bool idle_seen = false;
    for (int w = 0; w < kRowWaves; ++w) {
      const auto& item = wg[w];
      if (item.step_count < 0) {
        CHECK(!shared);
        idle_seen = true;
        continue;
      }
      CHECK(!idle_seen);
      if (shared) {
        CHECK(item.group == kRowWaves && item.lead == w && item.c_off == wg[0].c_off);
        CHECK(item.step_count > kPackSteps);
      } else {
        CHECK(item.group == 1 && item.lead == 0 && item.step_count <= kPackSteps);
      }
      const int32_t first = shared ? item.step_first + vbsr_amd::kStepRun * w : item.step_first;
      const bool has = first < item.step_first + item.step_count;
      CHECK(item.first.a_off == (has ? s.steps[size_t(first)].a_off : 0));
      CHECK(item.first.b_off == (has ? s.steps[size_t(first)].b_off : 0));
      if (!shared || w == 0) CHECK(by_offset.emplace(item.c_off, &item).second);
    }
  }
  for (int32_t i = 0; i < m.block_rows; ++i) {
    const auto& rec = sp.rows[size_t(i)];
    CHECK(rec.row == i && rec.h == m.row_size[i] && rec.c_off == m.row_scalar_off[i]);
    CHECK(rec.parts >= 1 && rec.w_off == virtual_rows);
    int32_t next = row_first[size_t(i)];
    for (int32_t q = 0; q < rec.parts; ++q) {
      const auto it = by_offset.find(rec.w_off + int64_t(q) * rec.h);
      CHECK(it != by_offset.end());
      const auto& item = *it->second;
      CHECK(item.row == i && item.h == rec.h && item.step_first == next);
      CHECK(item.step_count <= sp.part_steps && (item.step_count > 0 || rec.parts == 1));
      next += item.step_count;
    }
    CHECK(next == row_first[size_t(i)] + row_count[size_t(i)]);
    virtual_rows += int64_t(rec.parts) * rec.h;
  }
  CHECK(sp.virtual_rows == virtual_rows);
  int64_t parts = 0;
  for (const auto& rec : sp.rows) parts += rec.parts;
  CHECK(int64_t(by_offset.size()) == parts);
  int32_t longest = 0;
  int64_t units = 0;
  for (int64_t g = 0; g < s.groups; ++g)
    if (s.rows[size_t(g) * kRowWaves].step_count >= 0) ++units;
  for (int32_t i = 0; i < m.block_rows; ++i) longest = std::max(longest, row_count[size_t(i)]);
  CHECK(s.split_preferred == (units < 160 && longest > 2 * kRowWaves * vbsr_amd::kStepRun));
}

// The RHS 64 kernel choice, recomputed from the matrix alone: the tile split
// runs when the longest row's k steps are at most 3 x (all steps) / (256 x 6).
bool expected_tiles(const vbsr_host_view& m) {
  int64_t total = 0, longest = 0;
  for (int32_t i = 0; i < m.block_rows; ++i) {
    int64_t steps = 0;
    for (int32_t blk = m.row_ptr[i]; blk < m.row_ptr[i + 1]; ++blk) {
      const int32_t w = m.col_size[m.block_col[blk]];
      steps += w / 16 + (w % 16 != 0);
    }
    total += steps;
    longest = std::max(longest, steps);
  }
  return m.block_rows > 0 && longest * 256 * 6 <= 3 * total;
}

bool same(const std::vector<vbsr_amd::WaveItem>& a, const std::vector<vbsr_amd::WaveItem>& b) {
  return a.size() == b.size() && (a.empty() || std::memcmp(a.data(), b.data(), a.size() * sizeof(a[0])) == 0);
}

// reorders: the matrix is random enough that a chained order must differ
// from the heaviest-first one.
void check_view(const vbsr_host_view& m, const char* name, double max_seconds, bool reorders = false) {
  const int before = failures;
  const auto t0 = std::chrono::steady_clock::now();
  const vbsr_amd::HostSchedule s = vbsr_amd::build_schedule(m);
  const double seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  if (seconds > max_seconds) {
    std::fprintf(stderr, "FAILED: %s took %.2f s to schedule (limit %.0f s)\n", name, seconds, max_seconds);
    ++failures;
  }
  check_steps(m, s);
  check_split(m, s);
  CHECK(s.rhs64_tiles == expected_tiles(m));
  std::vector<int> xcd_of_row(size_t(m.block_rows), -1);
  check_order(m, s, s.rows, xcd_of_row, false, s.groups, vbsr_amd::kPackSteps);
  check_order(m, s, s.rows_wide, xcd_of_row, true, s.groups, vbsr_amd::kPackSteps);
  // The RHS 64 order packs more rows, so it places its own workgroups.
  std::vector<int> xcd_of_row64(size_t(m.block_rows), -1);
  check_order(m, s, s.rows_rhs64, xcd_of_row64, true, s.groups_rhs64, vbsr_amd::kPackStepsRhs64);
  // The tile split's order gives every row with steps a workgroup of its own.
  std::vector<int> xcd_of_row_tile(size_t(m.block_rows), -1);
  check_order(m, s, s.rows_tile, xcd_of_row_tile, true, s.groups_tile, 0);
  // Up to 192 workgroups per XCD the wide order is the heaviest-first one;
  // above it, on a random matrix, the chain reorders them.
  int64_t units = 0;
  for (size_t g = 0; g < s.rows.size(); g += vbsr_amd::kRowWaves) units += s.rows[g].step_count >= 0 ? 1 : 0;
  if (units <= int64_t(vbsr_amd::kXcds) * 192) {
    CHECK(same(s.rows, s.rows_wide));
  } else if (reorders) {
    CHECK(!same(s.rows, s.rows_wide));
  }
  const vbsr_amd::HostSchedule again = vbsr_amd::build_schedule(m);
  if (!(same(s.rows, again.rows) && same(s.rows_wide, again.rows_wide) && same(s.rows_rhs64, again.rows_rhs64) &&
        same(s.rows_tile, again.rows_tile) &&
        same(s.split.items, again.split.items) &&
        s.steps.size() == again.steps.size())) {
    std::fprintf(stderr, "FAILED: schedule not deterministic\n");
    ++failures;
  }
  std::printf("%s %s groups=%lld steps=%zu schedule=%.3f s\n", failures == before ? "ok" : "FAILED", name,
              static_cast<long long>(s.groups), s.steps.size(), seconds);
}

void check_host(const vbsr_amd::HostMatrix& host, const char* name, bool reorders = false) {
  const vbsr_host_view m = host.view();
  vbsr_amd::validate(m);
  check_view(m, name, 30.0, reorders);
}

// Block row i uses block columns (i + j) mod cols, j < degree, all blocks
// 64 x 64.  Only the metadata is built: the schedule never reads values.
void check_shared_columns(int32_t rows, int32_t cols, int32_t degree) {
  vbsr_amd::HostMatrix h;
  h.block_rows = rows;
  h.block_cols = cols;
  h.row_ptr.push_back(0);
  for (int32_t i = 0; i < rows; ++i) {
    for (int32_t j = 0; j < degree; ++j) h.block_col.push_back((i + j) % cols);
    h.row_ptr.push_back(int32_t(h.block_col.size()));
  }
  h.row_size.assign(size_t(rows), 64);
  h.col_size.assign(size_t(cols), 64);
  for (int32_t i = 0; i <= rows; ++i) h.row_scalar_off.push_back(int64_t(i) * 64);
  for (int32_t c = 0; c <= cols; ++c) h.col_scalar_off.push_back(int64_t(c) * 64);
  for (size_t b = 0; b <= h.block_col.size(); ++b) h.value_off.push_back(int64_t(b) * 64 * 64);
  vbsr_host_view m = h.view();
  m.values_len = h.value_off.back();
  char name[96];
  std::snprintf(name, sizeof(name), "shared columns: rows=%d cols=%d degree=%d", rows, cols, degree);
  check_view(m, name, 10.0);
}

// Three block rows, the middle one empty; block widths 8 (one half step),
// 24 (a full and a half step) and 64 (four full steps).
vbsr_amd::HostMatrix with_empty_row() {
  vbsr_amd::HostMatrix h;
  h.block_rows = 3;
  h.block_cols = 3;
  h.row_ptr = {0, 2, 2, 4};
  h.block_col = {0, 2, 1, 2};
  h.row_size = {16, 8, 40};
  h.col_size = {8, 24, 64};
  h.row_scalar_off = {0, 16, 24, 64};
  h.col_scalar_off = {0, 8, 32, 96};
  h.value_off = {0, 16 * 8, 16 * 8 + 16 * 64, 16 * 8 + 16 * 64 + 40 * 24, 16 * 8 + 16 * 64 + 40 * 24 + 40 * 64};
  h.values.assign(size_t(h.value_off.back()), 1.0f);
  return h;
}

// B holds K x rhs floats and C M x rhs: ranges that touch are accepted,
// ranges that share one float are not.
void check_panel_ranges() {
  const int before = failures;
  vbsr_device_view v{};
  v.scalar_rows = 96;
  v.scalar_cols = 80;
  const int rhs = 8;
  static float arena[4096];
  float* b = arena + 1024;
  const auto rejected = [&](const float* bb, const float* cc) {
    try {
      vbsr_amd::check_panels(v, bb, cc, rhs);
    } catch (const std::invalid_argument&) {
      return true;
    }
    return false;
  };
  [&] {
    CHECK(!rejected(b, b + 80 * rhs));      // C starts where B ends
    CHECK(!rejected(b, b - 96 * rhs));      // C ends where B starts
    CHECK(rejected(b, b + 80 * rhs - 1));   // C starts on B's last float
    CHECK(rejected(b, b - 96 * rhs + 1));   // C ends on B's first float
    CHECK(rejected(b, b));
    CHECK(rejected(nullptr, b));
    CHECK(rejected(b, nullptr));
  }();
  std::printf("%s panel ranges\n", failures == before ? "ok" : "FAILED");
}

}  // namespace

int main() {
  const int32_t shapes[][5] = {
      // rows, cols, degree, distribution, locality
      {4096, 4096, 8, VBSR_DIST_HIGH_VARIANCE, VBSR_LOCALITY_RANDOM},
      {4096, 4096, 8, VBSR_DIST_HIGH_VARIANCE, VBSR_LOCALITY_LOCAL},
      {1024, 1024, 4, VBSR_DIST_HIGH_VARIANCE, VBSR_LOCALITY_LOCAL_CLAMPED},
      {1024, 1024, 8, VBSR_DIST_LOW_VARIANCE, VBSR_LOCALITY_RANDOM},
      {4096, 4096, 16, VBSR_DIST_BIMODAL, VBSR_LOCALITY_RANDOM},
      {4096, 4096, 1, VBSR_DIST_UNIFORM, VBSR_LOCALITY_RANDOM},
      {4096, 4096, 1, VBSR_DIST_HIGH_VARIANCE, VBSR_LOCALITY_RANDOM},
      {2048, 2048, 2, VBSR_DIST_HIGH_VARIANCE, VBSR_LOCALITY_LOCAL_CLAMPED},
      {9, 17, 4, VBSR_DIST_HIGH_VARIANCE, VBSR_LOCALITY_LOCAL},
      {5, 3, 2, VBSR_DIST_BIMODAL, VBSR_LOCALITY_RANDOM},
      {1, 1, 1, VBSR_DIST_UNIFORM, VBSR_LOCALITY_RANDOM},
      {37, 64, 16, VBSR_DIST_LOW_VARIANCE, VBSR_LOCALITY_RANDOM},
  };
  uint64_t seed = 1;
  for (const auto& shape : shapes) {
    vbsr_generator_options options{};
    options.block_rows = shape[0];
    options.block_cols = shape[1];
    options.degree = shape[2];
    options.rhs_width = 32;
    options.distribution = shape[3];
    options.locality = shape[4];
    options.seed = seed++;
    char name[128];
    std::snprintf(name, sizeof(name), "rows=%d degree=%d dist=%d locality=%d seed=%llu", options.block_rows,
                  options.degree, options.distribution, options.locality,
                  static_cast<unsigned long long>(options.seed));
    check_host(vbsr_amd::generate(options), name, shape[0] == 4096 && shape[2] >= 8);
  }
  check_host(with_empty_row(), "hand-made, empty middle row");
  // The RHS 64 rule on shapes it was measured on: the tile split at 4096
  // block rows of degree 1 to 16 and at 1024 rows of degree 16; the split-k
  // kernel at 256 and 512 rows of degree 16 (a few long rows per CU).
  const int32_t tile_shapes[][5] = {
      // rows, degree, distribution, seed, expected
      {4096, 8, VBSR_DIST_HIGH_VARIANCE, 1, 1}, {4096, 16, VBSR_DIST_BIMODAL_8_OR_64, 3, 1},
      {1024, 16, VBSR_DIST_HIGH_VARIANCE, 1, 1}, {256, 16, VBSR_DIST_HIGH_VARIANCE, 1, 0},
      {512, 16, VBSR_DIST_HIGH_VARIANCE, 1, 0}, {4096, 2, VBSR_DIST_HIGH_VARIANCE, 1, 1},
      {4096, 1, VBSR_DIST_HIGH_VARIANCE, 1, 1}};
  for (const auto& t : tile_shapes) {
    vbsr_generator_options options{};
    options.block_rows = options.block_cols = t[0];
    options.degree = t[1];
    options.rhs_width = 64;
    options.distribution = t[2];
    options.locality = VBSR_LOCALITY_RANDOM;
    options.seed = uint64_t(t[3]);
    const vbsr_amd::HostMatrix host = vbsr_amd::generate(options);
    const vbsr_amd::HostSchedule s = vbsr_amd::build_schedule(host.view());
    if (s.rhs64_tiles != (t[4] != 0)) {
      std::fprintf(stderr, "FAILED: rhs64_tiles=%d at rows=%d degree=%d\n", int(s.rhs64_tiles), t[0], t[1]);
      ++failures;
    }
  }
  check_shared_columns(16384, 8, 8);
  check_shared_columns(65536, 16384, 16);
  check_panel_ranges();
  std::printf("%s\n", failures == 0 ? "ALL OK" : "FAILURES");
  return failures == 0 ? 0 : 1;
}
