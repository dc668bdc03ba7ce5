// l2_model: a CPU model of the B-line misses of the row-owned kernel in each
// XCD's L2, for a matrix, an RHS width and one of the schedule's launch
// orders.  It explains the kernel's L2-miss (FETCH_SIZE) traffic and bounds
// what any row order can save, without a GPU.
//
// What it models:
//  * the launch: workgroup i runs on XCD i mod 8 (the schedule's placement);
//    each XCD runs `occupancy` workgroups per CU on 32 CUs, starting the next
//    of its workgroups when one ends;
//  * a workgroup's waves: a shared row's runs of two steps dealt to four
//    waves, or one packed light row per wave;
//  * a workgroup's duration: c0 + c1 * (its largest per-wave step count), the
//    shape measured with per-workgroup timestamps on an MI355X (at RHS 32,
//    about 6 + 1 us per step of a wave);
//  * its B accesses: each k step reads, for each RHS column, its 16 (or 8) B
//    values, at start + c0/2 + (the step's position within its wave) * c1;
//    each access touches the one or two 128-byte lines the values lie in;
//  * C: each row's slab is written at its end, and allocates in L2;
//  * A: read with the non-temporal hint, modelled as not allocating;
//  * the L2: 4 MiB per XCD, 16 ways, 128-byte lines, LRU, a hashed set index.
//
// It reports B line misses (each one a 128-byte fetch) next to two bounds
// computed from the same accesses: no reuse at all, and an unbounded L2 per
// XCD (each XCD fetches every line it touches once).
//
//   make -C varblockspmm_amd/bench l2_model
//   varblockspmm_amd/bench/l2_model --rhs 32 [--rows 4096 --degree 8
//       --distribution high --locality random --seed 1 --order wide|rows]
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <queue>
#include <string>
#include <unordered_set>
#include <vector>

#include "internal.hpp"

namespace {

using vbsr_amd::HostMatrix;
using vbsr_amd::HostSchedule;
using vbsr_amd::kHalfStep;
using vbsr_amd::kRowWaves;
using vbsr_amd::kStepRun;
using vbsr_amd::kXcds;
using vbsr_amd::WaveItem;
using vbsr_amd::StepRec;

constexpr int64_t kLine = 128;
constexpr int kCusPerXcd = 32;

struct Options {
  int rows = 4096, degree = 8, rhs = 32, occupancy = 0;
  std::string distribution = "high", locality = "random", order = "";
  uint64_t seed = 1;
  double l2_mib = 4.0, c0 = 6.0, c1 = 1.0;
  int ways = 16;
  int c_allocates = 1;
  std::string b_layout = "columns";
};

int parse_distribution(const std::string& s) {
  const char* names[] = {"uniform", "low", "high", "bimodal", "bimodal8or64", "tied8to64"};
  for (int i = 0; i < 6; ++i)
    if (s == names[i]) return i;
  std::fprintf(stderr, "unknown distribution %s\n", s.c_str());
  std::exit(2);
}

int parse_locality(const std::string& s) {
  if (s == "random") return VBSR_LOCALITY_RANDOM;
  if (s == "local") return VBSR_LOCALITY_LOCAL;
  if (s == "clamped") return VBSR_LOCALITY_LOCAL_CLAMPED;
  std::fprintf(stderr, "unknown locality %s\n", s.c_str());
  std::exit(2);
}

// Set-associative LRU cache of 128-byte lines.
class Cache {
public:
  Cache(int64_t bytes, int ways) : ways_(ways), sets_(bytes / kLine / ways) {
    tags_.assign(size_t(sets_ * ways_), -1);
    stamp_.assign(tags_.size(), 0);
  }
  // Returns true on a miss; `allocate` inserts the line on a miss.
  bool access(int64_t line, bool allocate) {
    const uint64_t h = uint64_t(line) ^ (uint64_t(line) >> 11) ^ (uint64_t(line) >> 23);
    const int64_t set = int64_t(h % uint64_t(sets_));
    int64_t* tags = &tags_[size_t(set * ways_)];
    uint64_t* stamp = &stamp_[size_t(set * ways_)];
    ++clock_;
    int victim = 0;
    for (int w = 0; w < ways_; ++w) {
      if (tags[w] == line) {
        stamp[w] = clock_;
        return false;
      }
      if (stamp[w] < stamp[victim]) victim = w;
    }
    if (allocate) {
      tags[victim] = line;
      stamp[victim] = clock_;
    }
    return true;
  }

private:
  int ways_;
  int64_t sets_;
  std::vector<int64_t> tags_;
  std::vector<uint64_t> stamp_;
  uint64_t clock_ = 0;
};

struct Event {
  double time;
  int64_t line;
  bool is_b;
};

}  // namespace

int main(int argc, char** argv) {
  Options o;
  for (int i = 1; i + 1 < argc; i += 2) {
    const std::string k = argv[i];
    const char* v = argv[i + 1];
    if (k == "--rows") o.rows = std::atoi(v);
    else if (k == "--degree") o.degree = std::atoi(v);
    else if (k == "--rhs") o.rhs = std::atoi(v);
    else if (k == "--distribution") o.distribution = v;
    else if (k == "--locality") o.locality = v;
    else if (k == "--seed") o.seed = std::strtoull(v, nullptr, 10);
    else if (k == "--order") o.order = v;
    else if (k == "--occupancy") o.occupancy = std::atoi(v);
    else if (k == "--l2-mib") o.l2_mib = std::atof(v);
    else if (k == "--ways") o.ways = std::atoi(v);
    else if (k == "--c0") o.c0 = std::atof(v);
    else if (k == "--c1") o.c1 = std::atof(v);
    else if (k == "--c-allocates") o.c_allocates = std::atoi(v);
    else if (k == "--b-layout") o.b_layout = v;
    else {
      std::fprintf(stderr, "unknown option %s\n", k.c_str());
      return 2;
    }
  }
  if (o.order.empty()) o.order = o.rhs >= 32 ? "wide" : "rows";
  // Workgroups per CU of the row-owned kernel (its LDS and registers).
  if (o.occupancy == 0) o.occupancy = o.rhs == 8 ? 6 : o.rhs == 16 ? 5 : o.rhs == 32 ? 4 : 3;

  vbsr_generator_options g{};
  g.block_rows = g.block_cols = o.rows;
  g.degree = o.degree;
  g.rhs_width = o.rhs;
  g.distribution = parse_distribution(o.distribution);
  g.locality = parse_locality(o.locality);
  g.seed = o.seed;
  const HostMatrix m = vbsr_amd::generate(g);
  const vbsr_host_view view = m.view();
  const HostSchedule s = vbsr_amd::build_schedule(view);
  // The wide order is the one the library launches at RHS 32, and at RHS 64
  // with its own packing.
  const bool wide64 = o.order == "wide" && o.rhs == 64;
  const std::vector<WaveItem>& items = wide64 ? s.rows_rhs64 : o.order == "wide" ? s.rows_wide : s.rows;
  const int64_t groups = wide64 ? s.groups_rhs64 : s.groups;
  const int64_t K = view.col_scalar_off[view.col_scalar_off_len - 1];
  const int64_t M = view.row_scalar_off[view.row_scalar_off_len - 1];
  const int64_t b_base = 0, c_base = (K * o.rhs * 4 / kLine + 1024) * kLine;

  int64_t b_misses = 0, b_accesses = 0, c_misses = 0, unbounded = 0;
  for (int xcd = 0; xcd < kXcds; ++xcd) {
    std::vector<Event> events;
    // Workgroup start times: a list scheduler over the XCD's slots.
    std::priority_queue<double, std::vector<double>, std::greater<double>> free_at;
    for (int i = 0; i < kCusPerXcd * o.occupancy; ++i) free_at.push(0.0);
    for (int64_t gi = xcd; gi < groups; gi += kXcds) {
      const WaveItem* wg = &items[size_t(gi) * kRowWaves];
      if (wg[0].step_count < 0) continue;  // padding workgroup
      const double start = free_at.top();
      free_at.pop();
      // The waves' steps: a shared row's runs of kStepRun dealt round robin,
      // or each packed row's steps in order on its own wave.
      const bool shared = wg[0].group == kRowWaves;
      int longest = 0;
      for (int w = 0; w < kRowWaves; ++w) {
        const WaveItem& item = wg[w];
        if (item.step_count < 0 || (shared && w > 0)) continue;
        const int p = shared ? kRowWaves : 1;
        const int per_wave = (item.step_count + p * kStepRun - 1) / (p * kStepRun) * kStepRun;
        longest = std::max(longest, std::min(per_wave, item.step_count));
        for (int j = 0; j < item.step_count; ++j) {
          const StepRec& st = s.steps[size_t(item.step_first + j)];
          const int64_t k0 = st.b_off & (kHalfStep - 1);
          const int64_t len = (st.b_off & kHalfStep) ? 8 : 16;
          const int run = j / kStepRun;
          const int position = (run / p) * kStepRun + j % kStepRun;  // the step's place in its wave
          const double t = start + o.c0 * 0.5 + o.c1 * position + 1e-6 * (j % 7);
          if (o.b_layout == "rows") {
            const int64_t first = (b_base + k0 * o.rhs * 4) / kLine;
            const int64_t last = (b_base + (k0 + len) * o.rhs * 4 - 1) / kLine;
            for (int64_t line = first; line <= last; ++line) events.push_back({t, line, true});
          } else {
            for (int n = 0; n < o.rhs; ++n) {
              const int64_t first = (b_base + (n * K + k0) * 4) / kLine;
              const int64_t last = (b_base + (n * K + k0 + len) * 4 - 1) / kLine;
              for (int64_t line = first; line <= last; ++line) events.push_back({t, line, true});
            }
          }
        }
      }
      const double end = start + o.c0 + o.c1 * longest;
      free_at.push(end);
      for (int w = 0; w < kRowWaves; ++w) {
        const WaveItem& item = wg[w];
        if (item.step_count < 0 || (shared && w > 0)) continue;
        for (int n = 0; n < o.rhs; ++n) {
          const int64_t first = (c_base + (n * M + item.c_off) * 4) / kLine;
          const int64_t last = (c_base + (n * M + item.c_off + item.h) * 4 - 1) / kLine;
          for (int64_t line = first; line <= last; ++line) events.push_back({end, line, false});
        }
      }
    }
    std::stable_sort(events.begin(), events.end(), [](const Event& a, const Event& b) { return a.time < b.time; });
    Cache cache(int64_t(o.l2_mib * 1024 * 1024), o.ways);
    std::unordered_set<int64_t> seen;
    for (const Event& e : events) {
      const bool miss = cache.access(e.line, e.is_b || o.c_allocates != 0);
      if (e.is_b) {
        ++b_accesses;
        b_misses += miss;
        if (seen.insert(e.line).second) ++unbounded;
      } else {
        c_misses += miss;
      }
    }
  }
  std::printf("{\"rows\": %d, \"degree\": %d, \"distribution\": \"%s\", \"locality\": \"%s\", \"seed\": %llu, "
              "\"rhs\": %d, \"order\": \"%s\", \"occupancy\": %d, \"l2_mib\": %.1f, \"b_bytes\": %lld, "
              "\"b_line_accesses\": %lld, \"b_line_misses\": %lld, \"b_miss_mb\": %.1f, "
              "\"no_reuse_mb\": %.1f, \"unbounded_l2_mb\": %.1f}\n",
              o.rows, o.degree, o.distribution.c_str(), o.locality.c_str(), static_cast<unsigned long long>(o.seed),
              o.rhs, o.order.c_str(), o.occupancy, o.l2_mib, static_cast<long long>(K * o.rhs * 4),
              static_cast<long long>(b_accesses), static_cast<long long>(b_misses), b_misses * 128e-6,
              b_accesses * 128e-6, unbounded * 128e-6);
  return 0;
}
