// Mutation fuzzing of validate (varblockspmm_amd/csrc/host_format.cpp) on the
// CPU, meant to be built with AddressSanitizer and UBSan: starting from valid
// generated matrices, each round corrupts array entries and array lengths
// (every pointer still owns exactly its stated length), then calls validate.
// It must either accept or throw std::invalid_argument, and never read
// outside the arrays it is given.  Accepted mutants must also be accepted
// again (validate is deterministic) and build a schedule whose step records
// stay inside the matrix.  Prints a summary; exits non-zero on a failure.
#include <cstdio>
#include <limits>
#include <random>
#include <type_traits>
#include <stdexcept>
#include <vector>

#include "internal.hpp"

namespace {

struct Arrays {
  int32_t block_rows{}, block_cols{};
  std::vector<int32_t> row_ptr, block_col, row_size, col_size;
  std::vector<int64_t> row_scalar_off, col_scalar_off, value_off;
  std::vector<float> values;

  vbsr_host_view view() const {
    vbsr_host_view v{};
    v.block_rows = block_rows;
    v.block_cols = block_cols;
    v.row_ptr = row_ptr.data(), v.row_ptr_len = int64_t(row_ptr.size());
    v.block_col = block_col.data(), v.block_col_len = int64_t(block_col.size());
    v.row_size = row_size.data(), v.row_size_len = int64_t(row_size.size());
    v.col_size = col_size.data(), v.col_size_len = int64_t(col_size.size());
    v.row_scalar_off = row_scalar_off.data(), v.row_scalar_off_len = int64_t(row_scalar_off.size());
    v.col_scalar_off = col_scalar_off.data(), v.col_scalar_off_len = int64_t(col_scalar_off.size());
    v.value_off = value_off.data(), v.value_off_len = int64_t(value_off.size());
    v.values = values.data(), v.values_len = int64_t(values.size());
    return v;
  }
};

Arrays from(const vbsr_amd::HostMatrix& h) {
  Arrays a;
  a.block_rows = h.block_rows;
  a.block_cols = h.block_cols;
  a.row_ptr = h.row_ptr, a.block_col = h.block_col, a.row_size = h.row_size, a.col_size = h.col_size;
  a.row_scalar_off = h.row_scalar_off, a.col_scalar_off = h.col_scalar_off, a.value_off = h.value_off;
  a.values = h.values;
  return a;
}

template <class T>
void mutate_vector(std::vector<T>& v, std::mt19937_64& rng) {
  switch (rng() % 6) {
  case 0:
    if (!v.empty()) {
      T& x = v[rng() % v.size()];
      const T delta = T(int64_t(rng() % 17) - 8);
      if constexpr (std::is_integral_v<T>) {
        T sum{};
        if (!__builtin_add_overflow(x, delta, &sum)) x = sum;
      } else {
        x += delta;
      }
    }
    break;
  case 1:
    if (!v.empty()) v[rng() % v.size()] = T(int64_t(rng() % 200) - 100);
    break;
  case 2:
    if (!v.empty()) v.pop_back();
    break;
  case 3:
    v.push_back(T(int64_t(rng() % 100)));
    break;
  case 4:
    if (!v.empty()) v[rng() % v.size()] = std::numeric_limits<T>::max();
    break;
  default:
    if (!v.empty()) v[rng() % v.size()] = std::numeric_limits<T>::lowest();
    break;
  }
}

}  // namespace

int main() {
  std::mt19937_64 rng(2024);
  int64_t accepted = 0, rejected = 0, failures = 0;
  const int32_t shapes[][3] = {{9, 17, 4}, {5, 3, 2}, {1, 1, 1}, {12, 12, 6}};
  for (int round = 0; round < 4000; ++round) {
    const auto& shape = shapes[round % 4];
    vbsr_generator_options o{shape[0], shape[1], shape[2], 8, int32_t(round % 6), int32_t(round % 3), uint64_t(round)};
    Arrays a = from(vbsr_amd::generate(o));
    const int edits = 1 + int(rng() % 3);
    for (int e = 0; e < edits; ++e) {
      switch (rng() % 10) {
      case 0: mutate_vector(a.row_ptr, rng); break;
      case 1: mutate_vector(a.block_col, rng); break;
      case 2: mutate_vector(a.row_size, rng); break;
      case 3: mutate_vector(a.col_size, rng); break;
      case 4: mutate_vector(a.row_scalar_off, rng); break;
      case 5: mutate_vector(a.col_scalar_off, rng); break;
      case 6: mutate_vector(a.value_off, rng); break;
      case 7: mutate_vector(a.values, rng); break;
      case 8: a.block_rows += int32_t(rng() % 5) - 2; break;
      default: a.block_cols += int32_t(rng() % 5) - 2; break;
      }
    }
    const vbsr_host_view v = a.view();
    try {
      vbsr_amd::validate(v);
    } catch (const std::invalid_argument&) {
      ++rejected;
      continue;
    }
    ++accepted;
    try {
      vbsr_amd::validate(v);
      const vbsr_amd::HostSchedule s = vbsr_amd::build_schedule(v);
      for (const auto& rec : s.steps) {
        const int64_t b = rec.b_off & (vbsr_amd::kHalfStep - 1);
        if (rec.a_off < 0 || rec.a_off >= v.values_len || b < v.col_scalar_off[0] || b >= v.col_scalar_off[v.block_cols]) {
          std::fprintf(stderr, "FAILED round %d: step record outside the matrix\n", round);
          ++failures;
          break;
        }
      }
    } catch (const std::exception& e) {
      std::fprintf(stderr, "FAILED round %d: accepted matrix then threw %s\n", round, e.what());
      ++failures;
    }
  }
  std::printf("%lld accepted, %lld rejected, %lld failures\n", static_cast<long long>(accepted),
              static_cast<long long>(rejected), static_cast<long long>(failures));
  std::printf("%s\n", failures == 0 ? "ALL OK" : "FAILURES");
  return failures == 0 ? 0 : 1;
}
