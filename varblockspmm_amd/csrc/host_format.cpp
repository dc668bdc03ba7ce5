// Host VBSR format: validation, deterministic generation, test input.
//
// Reference: src/format/vbsr.cpp:29-82 (validate) and
// src/format/generator.cpp:7-88 (generate).  The generator uses the same
// standard engine (std::mt19937_64), the same distribution object
// (std::uniform_real_distribution<float>) and the same draw order as the
// reference, so equal options give equal matrices.
#include <algorithm>
#include <array>
#include <random>

#include "internal.hpp"

namespace vbsr_amd {

vbsr_host_view HostMatrix::view() const {
  vbsr_host_view v{};
  v.block_rows = block_rows;
  v.block_cols = block_cols;
  v.row_ptr = row_ptr.data();
  v.row_ptr_len = int64_t(row_ptr.size());
  v.block_col = block_col.data();
  v.block_col_len = int64_t(block_col.size());
  v.row_size = row_size.data();
  v.row_size_len = int64_t(row_size.size());
  v.col_size = col_size.data();
  v.col_size_len = int64_t(col_size.size());
  v.row_scalar_off = row_scalar_off.data();
  v.row_scalar_off_len = int64_t(row_scalar_off.size());
  v.col_scalar_off = col_scalar_off.data();
  v.col_scalar_off_len = int64_t(col_scalar_off.size());
  v.value_off = value_off.data();
  v.value_off_len = int64_t(value_off.size());
  v.values = values.data();
  v.values_len = int64_t(values.size());
  return v;
}

namespace {

[[noreturn]] void reject(const char* why) { throw std::invalid_argument(why); }

bool valid_block_extent(int32_t size) { return size >= 8 && size <= 64 && size % 8 == 0; }

// True when next - prev == expected.  A difference that overflows int64 is
// never equal (the reference's subtraction would be undefined there).
bool step_is(int64_t prev, int64_t next, int64_t expected) {
  int64_t difference = 0;
  return !__builtin_sub_overflow(next, prev, &difference) && difference == expected;
}

}  // namespace

// vbsr.cpp:29-82.  The checks run coarse to fine in the reference's order, so
// a matrix with several defects reports the same first defect.
void validate(const vbsr_host_view& m) {
  const int64_t rows = m.block_rows, cols = m.block_cols;
  if (rows <= 0 || cols <= 0) reject("positive block dimensions required");
  // The C view can carry null arrays, which the reference's vectors cannot:
  // any array with entries must be present.
  if ((m.row_ptr_len > 0 && !m.row_ptr) || (m.block_col_len > 0 && !m.block_col) ||
      (m.row_size_len > 0 && !m.row_size) || (m.col_size_len > 0 && !m.col_size) ||
      (m.row_scalar_off_len > 0 && !m.row_scalar_off) || (m.col_scalar_off_len > 0 && !m.col_scalar_off) ||
      (m.value_off_len > 0 && !m.value_off) || (m.values_len > 0 && !m.values) || m.block_col_len < 0 ||
      m.values_len < 0)
    reject("null array with entries, or a negative length");
  if (m.row_ptr_len != rows + 1 || m.row_size_len != rows || m.col_size_len != cols)
    reject("metadata size mismatch");
  if (m.row_scalar_off_len != rows + 1 || m.col_scalar_off_len != cols + 1)
    reject("scalar offsets size mismatch");
  const int64_t nnzb = m.block_col_len;
  if (m.row_ptr[0] != 0 || m.row_ptr[rows] < 0 || int64_t(m.row_ptr[rows]) != nnzb)
    reject("bad row_ptr");
  if (m.value_off_len != nnzb + 1 || m.value_off[0] != 0 || m.value_off[nnzb] != m.values_len)
    reject("bad value offsets");

  for (int64_t i = 0; i < rows; ++i) {
    const int32_t h = m.row_size[i];
    if (m.row_ptr[i] > m.row_ptr[i + 1] || !valid_block_extent(h) ||
        !step_is(m.row_scalar_off[i], m.row_scalar_off[i + 1], h))
      reject("bad block row");
  }
  for (int64_t j = 0; j < cols; ++j) {
    const int32_t w = m.col_size[j];
    if (!valid_block_extent(w) || !step_is(m.col_scalar_off[j], m.col_scalar_off[j + 1], w))
      reject("bad block column");
  }

  // row_ptr is monotone here, so one forward walk finds each block's row.
  int64_t owner = 0;
  for (int64_t blk = 0; blk < nnzb; ++blk) {
    while (m.row_ptr[owner + 1] <= blk) ++owner;
    const int32_t col = m.block_col[blk];
    if (col < 0 || col >= cols) reject("block column out of range");
    if (!step_is(m.value_off[blk], m.value_off[blk + 1], int64_t(m.row_size[owner]) * m.col_size[col]))
      reject("block payload mismatch");
  }
}

namespace {

// One block extent per call, consuming the engine as generator.cpp:14-30 does.
class BlockExtentSource {
public:
  BlockExtentSource(int32_t distribution, std::mt19937_64& engine)
      : distribution_(distribution), engine_(engine) {}

  int32_t next() {
    static constexpr std::array<int32_t, 8> every{8, 16, 24, 32, 40, 48, 56, 64};
    static constexpr std::array<int32_t, 3> low{24, 32, 40};
    static constexpr std::array<int32_t, 4> bimodal{8, 16, 48, 64};
    static constexpr std::array<int32_t, 2> two{8, 64};
    switch (distribution_) {
    case VBSR_DIST_UNIFORM: return 32;
    case VBSR_DIST_LOW_VARIANCE: return low[engine_() % low.size()];
    case VBSR_DIST_HIGH_VARIANCE:
    case VBSR_DIST_TIED_8_TO_64: return every[engine_() % every.size()];
    case VBSR_DIST_BIMODAL: return bimodal[engine_() % bimodal.size()];
    case VBSR_DIST_BIMODAL_8_OR_64: return two[engine_() % two.size()];
    default: reject("unknown block-size distribution");
    }
  }

private:
  int32_t distribution_;
  std::mt19937_64& engine_;
};

std::vector<int64_t> prefix_offsets(const std::vector<int32_t>& extents) {
  std::vector<int64_t> offsets(extents.size() + 1, 0);
  for (size_t i = 0; i < extents.size(); ++i) offsets[i + 1] = offsets[i] + extents[i];
  return offsets;
}

}  // namespace

HostMatrix generate(const vbsr_generator_options& o) {
  if (o.degree < 1 || o.degree > 16 || o.block_rows < 1 || o.block_cols < 1 || o.degree > o.block_cols)
    reject("invalid generator dimensions");
  if (o.distribution < VBSR_DIST_UNIFORM || o.distribution > VBSR_DIST_TIED_8_TO_64)
    reject("unknown block-size distribution");
  if (o.locality < VBSR_LOCALITY_RANDOM || o.locality > VBSR_LOCALITY_LOCAL_CLAMPED)
    reject("unknown column locality");

  std::mt19937_64 engine(o.seed);
  BlockExtentSource extents(o.distribution, engine);

  HostMatrix m;
  m.block_rows = o.block_rows;
  m.block_cols = o.block_cols;
  m.row_size.resize(size_t(o.block_rows));
  m.col_size.resize(size_t(o.block_cols));
  for (auto& h : m.row_size) h = extents.next();
  for (int32_t j = 0; j < o.block_cols; ++j) {
    const bool tied = o.distribution == VBSR_DIST_TIED_8_TO_64 && j < o.block_rows;
    m.col_size[size_t(j)] = tied ? m.row_size[size_t(j)] : extents.next();
  }
  m.row_scalar_off = prefix_offsets(m.row_size);
  m.col_scalar_off = prefix_offsets(m.col_size);

  const int64_t nnzb = int64_t(o.block_rows) * o.degree;
  m.row_ptr.reserve(size_t(o.block_rows) + 1);
  m.block_col.reserve(size_t(nnzb));
  m.value_off.reserve(size_t(nnzb) + 1);
  m.row_ptr.push_back(0);
  m.value_off.push_back(0);

  // Reserve about the expected value count (each row's height times degree
  // times the mean block width) so that the packed values grow in one piece.
  const double mean_width = double(m.col_scalar_off.back()) / double(o.block_cols);
  const double expected = double(m.row_scalar_off.back()) * double(o.degree) * mean_width;
  m.values.reserve(size_t(expected * 1.05) + 65536);

  std::uniform_real_distribution<float> value(-1.0f, 1.0f);
  const uint64_t window = uint64_t(2 * o.degree + 1);
  std::vector<int32_t> chosen;
  chosen.reserve(16);
  for (int32_t i = 0; i < o.block_rows; ++i) {
    // Distinct columns by rejection, then ascending order.
    chosen.clear();
    while (int32_t(chosen.size()) < o.degree) {
      int32_t col;
      if (o.locality == VBSR_LOCALITY_RANDOM) {
        col = int32_t(engine() % uint64_t(o.block_cols));
      } else {
        const int32_t offset = int32_t(engine() % window) - o.degree;
        // Clamped windows centre on the diagonal held inside [0, C), so every
        // window holds at least `degree` distinct columns.
        col = o.locality == VBSR_LOCALITY_LOCAL
                  ? (i + offset + o.block_cols) % o.block_cols
                  : std::clamp(std::min(i, o.block_cols - 1) + offset, 0, o.block_cols - 1);
      }
      if (std::find(chosen.begin(), chosen.end(), col) == chosen.end()) chosen.push_back(col);
    }
    std::sort(chosen.begin(), chosen.end());

    for (const int32_t col : chosen) {
      m.block_col.push_back(col);
      const int64_t count = int64_t(m.row_size[size_t(i)]) * m.col_size[size_t(col)];
      for (int64_t v = 0; v < count; ++v) m.values.push_back(value(engine));
      m.value_off.push_back(m.value_off.back() + count);
    }
    m.row_ptr.push_back(int32_t(m.block_col.size()));
  }

  validate(m.view());
  return m;
}

void make_random_input(int64_t count, uint64_t seed, float* out) {
  std::mt19937 engine{unsigned(seed)};
  std::uniform_real_distribution<float> value(-1.0f, 1.0f);
  for (int64_t i = 0; i < count; ++i) out[i] = value(engine);
}

}  // namespace vbsr_amd
