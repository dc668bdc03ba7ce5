// Internal declarations of libvarblockspmm_amd.  The public boundary is the
// C ABI in include/vbsr.h; everything here may throw std::invalid_argument or
// std::runtime_error, which capi.cpp maps to status codes.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "vbsr.h"

namespace vbsr_amd {

// Throws std::runtime_error carrying the HIP error string on failure.
void check_hip(hipError_t status, const char* what);

// ---- host format (host_format.cpp) --------------------------------------

// HostMatrix::validate (vbsr.cpp:29-82): same checks, same order.
void validate(const vbsr_host_view& host);

// Owning host matrix with the reference HostMatrix fields (vbsr.hpp:16-29).
struct HostMatrix {
  int32_t block_rows{}, block_cols{};
  std::vector<int32_t> row_ptr, block_col, row_size, col_size;
  std::vector<int64_t> row_scalar_off, col_scalar_off, value_off;
  std::vector<float> values;
  vbsr_host_view view() const;
};

// generate (generator.cpp:7-88) plus the extension distributions/localities.
HostMatrix generate(const vbsr_generator_options& options);

// make_random_input (tests/test_main.cpp:42-51).
void make_random_input(int64_t count, uint64_t seed, float* out);

// cpu_reference (vbsr.hpp:82-87; vbsr.cpp:167-201), cpu_reference.cpp.
// Validates the matrix (and non-negative scalar offset starts), then writes
// C (c_len == scalar_rows * rhs floats) from B (b_len == scalar_cols * rhs).
void cpu_reference(const vbsr_host_view& m, const float* b, int64_t b_len, int rhs, float* c, int64_t c_len);

// ---- row schedule (schedule.cpp) -------------------------------------------

// XCDs of an MI355X.  Workgroups are dispatched to XCDs round-robin by index.
constexpr int kXcds = 8;

// One k step of one block row: 16 columns of one block, or the 8 columns
// that end a block whose width is 8 mod 16 (a half step).
struct alignas(16) StepRec {
  int64_t a_off;  // value_off[blk] + k0 * h: first value of the step's columns
  int64_t b_off;  // col_scalar_off[block_col[blk]] + k0, | kHalfStep for a half step
};
static_assert(sizeof(StepRec) == 16, "StepRec is read as one dwordx4");
constexpr int64_t kHalfStep = int64_t(1) << 62;

// The row-owned kernel's workgroup: kRowWaves waves.  They hold either one
// block row together -- its k steps dealt to the waves in runs of kStepRun
// consecutive steps (wave w's first step is the row's step kStepRun * w) and
// their partial tiles summed in LDS -- or up to kRowWaves light rows of at
// most kPackSteps steps, one per wave, with no reduction.
constexpr int kRowWaves = 4;
constexpr int kStepRun = 2;
constexpr int kPackSteps = 4;
// At RHS 64, whose k steps cost about twice those of RHS 32, rows of up to
// kPackStepsRhs64 steps are packed.
constexpr int kPackStepsRhs64 = 8;

// One wave's work: its share of block row `row`, whose steps are
// steps[step_first .. step_first + step_count).  `group` waves share the row
// (kRowWaves, or 1 for a packed light row) and this wave is the `lead`-th of
// them.  An idle wave (a packed workgroup with fewer than kRowWaves rows, or
// a padding workgroup) has step_count < 0.  `first` repeats the wave's first
// step record (zero when it has none), so the kernel can issue that step's
// loads as soon as the item arrives instead of after the step records.
// 48 bytes; a workgroup's kRowWaves items are consecutive.
struct alignas(16) WaveItem {
  int64_t c_off;       // row_scalar_off[row]: first row of C written
  int32_t step_first;  // index of the row's first StepRec
  int32_t step_count;  // the row's k steps; < 0 for an idle wave
  int32_t h;           // row_size[row]: leading dimension of the row's blocks
  int32_t row;         // block row (diagnostics only; -1 when idle)
  int32_t group;       // waves sharing the row: kRowWaves or 1
  int32_t lead;        // this wave's index among them
  StepRec first;
};
static_assert(sizeof(WaveItem) == 48, "WaveItem is read as 12 dwords");

// The split-row path (SplitRow): each block row's k steps are cut into parts
// of at most `part_steps` steps; the row-owned kernel computes each part's
// h x RHS partial slab into a workspace of `virtual_rows` rows (part p of a
// row at virtual rows w_off + p * h), and a second kernel sums each row's
// slabs into C in part order.
struct alignas(16) SplitRowRec {
  int64_t c_off;  // row_scalar_off[row]
  int64_t w_off;  // the row's first virtual row
  int32_t h;      // row_size[row]
  int32_t parts;  // at least 1
  int32_t row;
  int32_t pad;
};
static_assert(sizeof(SplitRowRec) == 32, "SplitRowRec is read as 8 dwords");

struct HostSplitSchedule {
  std::vector<WaveItem> items;     // kRowWaves per workgroup; a part's c_off is its first virtual row
  std::vector<SplitRowRec> rows;   // one per block row
  int64_t groups{};                // workgroups of the partial launch (multiple of kXcds)
  int64_t virtual_rows{};          // workspace rows: the sum over parts of h
  int32_t part_steps{};
};

struct HostSchedule {
  std::vector<StepRec> steps;       // row after row, blocks in row_ptr order
  std::vector<WaveItem> rows;       // kRowWaves per workgroup, launch order for RHS 8 and 16
  std::vector<WaveItem> rows_wide;  // the same workgroups, launch order for RHS 32
  int64_t groups{};                 // workgroups of a launch from rows or rows_wide (multiple of kXcds)
  std::vector<WaveItem> rows_rhs64; // workgroups packed at kPackStepsRhs64, in the rows_wide order, for RHS 64
  int64_t groups_rhs64{};
  // The tile-split kernel's order for RHS 64: every row with k steps a
  // workgroup of its own (empty rows packed kRowWaves to one), placed and
  // chained like the other orders.
  std::vector<WaveItem> rows_tile;
  int64_t groups_tile{};
  // Whether RHS 64 runs the tile-split kernel over rows_tile instead of the
  // split-k kernel over rows_rhs64: a row's steps then run one after another
  // on one workgroup, so the longest row must stay within kTileSpanLimit
  // times the mean steps per workgroup slot.
  bool rhs64_tiles{};
  HostSplitSchedule split;
  // Whether the split-row path pays off for this matrix at RHS 16 and up:
  // the row-owned launch would leave most CUs idle while its rows are long.
  // Advice for the caller (split_row_advised); no plan switches by itself.
  bool split_preferred{};
};

// Step records plus three launch orders of the workgroups.  Rows of at most
// kPackSteps steps (kPackStepsRhs64 for the RHS 64 order) are packed
// kRowWaves to a workgroup (rows of similar work together); every other row
// has a workgroup of its own.  Both orders place
// each workgroup on the XCD whose eighth of the block columns holds most of
// its rows' block widths (so an XCD's B slices concentrate in one eighth of
// B), with equal work per XCD.  Within an XCD, `rows` runs the heaviest
// workgroups first; `rows_wide` and `rows_rhs64` chain the workgroups of the heavier three
// quarters whose rows share block columns and runs the lightest quarter
// after them, heaviest first -- when the matrix has more than 192
// workgroups per XCD; below that it is heaviest first like `rows`.
// Deterministic.
HostSchedule build_schedule(const vbsr_host_view& host);

// ---- device format (device_matrix.cpp) ----------------------------------

// Matrix (vbsr.hpp:41-64): owns device copies of every array plus the row
// schedule.  Immutable after construction.
class DeviceMatrix {
public:
  explicit DeviceMatrix(const vbsr_host_view& host);
  ~DeviceMatrix();
  DeviceMatrix(const DeviceMatrix&) = delete;
  DeviceMatrix& operator=(const DeviceMatrix&) = delete;

  // Device copy of the split-row schedule.
  struct Split {
    const WaveItem* items{};
    const SplitRowRec* rows{};
    int64_t groups{};
    int64_t virtual_rows{};
    bool preferred{};
  };

  const vbsr_device_view& view() const { return view_; }
  const vbsr_row_schedule& schedule() const { return schedule_; }
  const Split& split() const { return split_; }

private:
  vbsr_device_view view_{};
  vbsr_row_schedule schedule_{};
  Split split_{};
  std::vector<void*> allocations_;
  void release() noexcept;
};


// ---- kernels -------------------------------------------------------------

// True for the RHS widths the reference supports (plan.cpp:9-12).
inline bool supported_rhs(int rhs) { return rhs == 8 || rhs == 16 || rhs == 32 || rhs == 64; }

// B (K x rhs) and C (M x rhs) must be float-aligned device pointers whose
// ranges do not overlap: C is written while B is read (the reference's
// __restrict__ contract, row_owned.cu:12-13).  Checked on the host before
// every launch, so a null, misaligned or aliased panel is an invalid
// argument, not a device fault or corrupted output.
inline void check_panels(int64_t scalar_rows, int64_t scalar_cols, const float* b, const float* c, int rhs) {
  if (b == nullptr || c == nullptr) throw std::invalid_argument("B and C must be device pointers");
  const uintptr_t b0 = reinterpret_cast<uintptr_t>(b);
  const uintptr_t c0 = reinterpret_cast<uintptr_t>(c);
  if (b0 % alignof(float) != 0 || c0 % alignof(float) != 0)
    throw std::invalid_argument("B and C must be 4-byte aligned");
  const uintptr_t b1 = b0 + uintptr_t(scalar_cols) * uintptr_t(rhs) * sizeof(float);
  const uintptr_t c1 = c0 + uintptr_t(scalar_rows) * uintptr_t(rhs) * sizeof(float);
  if (b0 < c1 && c0 < b1) throw std::invalid_argument("B and C overlap");
}
inline void check_panels(const vbsr_device_view& a, const float* b, const float* c, int rhs) {
  check_panels(a.scalar_rows, a.scalar_cols, b, c, rhs);
}

// Order-preserving kernel (row_owned_scalar.hip).
void launch_scalar(const vbsr_device_view& a, const float* b, float* c, int rhs, hipStream_t stream);

// Row-owned MFMA kernel (row_owned_mfma.hip).  Launch count: 1 (0 for an
// empty schedule); any K.  B is read through 32-bit buffer offsets within a
// 16-column tile while narrow_b_offsets(a, rhs) holds (K <= 153,391,684 at
// rhs 8, 71,582,785 otherwise), and through 64-bit lane addresses past that
// (the same kernel otherwise; launch_row_owned_wide_b takes that form at any
// K, with bit-identical results).
bool narrow_b_offsets(const vbsr_device_view& a, int rhs);
void launch_row_owned(const vbsr_device_view& a, const vbsr_row_schedule& schedule, const float* b, float* c,
                      int rhs, hipStream_t stream);
void launch_row_owned_wide_b(const vbsr_device_view& a, const vbsr_row_schedule& schedule, const float* b, float* c,
                             int rhs, hipStream_t stream);
// The same kernel with the MFMA tiles replaced by one fmaf per output and k
// (same schedule, loads and LDS staging): the measured alternative to MFMA,
// slower at every width.  Needs narrow_b_offsets(a, rhs).
void launch_row_owned_valu(const vbsr_device_view& a, const vbsr_row_schedule& schedule, const float* b, float* c,
                           int rhs, hipStream_t stream);

// The split-row path: the row-owned kernel over the matrix's split schedule
// into `workspace` (split.virtual_rows * rhs floats), then the fixed-order
// sum of each row's partial slabs into C.  Two launches; the workspace is
// the caller's (a plan's own, or any buffer of at least that size that does
// not overlap B or C).  Any K, as for launch_row_owned.
int64_t split_workspace_floats(const DeviceMatrix::Split& split, int rhs);
// Whether the split-row path is expected to beat the row-owned launch for
// this matrix at this width: the schedule's rule (few row-owned workgroups,
// long rows), at RHS 16 and up only -- at RHS 8 the split was measured 3-7%
// slower at 64 and 128 block rows of degree 16.
inline bool split_row_advised(const DeviceMatrix::Split& split, int rhs) { return split.preferred && rhs >= 16; }
void launch_split_row(const vbsr_device_view& a, const vbsr_row_schedule& schedule, const DeviceMatrix::Split& split,
                      const float* b, float* c, int rhs, float* workspace, int64_t workspace_floats,
                      hipStream_t stream);
// The same with the library's static device scratch (split_scratch_floats()
// floats per device) as the workspace: allocates nothing, and rejects a
// matrix whose workspace would not fit.  Calls on one device share the
// scratch, so calls that overlap in time on one device race.
int64_t split_scratch_floats();
void launch_split_row_static(const vbsr_device_view& a, const vbsr_row_schedule& schedule,
                             const DeviceMatrix::Split& split, const float* b, float* c, int rhs, hipStream_t stream);

// ---- scalar CSR baseline on rocSPARSE (csr_baseline.cpp) ------------------

// The VBSR matrix expanded to scalar CSR in the reference's order
// (cusparse_baseline.cu:35-64): rows in order, blocks in row_ptr order, each
// block's columns ascending.
struct ScalarCsr {
  std::vector<int32_t> row_offsets;  // scalar_rows + 1
  std::vector<int32_t> columns;
  std::vector<float> values;
};
ScalarCsr expand_to_scalar_csr(const vbsr_host_view& host);

}  // namespace vbsr_amd

// rocSPARSE's opaque handle types (rocsparse-types.h), declared here so that
// only csr_baseline.cpp includes rocSPARSE.
typedef struct _rocsparse_handle* rocsparse_handle;
typedef struct _rocsparse_spmat_descr* rocsparse_spmat_descr;
typedef struct _rocsparse_dnmat_descr* rocsparse_dnmat_descr;

namespace vbsr_amd {

// ScalarCsrPlan (reference vbsr.hpp:121-136): device CSR copy plus a
// rocSPARSE SpMM whose dense descriptors and workspace are created at the
// first execute.  Not thread-safe, like the reference's.
class CsrPlan {
public:
  CsrPlan(const vbsr_host_view& host, int rhs);
  ~CsrPlan();
  CsrPlan(const CsrPlan&) = delete;
  CsrPlan& operator=(const CsrPlan&) = delete;
  void execute(const float* b, float* c, hipStream_t stream);
  size_t workspace_bytes() const { return workspace_bytes_; }

private:
  int rhs_{};
  int64_t rows_{}, cols_{}, nnz_{};
  int32_t* row_offsets_{};
  int32_t* columns_{};
  float* values_{};
  void* workspace_{};
  size_t workspace_bytes_{};
  rocsparse_handle handle_{};
  rocsparse_spmat_descr matrix_{};
  rocsparse_dnmat_descr input_{};
  rocsparse_dnmat_descr output_{};
  void release() noexcept;
};

// ---- slot-grouped GEMM baseline on rocBLAS (gemm_baseline.cpp) -------------

}  // namespace vbsr_amd

// rocBLAS's opaque handle type (rocblas-types.h), declared here so that only
// gemm_baseline.cpp includes rocBLAS.
typedef struct _rocblas_handle* rocblas_handle;

namespace vbsr_amd {

// Writes b_pointers[i] = b + b_offset[i] and c_pointers[i] = c + c_offset[i]
// for i < count on `stream` (batch_pointers.hip).
void fill_batch_pointers(const int64_t* b_offset, const int64_t* c_offset, int64_t count, const float* b, float* c,
                         const float** b_pointers, float** c_pointers, hipStream_t stream);

// GroupedGemmPlan (reference vbsr.hpp:138-152): one rocblas_sgemm_batched
// call per (slot, block shape).  Not thread-safe, like the reference's.
class GemmPlan {
public:
  GemmPlan(const vbsr_host_view& host, int rhs);
  ~GemmPlan();
  GemmPlan(const GemmPlan&) = delete;
  GemmPlan& operator=(const GemmPlan&) = delete;
  void execute(const float* b, float* c, hipStream_t stream);
  // Sequential block slots (the reference's launch_count, slot_split.cu:137).
  int launch_count() const { return int(slots_.size()); }

private:
  struct Group {
    int32_t h, w;   // block shape
    int64_t first;  // first entry of the pointer arrays
    int32_t count;  // blocks of this shape in the slot
  };
  int rhs_{};
  int64_t rows_{}, cols_{}, entries_{};
  std::vector<std::vector<Group>> slots_;
  float* values_{};
  const float** a_pointers_{};
  int64_t* b_offset_{};
  int64_t* c_offset_{};
  const float** b_pointers_{};
  float** c_pointers_{};
  rocblas_handle handle_{};
  void release() noexcept;
};

// ---- plan (plan.cpp) -------------------------------------------------------

// Plan (reference plan.cpp:5-31).  A plan on the split-row path owns its
// workspace, allocated here and freed with the plan; execute allocates
// nothing.
class Plan {
public:
  Plan(const DeviceMatrix& matrix, const vbsr_plan_options& options);
  ~Plan();
  Plan(const Plan&) = delete;
  Plan& operator=(const Plan&) = delete;
  void execute(const float* b, float* c, hipStream_t stream) const;
  int launch_count() const;
  bool split_row() const { return split_row_; }

private:
  vbsr_device_view a_{};
  vbsr_row_schedule schedule_{};
  DeviceMatrix::Split split_{};
  vbsr_plan_options options_{};
  bool split_row_{};
  float* workspace_{};
  int64_t workspace_floats_{};
};

}  // namespace vbsr_amd
