/*
 * vbsr.h -- C ABI of the MI355X VBSR SpMM library (libvarblockspmm_amd.so).
 *
 * Computes FP32 C = A * B for a packed variable-block sparse-row matrix A
 * (block heights/widths in {8,16,...,64}, blocks column-major, packed without
 * padding) and dense column-major panels B (K x rhs, ld = K) and
 * C (M x rhs, ld = M), rhs in {8,16,32,64}.
 *
 * This is the drop-in boundary for the reference's C++ API
 * (King-Clawthorne/VarBlockSpMM, include/varblockspmm/vbsr.hpp).  Each entry
 * point names the reference declaration it replaces.  Plain pointers, sizes
 * and status codes only; no C++ exception crosses it.  The C++ mirror of the
 * reference API is include/varblockspmm/vbsr.hpp (header-only, over this ABI).
 *
 * Errors: every function returning int returns VBSR_OK (0),
 * VBSR_INVALID_ARGUMENT (1) where the reference throws std::invalid_argument,
 * or VBSR_RUNTIME_ERROR (2) where it throws std::runtime_error (HIP errors,
 * launch errors, allocation failures).  vbsr_last_error() returns the message
 * of the calling thread's last failure.
 *
 * Execution: vbsr_plan_execute and the launchers only enqueue kernels on the
 * given stream; they never synchronise, never allocate and use no workspace.
 * B (K x N floats) and C (M x N floats) must be non-null, 4-byte aligned and
 * must not overlap; all three are checked on the host before any launch
 * (VBSR_INVALID_ARGUMENT otherwise).  C is fully overwritten.  Results are bit-identical
 * from run to run (no atomics, fixed accumulation order).
 */
#ifndef VARBLOCKSPMM_AMD_VBSR_H
#define VARBLOCKSPMM_AMD_VBSR_H

#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum vbsr_status { VBSR_OK = 0, VBSR_INVALID_ARGUMENT = 1, VBSR_RUNTIME_ERROR = 2 };

/* Host VBSR matrix, field for field the reference HostMatrix
 * (vbsr.hpp:16-29), with each std::vector given as pointer + length. */
typedef struct vbsr_host_view {
  int32_t block_rows, block_cols;
  const int32_t* row_ptr;        int64_t row_ptr_len;        /* block_rows + 1 */
  const int32_t* block_col;      int64_t block_col_len;      /* nnzb */
  const int32_t* row_size;       int64_t row_size_len;       /* block_rows */
  const int32_t* col_size;       int64_t col_size_len;       /* block_cols */
  const int64_t* row_scalar_off; int64_t row_scalar_off_len; /* block_rows + 1 */
  const int64_t* col_scalar_off; int64_t col_scalar_off_len; /* block_cols + 1 */
  const int64_t* value_off;      int64_t value_off_len;      /* nnzb + 1 */
  const float* values;           int64_t values_len;         /* sum h*w */
} vbsr_host_view;

/* Non-owning device view; same fields and meaning as the reference
 * DeviceMatrix (vbsr.hpp:32-38).  All pointers are device pointers. */
typedef struct vbsr_device_view {
  int32_t block_rows, block_cols, nnzb;
  int64_t scalar_rows, scalar_cols;
  const int32_t *row_ptr, *block_col, *row_size, *col_size;
  const int64_t *row_scalar_off, *col_scalar_off, *value_off;
  const float* values;
} vbsr_device_view;

/* Block-size distributions: 0..3 are the reference Distribution enumerators
 * (vbsr.hpp:67; generator.cpp:14-30).  4 and 5 are extensions used by the
 * benchmark configurations: sizes {8,64} with p = 1/2 each, and sizes
 * {8,...,64} with the column partition equal to the row partition. */
enum vbsr_distribution {
  VBSR_DIST_UNIFORM = 0,
  VBSR_DIST_LOW_VARIANCE = 1,
  VBSR_DIST_HIGH_VARIANCE = 2,
  VBSR_DIST_BIMODAL = 3,
  VBSR_DIST_BIMODAL_8_OR_64 = 4,
  VBSR_DIST_TIED_8_TO_64 = 5
};

/* Column patterns: the reference's random and cyclic-local patterns
 * (generator.cpp:62-66; `local_columns`), plus a clamped local pattern:
 * column = clamp(min(i, C-1) + e() % (2d+1) - d, 0, C-1). */
enum vbsr_locality { VBSR_LOCALITY_RANDOM = 0, VBSR_LOCALITY_LOCAL = 1, VBSR_LOCALITY_LOCAL_CLAMPED = 2 };

/* GeneratorOptions (vbsr.hpp:70-76); `locality` replaces the reference's
 * `bool local_columns` (1 == true, 0 == false). */
typedef struct vbsr_generator_options {
  int32_t block_rows, block_cols, degree, rhs_width;
  int32_t distribution; /* enum vbsr_distribution */
  int32_t locality;     /* enum vbsr_locality */
  uint64_t seed;
} vbsr_generator_options;

/* Kernel (vbsr.hpp:91) and PlanOptions (vbsr.hpp:94-97). */
enum vbsr_kernel { VBSR_KERNEL_AUTO = 0, VBSR_KERNEL_ROW_OWNED = 1, VBSR_KERNEL_SPLIT_ROW = 2 };
typedef struct vbsr_plan_options {
  int32_t rhs_width;
  int32_t kernel; /* enum vbsr_kernel */
} vbsr_plan_options;

typedef struct vbsr_host_matrix vbsr_host_matrix; /* owning host matrix (generator output) */
typedef struct vbsr_matrix vbsr_matrix;           /* owning device matrix: reference Matrix */
typedef struct vbsr_plan vbsr_plan;               /* execution plan: reference Plan */

/* Message of the calling thread's most recent failure ("" if none). */
const char* vbsr_last_error(void);

/* HostMatrix::validate (vbsr.hpp:28; vbsr.cpp:29-82): same accept/reject set
 * for every view the reference's vectors can express.  A view can also carry
 * a null array with entries or a negative length; those are rejected
 * (VBSR_INVALID_ARGUMENT), as are scalar/value offset steps whose difference
 * overflows int64. */
int vbsr_validate(const vbsr_host_view* host);

/* generate (vbsr.hpp:80; generator.cpp:7-88): same engine, same draw order,
 * same matrices for the reference's distributions and localities. */
int vbsr_generate(const vbsr_generator_options* options, vbsr_host_matrix** out);
/* Views the arrays of a generated matrix (valid until it is destroyed). */
int vbsr_host_matrix_view(const vbsr_host_matrix* matrix, vbsr_host_view* out);
void vbsr_host_matrix_destroy(vbsr_host_matrix* matrix);

/* The reference test's B generator (tests/test_main.cpp:42-51):
 * std::mt19937{unsigned(seed)} feeding uniform_real_distribution<float>(-1,1)
 * into out[0..count). */
int vbsr_make_random_input(int64_t count, uint64_t seed, float* out);

/* cpu_reference (vbsr.hpp:82-87; vbsr.cpp:167-201): C = A * B on the host,
 * single-threaded, each block's contribution to C[r, n] summed in double over
 * k ascending and added to C in float, blocks in row_ptr order -- the
 * reference's arithmetic, so its results are bit-identical to the
 * reference's.  B holds b_len == scalar_cols * rhs floats and C receives
 * c_len == scalar_rows * rhs floats (column-major, fully overwritten); a
 * wrong size is VBSR_INVALID_ARGUMENT ("B size", as the reference's
 * std::invalid_argument).  Unlike the reference, the matrix is validated
 * first and negative scalar offset starts are rejected, so no invalid view
 * is read out of bounds.  Host memory only; no GPU is used. */
int vbsr_cpu_reference(const vbsr_host_view* host, const float* B, int64_t b_len, int32_t rhs, float* C,
                       int64_t c_len);

/* Matrix(const HostMatrix&) (vbsr.hpp:44; vbsr.cpp:84-113): validates, then
 * copies every array to the current HIP device and builds the row schedule.
 * Additionally rejects (VBSR_INVALID_ARGUMENT) row/col scalar offsets that do
 * not start at 0, which the reference accepts but which would leave C rows
 * unwritten or index outside B and C. */
int vbsr_matrix_create(const vbsr_host_view* host, vbsr_matrix** out);
/* ~Matrix (vbsr.cpp:114-127).  Null is a no-op. */
void vbsr_matrix_destroy(vbsr_matrix* matrix);
/* Matrix::device_view (vbsr.hpp:51; vbsr.cpp:163-166). */
int vbsr_matrix_device_view(const vbsr_matrix* matrix, vbsr_device_view* out);
/* Matrix::scalar_rows / scalar_cols (vbsr.hpp:52-53). */
int64_t vbsr_matrix_scalar_rows(const vbsr_matrix* matrix);
int64_t vbsr_matrix_scalar_cols(const vbsr_matrix* matrix);
/* The matrix's row schedule, built at vbsr_matrix_create: the
 * counterpart of the reference's private row_shape_order and its small/large
 * counts (vbsr.cpp:96-102), which Plan passes to launch_row_owned.  Device
 * arrays owned by the matrix; opaque to callers. */
typedef struct vbsr_row_schedule {
  const void* steps;     /* device: one 16-byte record per k step */
  const void* rows;       /* device: four 48-byte wave items per workgroup, launch order for rhs 8 and 16 */
  int64_t groups;         /* workgroups of a launch from rows or rows_wide */
  int32_t step_limit;     /* index of the last step record */
  const void* rows_wide;  /* device: the same row items, launch order for rhs 32 */
  const void* rows_rhs64; /* device: row items for rhs 64, which packs longer light rows */
  int64_t groups_rhs64;   /* workgroups of a launch from rows_rhs64 */
  const void* rows_tile;  /* device: row items of the rhs 64 tile split, one row per workgroup */
  int64_t groups_tile;    /* workgroups of a launch from rows_tile */
  /* Which kernel an rhs 64 launch runs: 0 the split-k kernel over rows_rhs64
   * (a row's k steps shared by four waves, each with all four 16-column RHS
   * tiles), 1 the tile split over rows_tile (four waves on one row, each
   * with one RHS tile over all the row's steps).  vbsr_matrix_create sets it
   * by the matrix's rule; both kernels are correct for any matrix, so a
   * caller may set either value in its copy of the struct. */
  int32_t rhs64_tiles;
} vbsr_row_schedule;
int vbsr_matrix_row_schedule(const vbsr_matrix* matrix, vbsr_row_schedule* out);

/* Plan(const Matrix&, PlanOptions) (vbsr.hpp:106; plan.cpp:5-18): rejects
 * rhs_width outside {8,16,32,64}.  VBSR_KERNEL_ROW_OWNED runs the row-owned
 * kernel; VBSR_KERNEL_SPLIT_ROW (reserved and rejected in the reference,
 * plan.cpp:13-17) runs the split-row path (vbsr_launch_split_row) with a
 * workspace the plan allocates here and frees when destroyed;
 * VBSR_KERNEL_AUTO runs the row-owned kernel, as the reference's Auto does
 * (docs/design.md:17), so a default plan owns no device memory.  The plan
 * views the matrix, which must outlive it. */
int vbsr_plan_create(const vbsr_matrix* matrix, const vbsr_plan_options* options, vbsr_plan** out);
void vbsr_plan_destroy(vbsr_plan* plan);
/* Plan::execute (vbsr.hpp:110; plan.cpp:19-22): enqueues C = A * B on
 * `stream` (0 = null stream).  Allocates nothing.  A row-owned plan (AUTO,
 * ROW_OWNED) keeps no state, so its executes may run concurrently on any
 * streams.  A split-row plan's executes share its workspace: they must not
 * overlap in time (one stream, or events between streams), and a HIP graph
 * captured from one reads and writes that workspace, so the plan must
 * outlive every replay of the graph. */
int vbsr_plan_execute(const vbsr_plan* plan, const float* B, float* C, hipStream_t stream);
/* Plan::launch_count (vbsr.hpp:112; plan.cpp:23-31): kernels enqueued by one
 * vbsr_plan_execute: 2 on the split-row path, else 1 (0 for a matrix
 * without block rows). */
int vbsr_plan_launch_count(const vbsr_plan* plan);

/* launch_row_owned (vbsr.hpp:158-159; row_owned.cu:397-423): the tuned
 * row-owned kernel for `rhs` over `matrix`, scheduled by `schedule` (from
 * vbsr_matrix_row_schedule of the matrix that `matrix` views; the reference
 * passes row_shape_order/small/large in the same role).  Any K: B is read
 * through 32-bit offsets within a 16-column tile up to K = 153,391,684 at
 * rhs 8 and 71,582,785 otherwise, and through 64-bit lane addresses past
 * that. */
int vbsr_launch_row_owned(const vbsr_device_view* matrix, const vbsr_row_schedule* schedule,
                          const float* B, float* C, int32_t rhs, hipStream_t stream);

/* vbsr_launch_row_owned with B read through 64-bit lane addresses at every
 * K: the form vbsr_launch_row_owned and vbsr_plan_execute take past the
 * 32-bit offset bound, here at any K, so that it can be checked against the
 * offset form (the results are bit-identical: only the addressing differs).
 * No counterpart in the reference. */
int vbsr_launch_row_owned_wide_b(const vbsr_device_view* matrix, const vbsr_row_schedule* schedule,
                                 const float* B, float* C, int32_t rhs, hipStream_t stream);

/* vbsr_launch_row_owned with plain FP32 multiply-adds (one fmaf per output
 * and k, k ascending within each step) in place of the MFMA tiles: the same
 * schedule, loads and LDS staging, within the same tolerance.  No
 * counterpart in the reference; kept as the measured alternative to the
 * MFMA kernel, which is faster at every RHS width (bench.py --kernel valu).
 * Unlike the MFMA kernel, it keeps the 32-bit B offset bound on K
 * (VBSR_INVALID_ARGUMENT past it). */
int vbsr_launch_row_owned_valu(const vbsr_device_view* matrix, const vbsr_row_schedule* schedule,
                               const float* B, float* C, int32_t rhs, hipStream_t stream);

/* The split-row path (the reference's reserved Kernel::SplitRow,
 * vbsr.hpp:91, plan.cpp:13-17).  Each block row's k steps are cut into parts
 * (the matrix's split schedule, built at vbsr_matrix_create); the row-owned
 * kernel computes each part's partial slab into `workspace`, and a second
 * launch sums each row's partial slabs into C in part order.  Results are
 * bit-identical from run to run (fixed order, no atomics) and within the
 * row-owned kernel's tolerance of cpu_reference.  `workspace` is a device
 * buffer of at least vbsr_split_row_workspace_bytes(matrix, rhs) bytes,
 * 4-byte aligned, overlapping neither B nor C, that no other launch uses
 * until this one has finished.  Any K, as for vbsr_launch_row_owned.
 * Two launches; allocates nothing. */
int vbsr_split_row_workspace_bytes(const vbsr_matrix* matrix, int32_t rhs, int64_t* bytes);
/* *advised = 1 when the split-row path is expected to beat the row-owned
 * kernel for this matrix at this rhs, else 0.  The rule: the row-owned
 * launch has fewer than 160 workgroups (most of the 256 CUs idle), its
 * longest row has more than 16 k steps, and rhs >= 16.  Plans never act on
 * it by themselves; a caller that wants the split asks for
 * VBSR_KERNEL_SPLIT_ROW.  No counterpart in the reference. */
int vbsr_matrix_split_row_advised(const vbsr_matrix* matrix, int32_t rhs, int32_t* advised);
int vbsr_launch_split_row(const vbsr_matrix* matrix, const float* B, float* C, int32_t rhs, void* workspace,
                          int64_t workspace_bytes, hipStream_t stream);

/* vbsr_launch_split_row without a workspace argument; no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * partial slabs go to the library's static device scratch, 16 MiB per device
 * (set aside when the library is loaded on the device, held until the
 * process ends), so the call allocates nothing.  A matrix whose workspace
 * (vbsr_split_row_workspace_bytes) exceeds 16 MiB is rejected
 * (VBSR_INVALID_ARGUMENT) before any launch.  Every call on a device shares
 * that device's scratch: calls that overlap in time on one device race, so
 * serialise them (one stream, or events).  Results are bit-identical to
 * vbsr_launch_split_row's. */
int vbsr_launch_split_row_static(const vbsr_matrix* matrix, const float* B, float* C, int32_t rhs,
                                 hipStream_t stream);

/* launch_row_owned_scalar (vbsr.hpp:161; row_owned.cu:376-395): one output
 * per lane, accumulated with fmaf over blocks in row_ptr order and k
 * ascending from 0 -- the reference kernels' exact order, so its results are
 * bit-identical to theirs. */
int vbsr_launch_row_owned_scalar(const vbsr_device_view* matrix, const float* B, float* C,
                                 int32_t rhs, hipStream_t stream);

/* ScalarCsrPlan (vbsr.hpp:121-136; cusparse_baseline.cu:35-188): the
 * library baseline, on rocSPARSE.  vbsr_csr_plan_create validates the host
 * matrix (and, like vbsr_matrix_create, requires scalar offsets that start at
 * 0), expands it to scalar CSR in the reference's order (rows, then blocks in
 * row_ptr order, then columns) and copies that to the current HIP device;
 * it rejects rhs outside {8,16,32,64} and matrices of 2^31 or more stored
 * values (32-bit CSR indices).  vbsr_csr_plan_execute enqueues C = A * B with
 * rocsparse_spmm (default algorithm); the first call also creates the dense
 * descriptors and allocates the workspace, which later calls reuse.  Not
 * thread-safe, like the reference's baseline plans (README.md:88). */
typedef struct vbsr_csr_plan vbsr_csr_plan;
int vbsr_csr_plan_create(const vbsr_host_view* host, int32_t rhs, vbsr_csr_plan** out);
void vbsr_csr_plan_destroy(vbsr_csr_plan* plan);
int vbsr_csr_plan_execute(vbsr_csr_plan* plan, const float* B, float* C, hipStream_t stream);
/* ScalarCsrPlan::workspace_bytes (vbsr.hpp:131-132): bytes of workspace
 * allocated by the first execute (0 before it, and for a null plan). */
int64_t vbsr_csr_plan_workspace_bytes(const vbsr_csr_plan* plan);

/* GroupedGemmPlan (vbsr.hpp:138-152; slot_split.cu:22-145): the slot-grouped
 * library baseline, on rocBLAS.  Slot s holds the s-th block of every block
 * row; within a slot, blocks are grouped by (h, w).  vbsr_gemm_plan_create
 * validates the host matrix (scalar offsets must start at 0), rejects rhs
 * outside {8,16,32,64} and copies the packed values to the current HIP
 * device.  vbsr_gemm_plan_execute zeroes C and runs the slots in order, one
 * rocblas_sgemm_batched call per (slot, shape) group (rocBLAS has no grouped
 * batched GEMM).  Not thread-safe, like the reference's baseline plans. */
typedef struct vbsr_gemm_plan vbsr_gemm_plan;
int vbsr_gemm_plan_create(const vbsr_host_view* host, int32_t rhs, vbsr_gemm_plan** out);
void vbsr_gemm_plan_destroy(vbsr_gemm_plan* plan);
int vbsr_gemm_plan_execute(vbsr_gemm_plan* plan, const float* B, float* C, hipStream_t stream);
/* GroupedGemmPlan::launch_count (vbsr.hpp:146-147): the number of block
 * slots, i.e. the largest block-row degree (0 for a null plan). */
int vbsr_gemm_plan_launch_count(const vbsr_gemm_plan* plan);

/* cusparse_scalar_baseline (vbsr.hpp:163-165; cusparse_baseline.cu:183-188):
 * one-shot and synchronising -- builds a ScalarCsrPlan for `host`, executes
 * it on `stream`, waits for the stream and releases the plan.  Same checks
 * and errors as vbsr_csr_plan_create / _execute.  Prefer the plan for
 * repeated work. */
int vbsr_scalar_csr_baseline(const vbsr_host_view* host, const float* B, float* C, int32_t rhs,
                             hipStream_t stream);
/* slot_split_baseline (vbsr.hpp:166-168; slot_split.cu:147-152): the same,
 * one-shot and synchronising, with a GroupedGemmPlan. */
int vbsr_slot_split_baseline(const vbsr_host_view* host, const float* B, float* C, int32_t rhs,
                             hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
