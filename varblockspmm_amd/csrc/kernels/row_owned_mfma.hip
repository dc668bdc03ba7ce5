// Row-owned MFMA kernel: the MI355X kernel behind Plan::execute, the
// counterpart of the reference's tuned row-owned family
// (src/kernels/row_owned.cu:47-310, dispatched at 397-423).
//
// Work unit.  One workgroup (4 waves) owns one block row of height h and
// writes its h x RHS slab of C; nothing else writes it, so there are no
// atomics and no global workspace.  The row's k steps (16 k of one block, or
// the 8 k that end a block whose width is 8 mod 16) are dealt to the four
// waves in runs of kRun consecutive steps; each wave accumulates all T =
// ceil(h/16) row tiles for its steps, and the four partial slabs are summed
// in LDS in a fixed order, (w0 + w2) + (w1 + w3).  Every A line and every B
// line of the row is therefore requested by one wave only, with both halves
// of each 128-byte line in adjacent loads, and the accumulation order depends
// only on the matrix, so results are bit-identical from run to run.
//
// Arithmetic.  v_mfma_f32_16x16x4_f32 on transposed 16x16 output tiles,
//   D[n][r] = sum_k B[k, n0 + n] * A[16t + r, k],
// lane 16*g + x supplies src0 = B[k, n0 + x] and src1 = A[16t + x, k] for the
// k that lane group g holds, and result register v of lane 16*g + x is
// C[16t + x, n0 + 4*g + v]: 16 lanes store 64 consecutive bytes of a C column.
// Output column r of a tile depends only on src1 lanes with x == r, and
// output row n only on src0 lanes with x == n, so lanes beyond the last
// tile's rows (h = 8, 24, 40, 56) or beyond RHS (rhs 8) may hold any value:
// their results are never stored.  They load duplicate in-bounds addresses
// instead of branching.
//
// k steps.  Every step loads, per lane and tile, A[r, k0 + 4*j + i]
// (i = 0..3) and one 16-byte B[k0 + 4*j .. k0 + 4*j + 3, n] per 16-column
// RHS tile, with j = g for a full step and j = g & 1 for a half step; MFMA i
// takes element i.  In a half step lane groups 2-3 repeat the k of groups
// 0-1 and are dead: they feed 0 * 0, so each k enters once and non-finite
// inputs reach C exactly as in the reference.  Every step issues the same
// loads and MFMAs, so the loop has no branch but its back edge.
//
// Memory.  A and B are read with raw buffer loads: per block, one buffer
// resource for the block payload (exact byte bounds) and one per RHS tile for
// the B slice; the k offset of A rides in the scalar offset.  Loads run
// kDepth - 1 steps ahead of the MFMAs through a register ring; past a wave's
// last step the ring re-loads that step, whose lanes are all dead.  Block
// descriptors are read once per chunk of 64 blocks (lane j holds block j) and
// broadcast with v_readlane.
#include <hip/hip_runtime.h>

#include "../internal.hpp"

#ifndef VBSR_RING_DEPTH
#define VBSR_RING_DEPTH 2
#endif
#ifndef VBSR_STEP_RUN
#define VBSR_STEP_RUN 2
#endif

namespace vbsr_amd {
namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));
using rsrc_t = __amdgpu_buffer_rsrc_t;

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kMaxTiles = 4;  // h <= 64
constexpr int kDepth = VBSR_RING_DEPTH;
constexpr int kRun = VBSR_STEP_RUN;
constexpr int64_t kOffsetMask = (int64_t(1) << kWidthShift) - 1;
// Buffer resource word 3 for raw (unformatted, unswizzled) dword access.
constexpr int kRawBufferFlags = 0x00020000;
static_assert(kDepth >= 1 && kDepth <= 6, "ring depth");
static_assert(kRun >= 1, "step run");

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ int64_t lane_value(int64_t v, int lane) {
  const int lo = __builtin_amdgcn_readlane(int(uint32_t(uint64_t(v))), lane);
  const int hi = __builtin_amdgcn_readlane(int(uint32_t(uint64_t(v) >> 32)), lane);
  return int64_t((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

__device__ __forceinline__ rsrc_t make_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), short(0), int(bytes), kRawBufferFlags);
}

template <int RHS>
constexpr int rhs_tiles() {
  return RHS < 16 ? 1 : RHS / 16;
}

template <int RHS, int T>
struct Step {
  float a[T][4];
  f32x4 b[rhs_tiles<RHS>()];
  bool half;
};

template <int RHS>
struct Shared {
  f32x4 partial[2][kMaxTiles * rhs_tiles<RHS>()][kWave];
};

// The steps of one chunk owned by `wave`: runs r = wave, wave + 4, ... of kRun
// steps each, the last run possibly short.
__device__ __forceinline__ int owned_steps(int steps, int wave) {
  const int full = steps / kRun;
  const int rest = steps % kRun;
  const int full_owned = full > wave ? (full - wave + kWaves - 1) / kWaves : 0;
  return full_owned * kRun + ((rest > 0 && full % kWaves == wave) ? rest : 0);
}

template <int RHS, int T>
__device__ __forceinline__ void row_body(const vbsr_device_view& a, const RowItem& item, const BlockDesc* blocks,
                                         const float* b, float* c, Shared<RHS>& shared, int wave, int lane) {
  constexpr int kRhsTiles = rhs_tiles<RHS>();
  constexpr int kRhsLanes = RHS < 16 ? RHS : 16;
  const int group = lane >> 4;
  const int x = lane & 15;
  const bool upper = group >= 2;
  const int h = uniform(item.h);
  const int nblocks = uniform(item.nblocks);
  const int first = uniform(item.first);
  const int last_rows = h - 16 * (T - 1);  // 8 or 16
  const uint32_t ldb = uint32_t(a.scalar_cols);

  // Per-lane byte offsets.  Rows past h and rhs columns past RHS read a
  // duplicate in-bounds address.
  uint32_t a_row[T];
#pragma unroll
  for (int t = 0; t < T; ++t) a_row[t] = uint32_t(16 * t + (t == T - 1 ? (x & (last_rows - 1)) : x)) * 4u;
  const uint32_t a_full = uint32_t(4 * group * h) * 4u;
  const uint32_t a_half = uint32_t(4 * (group & 1) * h) * 4u;
  const uint32_t b_row = uint32_t(x & (kRhsLanes - 1)) * ldb * 4u;
  const uint32_t b_full = uint32_t(4 * group) * 4u;
  const uint32_t b_half = uint32_t(4 * (group & 1)) * 4u;
  const uint32_t a_stride = uint32_t(h) * 4u;                   // bytes between columns of a block
  const uint32_t b_span = (uint32_t(kRhsLanes - 1) * ldb) * 4u;  // bytes of a B tile past its first column

  f32x4 acc[T][kRhsTiles];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int nt = 0; nt < kRhsTiles; ++nt) acc[t][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int chunk = 0; chunk < nblocks; chunk += kWave) {
    const int count = min(kWave, nblocks - chunk);
    const BlockDesc desc = blocks[first + chunk + min(lane, count - 1)];
    const int w_lane = int(uint64_t(desc.b_off) >> kWidthShift);
    int steps = 0;
    for (int j = 0; j < count; ++j) steps += (__builtin_amdgcn_readlane(w_lane, j) + 8) >> 4;
    const int mine = owned_steps(steps, wave);
    if (mine == 0) continue;

    // Load stream: global step `s` = block `lb` at k offset `lk`.
    int s = 0, lb = 0, lk = 0, w = 0, issued = 0;
    rsrc_t a_rsrc;
    rsrc_t b_rsrc[kRhsTiles];
    auto enter_block = [&](int blk) {
      const int64_t a_off = lane_value(desc.a_off, blk);
      const int64_t bw = lane_value(desc.b_off, blk);
      w = int(bw >> kWidthShift);
      a_rsrc = make_rsrc(a.values + a_off, uint32_t(h * w) * 4u);
      const float* b_base = b + (bw & kOffsetMask);
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt)
        b_rsrc[nt] = make_rsrc(b_base + int64_t(nt) * 16 * ldb, b_span + uint32_t(w) * 4u);
    };
    auto next_step = [&]() {
      lk += (w - lk) == 8 ? 8 : 16;
      if (lk >= w) {
        lk = 0;
        enter_block(++lb);
      }
      ++s;
    };
    enter_block(0);
    while ((s / kRun) % kWaves != wave) next_step();

    Step<RHS, T> ring[kDepth];
    auto issue = [&](Step<RHS, T>& st) {
      const bool half = (w - lk) == 8;
      const uint32_t va = half ? a_half : a_full;
      const uint32_t vb = b_row + (half ? b_half : b_full);
      const int ka = lk * int(a_stride);
      // The buffer-load builtins return raw bits (u32 / u32x4): bit-cast them.
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          st.a[t][i] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(a_rsrc, int(a_row[t] + va), ka + i * int(a_stride), 0));
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt)
        st.b[nt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc[nt], int(vb), lk * 4, 0));
      st.half = half;
      if (issued + 1 < mine) {
        ++issued;
        do next_step();
        while ((s / kRun) % kWaves != wave);
      }
    };
    // Branch-free: a dead lane feeds 0 * 0 and every step runs the same MFMAs.
    auto compute = [&](const Step<RHS, T>& st, bool live) {
      const bool dead = !live || (st.half && upper);
      f32x4 bv[kRhsTiles];
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) bv[nt][i] = dead ? 0.0f : st.b[nt][i];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float av = dead ? 0.0f : st.a[t][i];
#pragma unroll
          for (int nt = 0; nt < kRhsTiles; ++nt)
            acc[t][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[nt][i], av, acc[t][nt], 0, 0, 0);
        }
    };

#pragma unroll
    for (int k = 0; k < kDepth - 1; ++k) issue(ring[k]);
    for (int j = 0; j < mine; j += kDepth) {
#pragma unroll
      for (int u = 0; u < kDepth; ++u) {
        issue(ring[(u + kDepth - 1) % kDepth]);
        compute(ring[u], j + u < mine);
      }
    }
  }

  // Fixed-order reduction of the four partial slabs: (w0 + w2) + (w1 + w3).
  if (wave >= 2) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) shared.partial[wave - 2][t * kRhsTiles + nt][lane] = acc[t][nt];
  }
  __syncthreads();
  if (wave < 2) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) acc[t][nt] += shared.partial[wave][t * kRhsTiles + nt][lane];
  }
  __syncthreads();
  if (wave == 1) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) shared.partial[0][t * kRhsTiles + nt][lane] = acc[t][nt];
  }
  __syncthreads();
  if (wave != 0) return;
  const int64_t ldc = a.scalar_rows;
  float* c_row = c + item.c_off + x;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t < T - 1 || x < last_rows) {
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) {
        const f32x4 sum = acc[t][nt] + shared.partial[0][t * kRhsTiles + nt][lane];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int n = nt * 16 + 4 * group + v;
          if (n < RHS) c_row[16 * t + int64_t(n) * ldc] = sum[v];
        }
      }
    }
  }
}

template <int RHS>
__global__ __launch_bounds__(kThreads) void row_owned_mfma_kernel(vbsr_device_view a, const RowItem* __restrict__ rows,
                                                                  const BlockDesc* __restrict__ blocks,
                                                                  const float* __restrict__ b, float* __restrict__ c) {
  __shared__ Shared<RHS> shared;
  const int wave = uniform(int(threadIdx.x) / kWave);
  const int lane = int(threadIdx.x) % kWave;
  const RowItem item = rows[blockIdx.x];
  if (uniform(item.nblocks) < 0) return;  // padding slot: the whole workgroup leaves
  switch ((uniform(item.h) + 15) >> 4) {
  case 1: row_body<RHS, 1>(a, item, blocks, b, c, shared, wave, lane); break;
  case 2: row_body<RHS, 2>(a, item, blocks, b, c, shared, wave, lane); break;
  case 3: row_body<RHS, 3>(a, item, blocks, b, c, shared, wave, lane); break;
  default: row_body<RHS, 4>(a, item, blocks, b, c, shared, wave, lane); break;
  }
}

template <int RHS>
void launch(const vbsr_device_view& a, const vbsr_row_schedule& s, const float* b, float* c, hipStream_t stream) {
  row_owned_mfma_kernel<RHS><<<dim3(unsigned(s.groups)), dim3(kThreads), 0, stream>>>(
      a, static_cast<const RowItem*>(s.rows), static_cast<const BlockDesc*>(s.blocks), b, c);
}

}  // namespace

bool row_owned_supported(const vbsr_device_view& a, const float* b) {
  // 32-bit buffer offsets: a B tile spans 15 columns of ld K plus one block.
  return reinterpret_cast<uintptr_t>(b) % 16 == 0 && a.scalar_cols < (int64_t(1) << 26);
}

void launch_row_owned(const vbsr_device_view& a, const vbsr_row_schedule& s, const float* b, float* c, int rhs,
                      hipStream_t stream) {
  if (!supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
  if (!row_owned_supported(a, b))
    throw std::invalid_argument("row-owned kernel needs a 16-byte aligned B and fewer than 2^26 scalar columns");
  if (s.groups <= 0) return;
  if (s.groups > int64_t(0x7fffffff)) throw std::invalid_argument("schedule too large for one launch");
  switch (rhs) {
  case 8: launch<8>(a, s, b, c, stream); break;
  case 16: launch<16>(a, s, b, c, stream); break;
  case 32: launch<32>(a, s, b, c, stream); break;
  default: launch<64>(a, s, b, c, stream); break;
  }
  check_hip(hipGetLastError(), "row_owned_mfma launch");
}

}  // namespace vbsr_amd
