// Row-owned MFMA kernel: the MI355X kernel behind Plan::execute, the
// counterpart of the reference's tuned row-owned family
// (src/kernels/row_owned.cu:47-310, dispatched at 397-423).
//
// Work unit.  One workgroup (4 waves) owns one block row of height h and
// writes its h x RHS slab of C, or owns up to four light rows, one per wave
// (the schedule packs rows of at most kPackSteps k steps, kPackStepsRhs64 at
// RHS 64); nothing else writes those slabs, so there are no atomics and no
// global workspace.  A
// row's k steps (16 columns of one block, or the 8 that end a block whose
// width is 8 mod 16; one precomputed record each) are dealt to the waves
// that share it -- four, in runs of two, or a packed row's one wave; each
// wave accumulates all T = ceil(h/16) row tiles for its steps.  The four
// partial slabs of a shared row are summed in LDS in a fixed order,
// (w0 + w2) + (w1 + w3): at RHS 16 and 32 by wave 0 after one barrier, at
// RHS 8 and 64 in pairs over three barriers.  A packed row's wave stores its
// sums itself.  The accumulation order depends only on the matrix, so
// results are bit-identical from run to run.
//
// Arithmetic.  v_mfma_f32_16x16x4_f32 on transposed 16x16 output tiles,
//   D[n][r] = sum_k B[k, n0 + n] * A[16t + r, k],
// lane 16*g + x supplies src0 = B[k, n0 + x] and src1 = A[16t + x, k] with
// k = k0 + 4*g + i for MFMA i, and result register v of lane 16*g + x is
// C[16t + x, n0 + 4*g + v]: 16 lanes store 64 consecutive bytes of a C column.
// Output column r of a tile depends only on src1 lanes with x == r, and
// output row n only on src0 lanes with x == n, so lanes beyond the last
// tile's rows (h = 8, 24, 40, 56) or beyond RHS (rhs 8) may hold any value:
// their results are never stored.
//
// Memory.  A and B are read with raw buffer loads whose resources cover
// exactly one step: the step's 16 (or 8) columns of the block, and the
// step's k range of each B column.  Lanes that must contribute nothing get
// zeros from the hardware range check instead of from extra instructions:
// in a half step A columns 8-15 lie past the 8-column resource and the B
// lanes holding k0 + 8 .. k0 + 15 use an offset past every resource (so do
// the B lanes of columns 8-15 at RHS 8); a step beyond a wave's last one gets
// zero-byte resources.  Those lanes therefore
// feed 0 * 0, so each k enters once and non-finite inputs reach C exactly as
// in the reference.  B's offsets within a 16-column tile are 32-bit; past
// that bound on K (narrow_b_offsets) the kWideB instantiation reads B at the
// same addresses through 64-bit lane pointers, and the lanes the range check
// would zero skip the load instead (bit-identical, 3-9% slower).
//
// A step's A tile is 16 contiguous block columns (64 h bytes).  It is read
// whole, 16 bytes per lane and 1 KB per load, with the non-temporal hint:
// every load covers whole 128-byte lines, and A, which is read exactly once,
// does not displace B from L2.  The tile goes through the wave's LDS slot,
// stored column-major with a leading dimension of 16 T + 4 floats so that the
// MFMA-layout reads hit 64 distinct banks.  B is loaded four lanes per column
// (each quarter reads 64 contiguous bytes of four columns), written to the
// wave's B slot and read back in MFMA layout; that slot is XOR-swizzled so
// that both the 16-byte writes and reads are free of bank conflicts.
//
// At RHS 8, rows of 56 or 64 (four row tiles) skip the LDS round trip for A:
// row tile t of lane x holds row 4 x + t instead of 16 t + x, so the lane's
// four rows of block column 4 g + i are 16 contiguous bytes, read by load i
// straight into MFMA layout; lanes past h (h = 56) hold values of the next
// column, which only reach output rows that are never stored.  That frees
// the registers that address the A slot, and RHS 8 runs 6 waves per SIMD
// instead of 5 (about 2% faster); at the other widths the same path is not
// faster and the A slot stays.
//
// Pipeline.  A wave's step records are read with one load (lane j holds its
// j-th step); its first step's record also comes with its work item, so that
// step's loads are issued without waiting for that load.  Two register
// stages alternate: the loads of step j + 1 are in flight while step j
// computes.  All lane offsets are per-row constants, so
// a step costs its loads, its buffer resources, its LDS round trip and its
// MFMAs.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../internal.hpp"

namespace vbsr_amd {
namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));
// The same vector at float alignment: B and C panels need only be 4-byte
// aligned.  gfx950 serves 16-byte global and buffer accesses at any 4-byte
// aligned address (ROCm runs it in unaligned access mode, and the compiler
// itself merges adjacent 4-byte accesses into them).
typedef float f32x4_unaligned __attribute__((ext_vector_type(4), aligned(4)));
using rsrc_t = __amdgpu_buffer_rsrc_t;

constexpr int kWave = 64;
constexpr int kWaves = kRowWaves;
constexpr int kThreads = kWave * kWaves;
constexpr int kMaxTiles = 4;  // h <= 64
constexpr int kRun = kStepRun;  // consecutive steps dealt to one wave
constexpr int64_t kOffsetMask = kHalfStep - 1;
// Buffer resource word 3 for raw (unformatted, unswizzled) dword access.
constexpr int kRawBufferFlags = 0x00020000;
// A buffer offset past the end of every resource: its loads return zeros.
constexpr uint32_t kOutOfRange = 0xfffffff0u;
// Cache policy of the A loads: non-temporal (streamed, read once).
constexpr int kNonTemporal = 2;

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

// The VALU variant's k-major B slot: floats per k of one RHS tile (16
// columns and 4 of padding, so that the transposing writes of lanes 4 n + q
// land in 64 distinct banks).
constexpr int kValuBLd = 20;

// LDS of one workgroup: one area per wave holding its B slot and its A slot.
// The reduction's partial slabs reuse the areas of the waves that leave
// them (their main loops are over by then), which are sized for them.
// kValu: the VALU variant's B slot is k-major with 20 floats per k (1280
// bytes per RHS tile), and its A slot always holds four tiles.
template <int RHS, bool kValu>
struct Lds {
  static constexpr int kBBytes = rhs_tiles<RHS>() * (kValu ? 16 * kValuBLd * 4 : kWave * 16);
  // Row tiles that go through the A slot: at RHS 8 the MFMA path reads
  // four-tile rows straight into registers.
  static constexpr int kSlotTiles = RHS == 8 && !kValu ? kMaxTiles - 1 : kMaxTiles;
  static constexpr int kABytes = 16 * (16 * kSlotTiles + 4) * 4;
  static constexpr int kSlotBytes = kBBytes + kABytes;
  static constexpr int kPartialBytes = kMaxTiles * rhs_tiles<RHS>() * kWave * 16;
  static constexpr int kBigBytes = kSlotBytes > kPartialBytes ? kSlotBytes : kPartialBytes;
  // RHS 16 and 32 reduce in one barrier through the areas of waves 1-3, so
  // those three are sized for a partial slab; RHS 8 and 64 reduce in three
  // barriers through the areas of waves 2 and 3 (at RHS 64 a third large
  // area would cost a workgroup per CU; at RHS 8 the one-barrier sum costs
  // registers without a measurable gain).
  static constexpr bool kOneBarrier = RHS == 16 || RHS == 32;
  static constexpr int kSmall = kOneBarrier ? 1 : 2;  // areas that hold a slot only
  static constexpr int kTotal = kSmall * kSlotBytes + (kWaves - kSmall) * kBigBytes;
  static __device__ __forceinline__ int area(int wave) {
    return wave < kSmall ? wave * kSlotBytes : kSmall * kSlotBytes + (wave - kSmall) * kBigBytes;
  }
};

// Position, within a wave's 1 KB B slot of one RHS tile, of the 16 bytes
// B[k0 + 4q .. k0 + 4q + 3, n0 + n]: column-major with the four 16-byte
// pieces of column n permuted by an XOR of n's bits 1-2.  Writers (lane
// 4n + q) and readers (lane 16q + n) then each cover all banks.
__device__ __forceinline__ int b_slot_index(int n, int q) {
  return n * 4 + ((q ^ (n >> 1) ^ (n >> 2)) & 3);
}

// Steps of a segment dealt to the lead-th of the 2^shift waves sharing a row:
// runs r = lead, lead + 2^shift, ... of kRun steps each, the last run
// possibly short.
__device__ __forceinline__ int owned_steps(int count, int lead, int shift) {
  const int full = count / kRun;
  const int rest = count % kRun;
  const int full_owned = full > lead ? (full - lead + (1 << shift) - 1) >> shift : 0;
  return full_owned * kRun + ((rest > 0 && (full & ((1 << shift) - 1)) == lead) ? rest : 0);
}

// Index within its segment of the wave's j-th step.
__device__ __forceinline__ int owned_step(int j, int lead, int shift) {
  return (((j / kRun) << shift) + lead) * kRun + j % kRun;
}

// One step's operands as loaded: A load q holds floats 256 q + 4 lane .. + 3
// of the step's column-major tile (or, on the direct path, rows 4 x .. 4 x + 3
// of block column 4 g + q).
template <int RHS, int T>
struct Stage {
  f32x4 a[T];
  f32x4 b[rhs_tiles<RHS>()];
};

struct Launch {
  vbsr_device_view a;
  const StepRec* steps;
  const WaveItem* items;  // kWaves per workgroup
  int32_t step_limit;     // index of the last StepRec
  const float* b;
  float* c;
  int64_t ldc;  // C's leading dimension: scalar_rows, or a split-row workspace's virtual rows
};

// Fixed-order reduction of the four partial slabs of a shared row,
// (w0 + w2) + (w1 + w3), after every wave's main loop.  Afterwards wave 0's
// acc holds the row's sums; returns true for wave 0 only.  The whole
// workgroup shares the row, so every wave reaches the barriers.
template <int RHS, int T, bool kValu>
__device__ __forceinline__ bool reduce_partials(f32x4 (&acc)[T][rhs_tiles<RHS>()], char* lds, int wave, int lane) {
  using Layout = Lds<RHS, kValu>;
  constexpr int kRhsTiles = rhs_tiles<RHS>();
  f32x4* part1 = reinterpret_cast<f32x4*>(lds + Layout::area(1));
  f32x4* part2 = reinterpret_cast<f32x4*>(lds + Layout::area(2));
  f32x4* part3 = reinterpret_cast<f32x4*>(lds + Layout::area(3));
  auto slab = [&](int t, int nt) { return (t * kRhsTiles + nt) * kWave + lane; };
  if constexpr (Layout::kOneBarrier) {
    // Waves 1-3 leave their slabs in their own LDS areas; wave 0 sums them.
    if (wave > 0) {
      f32x4* part = wave == 1 ? part1 : wave == 2 ? part2 : part3;
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int nt = 0; nt < kRhsTiles; ++nt) part[slab(t, nt)] = acc[t][nt];
    }
    __syncthreads();
    if (wave != 0) return false;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt)
        acc[t][nt] = (acc[t][nt] + part2[slab(t, nt)]) + (part1[slab(t, nt)] + part3[slab(t, nt)]);
  } else {
    // Waves 2 and 3 leave their slabs; waves 0 and 1 add them; wave 1 passes
    // its sum to wave 0 through wave 2's area.
    if (wave >= 2) {
      f32x4* part = wave == 2 ? part2 : part3;
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int nt = 0; nt < kRhsTiles; ++nt) part[slab(t, nt)] = acc[t][nt];
    }
    __syncthreads();
    if (wave < 2) {
      const f32x4* part = wave == 0 ? part2 : part3;
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int nt = 0; nt < kRhsTiles; ++nt) acc[t][nt] += part[slab(t, nt)];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int nt = 0; nt < kRhsTiles; ++nt) part2[slab(t, nt)] = acc[t][nt];
    }
    __syncthreads();
    if (wave != 0) return false;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) acc[t][nt] += part2[slab(t, nt)];
  }
  return true;
}

// One k step of the VALU variant: B goes into the k-major slot (lane 4 n + q
// holds B[k0 + 4 q + e, n0 + n], e < 4), then lane (g, x) accumulates rows
// 16 t + x of RHS columns [g * RHS / 4, (g + 1) * RHS / 4) with one fmaf per
// output and k, k ascending: 16 T RHS / 4 multiply-adds per lane per step,
// on the same A slot as the MFMA path.  The 16 lanes of a group read the
// same B address (a broadcast) and 16 consecutive A rows.
template <int RHS, int T>
__device__ __forceinline__ void valu_step(const f32x4 (&b)[rhs_tiles<RHS>()], float* bk, const float* a_slot,
                                          f32x4 (&acc)[T][rhs_tiles<RHS>()], int group, int x, int b_n, int b_q,
                                          int last_rows) {
  constexpr int kRhsTiles = rhs_tiles<RHS>();
  constexpr int ld = 16 * T + 4;
  constexpr int kTile = 16 * kValuBLd;
#pragma unroll
  for (int nt = 0; nt < kRhsTiles; ++nt)
#pragma unroll
    for (int e = 0; e < 4; ++e) bk[nt * kTile + (4 * b_q + e) * kValuBLd + b_n] = b[nt][e];
  constexpr int kCols = RHS / 4;
  const int tile = (group * kCols) / 16;
  const int n0 = (group * kCols) % 16;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    float bv[kCols];
    if constexpr (kCols >= 4) {
#pragma unroll
      for (int j = 0; j < kCols; j += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(bk + (tile + j / 16) * kTile + k * kValuBLd + (n0 + j) % 16);
        bv[j] = v[0];
        bv[j + 1] = v[1];
        bv[j + 2] = v[2];
        bv[j + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int j = 0; j < kCols; ++j) bv[j] = bk[tile * kTile + k * kValuBLd + n0 + j];
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float av = t < T - 1 ? a_slot[k * ld + 16 * t + x] : a_slot[k * ld + 16 * (T - 1) + (x & (last_rows - 1))];
#pragma unroll
      for (int j = 0; j < kCols; ++j) acc[t][j / 4][j % 4] = __builtin_fmaf(av, bv[j], acc[t][j / 4][j % 4]);
    }
  }
}

// kWideB: B is addressed with 64-bit lane pointers instead of 32-bit buffer
// offsets, for K past the offset bound (narrow_b_offsets); lanes that must
// contribute nothing skip the load and hold zeros.
template <int RHS, int T, bool kValu, bool kWideB>
__device__ __forceinline__ void row_body(const Launch& L, const WaveItem& item, char* lds, int wave, int lane) {
  using Layout = Lds<RHS, kValu>;
  constexpr int kRhsTiles = rhs_tiles<RHS>();
  constexpr int kRhsLanes = RHS < 16 ? RHS : 16;
  constexpr int ld = 16 * T + 4;  // A slot: float (r, k) of the step at k * ld + r
  const int group = lane >> 4;
  const int x = lane & 15;
  const int h = uniform(item.h);
  const int count = uniform(item.step_count);
  const int first = uniform(item.step_first);
  // The row is shared by all kWaves waves (lead = wave) or is this wave's own.
  const bool shared = uniform(item.group) > 1;
  const int lead = shared ? wave : 0;
  const int shift = shared ? 2 : 0;
  static_assert(kWaves == 4, "a shared row is dealt to 2^2 waves");
  const int last_rows = h - 16 * (T - 1);  // 8 or 16
  const uint32_t ldb = uint32_t(L.a.scalar_cols);

  char* area = lds + Layout::area(wave);
  f32x4* b_slot = reinterpret_cast<f32x4*>(area);
  float* a_slot = reinterpret_cast<float*>(area + Layout::kBBytes);
  constexpr bool kDirect = !kValu && RHS == 8 && T == kMaxTiles;  // A straight into MFMA layout
  static_assert(kDirect || T <= Layout::kSlotTiles, "the A slot holds the rows that use it");
  // Direct path: load i of lane 16 g + x reads rows 4 x .. 4 x + 3 of block
  // column 4 g + i.
  const int a_direct = (4 * group * h + 4 * x) * 4;

  // A slot positions of this lane's loaded floats.  Lanes past the tile
  // (h = 8 mod 16) hold zeros and write them to the slot's padding (rows
  // 16 T .. 16 T + 3 of column lane & 15), which is never read.
  // f / h is computed as (f * ceil(2^16 / h)) >> 16, which is exact for
  // f < 1024 and h a multiple of 8 up to 64 (one uniform division per row
  // instead of T per lane).
  const uint32_t h_recip = uint32_t(uniform(int((65536u + uint32_t(h) - 1u) / uint32_t(h))));
  int a_write[T];
#pragma unroll
  for (int q = 0; q < T; ++q) {
    const int f = 256 * q + 4 * lane;
    const int k = int((uint32_t(f) * h_recip) >> 16);
    a_write[q] = f < 16 * h ? k * ld + (f - k * h) : (lane & 15) * ld + 16 * T;
  }
  // MFMA-layout reads: row 16 t + x of column 4 g + i; rows past h read a
  // duplicate row.
  const int a_read = 4 * group * ld + x;
  const int a_read_last = 4 * group * ld + 16 * (T - 1) + (x & (last_rows - 1));
  const uint32_t a_full_bytes = uint32_t(16 * h) * 4u;
  const uint32_t a_half_bytes = uint32_t(8 * h) * 4u;

  // B load layout: lane 4n + q reads B[k0 + 4q .. k0 + 4q + 3, n0 + n] (at
  // RHS 8 the lanes of columns 8-15 read nothing, and in a half step q = 2, 3
  // read nothing: those lanes hold zeros, and the outputs they feed are never
  // stored).
  const int b_n = lane >> 2;
  const int b_q = lane & 3;
  const bool b_column = b_n < kRhsLanes;
  const uint32_t b_full = b_column ? uint32_t(b_n) * ldb * 4u + uint32_t(16 * b_q) : kOutOfRange;
  const uint32_t b_half = b_q < 2 ? b_full : kOutOfRange;
  const uint32_t b_span = uint32_t(kRhsLanes - 1) * ldb * 4u;  // a B tile's bytes before its last column
  const int64_t ldb_wide = L.a.scalar_cols;
  const int64_t b_lane = int64_t(b_n & (kRhsLanes - 1)) * ldb_wide + 4 * b_q;  // kWideB: the lane's float offset
  const int slot_write = b_slot_index(b_n, b_q);
  const int slot_read = b_slot_index(x, group);

  f32x4 acc[T][kRhsTiles];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int nt = 0; nt < kRhsTiles; ++nt) acc[t][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int segment = kWave << shift;  // steps whose records the row's waves hold at once, one per lane
  for (int seg = 0; seg < count; seg += segment) {
    const int seg_count = min(segment, count - seg);
    const int mine = owned_steps(seg_count, lead, shift);
    if (mine == 0) continue;
    const StepRec rec = L.steps[min(first + seg + owned_step(min(lane, mine - 1), lead, shift), L.step_limit)];
    const StepRec lead_rec = item.first;

    // Loads the wave's j-th step of the segment; a dead step (live == false)
    // gets zero-byte resources.  The row's first step comes from the row item,
    // so its loads do not wait for the step records.
    auto issue = [&](Stage<RHS, T>& st, int j, bool live) {
      const int l = min(j, kWave - 1);
      const bool leading = seg == 0 && j == 0;
      const int64_t a_off = leading ? lead_rec.a_off : lane_value(rec.a_off, l);
      const int64_t b_word = leading ? lead_rec.b_off : lane_value(rec.b_off, l);
      const bool half = (b_word & kHalfStep) != 0;
      const rsrc_t a_rsrc = make_rsrc(L.a.values + a_off, live ? (half ? a_half_bytes : a_full_bytes) : 0u);
      // The buffer-load builtins return raw bits (u32x4): bit-cast them.
#pragma unroll
      for (int q = 0; q < T; ++q)
        st.a[q] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       a_rsrc, kDirect ? a_direct + q * h * 4 : 16 * lane + 1024 * q, 0, kNonTemporal));
      const float* b_base = L.b + (b_word & kOffsetMask);
      if constexpr (kWideB) {
        // The same addresses as the buffer loads below; the lanes those give
        // zeros (a dead step, the upper half of a half step, columns past
        // RHS 8) load nothing.
        const bool take = live && (!half || b_q < 2) && b_column;
#pragma unroll
        for (int nt = 0; nt < kRhsTiles; ++nt) {
          st.b[nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          if (take) st.b[nt] = *reinterpret_cast<const f32x4_unaligned*>(b_base + b_lane + int64_t(nt) * 16 * ldb_wide);
        }
      } else {
        const uint32_t vb = half ? b_half : b_full;
        const uint32_t b_bytes = live ? b_span + (half ? 32u : 64u) : 0u;
#pragma unroll
        for (int nt = 0; nt < kRhsTiles; ++nt) {
          const rsrc_t b_rsrc = make_rsrc(b_base + int64_t(nt) * 16 * ldb, b_bytes);
          st.b[nt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, int(vb), 0, 0));
        }
      }
    };
    // Moves A and B through the wave's LDS slots into MFMA layout, then runs
    // the step.
    auto compute = [&](const Stage<RHS, T>& st) {
      if constexpr (!kDirect) {
#pragma unroll
        for (int q = 0; q < T; ++q) *reinterpret_cast<f32x4*>(a_slot + a_write[q]) = st.a[q];
      }
      if constexpr (kValu) {
        valu_step<RHS, T>(st.b, reinterpret_cast<float*>(b_slot), a_slot, acc, group, x, b_n, b_q, last_rows);
        return;
      }
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) b_slot[nt * kWave + slot_write] = st.b[nt];
      f32x4 bv[kRhsTiles];
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) bv[nt] = b_slot[nt * kWave + slot_read];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float av = kDirect ? st.a[i][t]
                           : t < T - 1 ? a_slot[a_read + 16 * t + i * ld]
                                       : a_slot[a_read_last + i * ld];
#pragma unroll
          for (int nt = 0; nt < kRhsTiles; ++nt)
            acc[t][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[nt][i], av, acc[t][nt], 0, 0, 0);
        }
    };

    // Two stages: step j + 1 loads while step j computes.  The loop has one
    // exit, at its back edge, so the compiler keeps the accumulators in
    // place; with runs of two steps only a wave holding a short final run
    // has an odd count, and its last compute multiplies a dead step's zeros.
    // A scheduling barrier after each issue keeps the compiler from moving
    // the prefetch below the compute it must overlap.
    Stage<RHS, T> r0, r1;
    issue(r0, 0, true);
    for (int j = 0; j < mine; j += 2) {
      issue(r1, j + 1, j + 1 < mine);
      __builtin_amdgcn_sched_barrier(0);
      compute(r0);
      issue(r0, j + 2, j + 2 < mine);
      __builtin_amdgcn_sched_barrier(0);
      compute(r1);
    }
  }

  // A shared row's partial slabs are summed into wave 0's acc; a packed
  // row's wave already holds its row's sums.
  if (shared && !reduce_partials<RHS, T, kValu>(acc, lds, wave, lane)) return;
  const int64_t ldc = L.ldc;
  if constexpr (kDirect) {
    // Lane x holds rows 4 x .. 4 x + 3 of output columns 4 g + v: one
    // 16-byte store each, for the lanes whose rows are below h (a multiple
    // of 8, so a lane's four rows are all below h or all past it).
    if (4 * x + 3 < h) {
      float* c_rows = L.c + item.c_off + 4 * x;
      f32x4 sum[T];
#pragma unroll
      for (int t = 0; t < T; ++t) sum[t] = acc[t][0];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int n = 4 * group + v;
        if (n < RHS)
          *reinterpret_cast<f32x4_unaligned*>(c_rows + int64_t(n) * ldc) =
              f32x4{sum[0][v], sum[1][v], sum[2][v], sum[3][v]};
      }
    }
    return;
  }
  float* c_row = L.c + item.c_off + x;
  if constexpr (kValu) {
    // Lane (g, x) holds rows 16 t + x of RHS columns g * RHS / 4 + j.
    constexpr int kCols = RHS / 4;
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (t < T - 1 || x < last_rows)
#pragma unroll
        for (int j = 0; j < kCols; ++j) c_row[16 * t + int64_t(group * kCols + j) * ldc] = acc[t][j / 4][j % 4];
    return;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t < T - 1 || x < last_rows) {
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) {
        const f32x4 sum = acc[t][nt];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int n = nt * 16 + 4 * group + v;
          if (n < RHS) c_row[16 * t + int64_t(n) * ldc] = sum[v];
        }
      }
    }
  }
}

template <int RHS, bool kValu, bool kWideB>
__global__ __launch_bounds__(kThreads) void row_owned_mfma_kernel(Launch L) {
  __shared__ __attribute__((aligned(16))) char lds[Lds<RHS, kValu>::kTotal];
  const int wave = uniform(int(threadIdx.x) / kWave);
  const int lane = int(threadIdx.x) % kWave;
  const WaveItem item = L.items[int64_t(blockIdx.x) * kWaves + wave];
  // An idle wave leaves.  A workgroup whose row is shared has no idle wave,
  // so no wave that leaves here is awaited at a barrier.
  if (uniform(item.step_count) < 0) return;
  switch ((uniform(item.h) + 15) >> 4) {
  case 1: row_body<RHS, 1, kValu, kWideB>(L, item, lds, wave, lane); break;
  case 2: row_body<RHS, 2, kValu, kWideB>(L, item, lds, wave, lane); break;
  case 3: row_body<RHS, 3, kValu, kWideB>(L, item, lds, wave, lane); break;
  default: row_body<RHS, 4, kValu, kWideB>(L, item, lds, wave, lane); break;
  }
}

// RHS 64 tile split (row_tiles_kernel).  A workgroup takes one block row
// (the schedule's tile order gives every row with k steps a workgroup of its
// own and packs only empty rows, four to a workgroup, which it takes one
// after another), and all four waves work on it: wave w computes RHS tile w
// (C columns 16 w .. 16 w + 15) over all of the row's k steps, in step
// order.
// A step's A tile (16 block columns, 64 h bytes) is loaded once for the
// workgroup, 16 bytes per lane, into one of two LDS buffers, and one barrier
// per step publishes it; each wave moves its own B tile through its own LDS
// slot.  There is no cross-wave reduction, and a wave holds T row tiles of
// one RHS tile: a quarter of the split-k kernel's accumulators, so a SIMD
// holds 6 of these waves against 3 of the split-k kernel's.  The price is
// that a row's steps run one after another on one workgroup, so the launch
// is as long as its longest row; the schedule takes this kernel only where
// that stays short against the work per workgroup slot (rhs64_tiles).
constexpr int kTileLd = 16 * kMaxTiles + 4;  // A buffer: float (r, k) at k * kTileLd + r
constexpr int kTileFloats = 16 * kTileLd;
constexpr int kTileLdsBytes = 2 * kTileFloats * 4 + kWaves * kWave * 16;

template <int T, bool kWideB>
__device__ __forceinline__ void tile_row(const Launch& L, const WaveItem& item, char* lds, int wave, int lane) {
  constexpr int ld = kTileLd;
  const int tid = wave * kWave + lane;
  const int group = lane >> 4;
  const int x = lane & 15;
  const int h = uniform(item.h);
  const int count = uniform(item.step_count);
  const int first = uniform(item.step_first);
  const int last_rows = h - 16 * (T - 1);
  const uint32_t ldb = uint32_t(L.a.scalar_cols);
  float* a_bufs = reinterpret_cast<float*>(lds);
  f32x4* b_slot = reinterpret_cast<f32x4*>(lds + 2 * kTileFloats * 4) + wave * kWave;

  // This thread's 16 bytes of the step's column-major h x 16 A tile go to
  // float (k, r) of the buffer (f / h computed as in row_body); threads past
  // the tile hold zeros and write them to the never-read padding rows.
  const uint32_t h_recip = uint32_t(uniform(int((65536u + uint32_t(h) - 1u) / uint32_t(h))));
  const int f = 4 * tid;
  const int fk = int((uint32_t(f) * h_recip) >> 16);
  const int a_write = f < 16 * h ? fk * ld + (f - fk * h) : (tid & 15) * ld + 16 * kMaxTiles;
  const int a_read = 4 * group * ld + x;
  const int a_read_last = 4 * group * ld + 16 * (T - 1) + (x & (last_rows - 1));
  const uint32_t a_full_bytes = uint32_t(16 * h) * 4u;
  const uint32_t a_half_bytes = uint32_t(8 * h) * 4u;

  // B: lane 4n + q of wave w reads B[k0 + 4q .. k0 + 4q + 3, 16 w + n], as
  // one tile of the split-k kernel.
  const int b_n = lane >> 2;
  const int b_q = lane & 3;
  const uint32_t b_full = uint32_t(b_n) * ldb * 4u + uint32_t(16 * b_q);
  const uint32_t b_half = b_q < 2 ? b_full : kOutOfRange;
  const uint32_t b_span = 15u * ldb * 4u;
  const int64_t b_lane = int64_t(b_n) * L.a.scalar_cols + 4 * b_q;  // kWideB: the lane's float offset
  const int slot_write = b_slot_index(b_n, b_q);
  const int slot_read = b_slot_index(x, group);

  f32x4 acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  struct TileStage {
    f32x4 a, b;
  };
  int parity = 0;  // A buffer of the next step
  for (int seg = 0; seg < count; seg += kWave) {
    const int seg_count = min(kWave, count - seg);
    const StepRec rec = L.steps[min(first + seg + min(lane, seg_count - 1), L.step_limit)];
    auto issue = [&](TileStage& st, int j) {
      const bool live = j < seg_count;
      const int l = min(j, kWave - 1);
      const int64_t a_off = lane_value(rec.a_off, l);
      const int64_t b_word = lane_value(rec.b_off, l);
      const bool half = (b_word & kHalfStep) != 0;
      const rsrc_t a_rsrc = make_rsrc(L.a.values + a_off, live ? (half ? a_half_bytes : a_full_bytes) : 0u);
      st.a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, 16 * tid, 0, kNonTemporal));
      const float* b_base = L.b + (b_word & kOffsetMask) + int64_t(wave) * 16 * L.a.scalar_cols;
      if constexpr (kWideB) {
        st.b = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (live && (!half || b_q < 2)) st.b = *reinterpret_cast<const f32x4_unaligned*>(b_base + b_lane);
      } else {
        const rsrc_t b_rsrc = make_rsrc(b_base, live ? b_span + (half ? 32u : 64u) : 0u);
        st.b = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, int(half ? b_half : b_full), 0, 0));
      }
    };
    // Writes the step's A quarter and B tile, publishes the A tile with one
    // barrier, runs the wave's T x 4 MFMAs.  The two A buffers alternate: a
    // wave writes buffer p only after the barrier of the step before, which
    // every wave reaches after its reads of buffer p two steps back.
    auto compute = [&](const TileStage& st) {
      float* a = a_bufs + parity * kTileFloats;
      parity ^= 1;
      *reinterpret_cast<f32x4*>(a + a_write) = st.a;
      b_slot[slot_write] = st.b;
      __syncthreads();
      const f32x4 bv = b_slot[slot_read];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float av = t < T - 1 ? a[a_read + 16 * t + i * ld] : a[a_read_last + i * ld];
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[i], av, acc[t], 0, 0, 0);
        }
    };
    // Two stages, as in row_body: step j + 1 loads while step j computes; an
    // odd count ends on a dead step (zero-byte loads, zeros multiplied in).
    TileStage r0, r1;
    issue(r0, 0);
    for (int j = 0; j < seg_count; j += 2) {
      issue(r1, j + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(r0);
      issue(r0, j + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(r1);
    }
  }
  // Every wave's reads of this row's A buffers end before the next row of
  // the unit writes one.
  __syncthreads();
  const int64_t ldc = L.ldc;
  float* c_row = L.c + item.c_off + x;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t < T - 1 || x < last_rows) {
#pragma unroll
      for (int v = 0; v < 4; ++v) c_row[16 * t + int64_t(wave * 16 + 4 * group + v) * ldc] = acc[t][v];
    }
  }
}

template <bool kWideB>
__global__ __launch_bounds__(kThreads) void row_tiles_kernel(Launch L) {
  __shared__ __attribute__((aligned(16))) char lds[kTileLdsBytes];
  const int wave = uniform(int(threadIdx.x) / kWave);
  const int lane = int(threadIdx.x) % kWave;
  const WaveItem* unit = L.items + int64_t(blockIdx.x) * kWaves;
  // Every wave reads the same items, so every branch below is uniform across
  // the workgroup and every wave reaches every barrier.
  const bool shared = uniform(unit[0].group) > 1;
  const int rows = shared ? 1 : kWaves;
  for (int r = 0; r < rows; ++r) {
    const WaveItem item = unit[r];
    if (uniform(item.step_count) < 0) continue;
    switch ((uniform(item.h) + 15) >> 4) {
    case 1: tile_row<1, kWideB>(L, item, lds, wave, lane); break;
    case 2: tile_row<2, kWideB>(L, item, lds, wave, lane); break;
    case 3: tile_row<3, kWideB>(L, item, lds, wave, lane); break;
    default: tile_row<4, kWideB>(L, item, lds, wave, lane); break;
    }
  }
}

// tiles: RHS 64 runs the tile-split kernel (the MFMA kernel only).
template <int RHS, bool kValu, bool kWideB>
void launch(const Launch& L, int64_t groups, bool tiles, hipStream_t stream) {
  if (RHS == 64 && !kValu && tiles)
    row_tiles_kernel<kWideB><<<dim3(unsigned(groups)), dim3(kThreads), 0, stream>>>(L);
  else
    row_owned_mfma_kernel<RHS, kValu, kWideB><<<dim3(unsigned(groups)), dim3(kThreads), 0, stream>>>(L);
}

template <bool kValu, bool kWideB>
void launch_rhs(const Launch& L, int64_t groups, int rhs, bool tiles, hipStream_t stream) {
  switch (rhs) {
  case 8: launch<8, kValu, kWideB>(L, groups, false, stream); break;
  case 16: launch<16, kValu, kWideB>(L, groups, false, stream); break;
  case 32: launch<32, kValu, kWideB>(L, groups, false, stream); break;
  default: launch<64, kValu, kWideB>(L, groups, tiles, stream); break;
  }
}

// wide: 64-bit B addressing (the MFMA kernel only; the VALU variant keeps
// the 32-bit offset bound).
template <bool kValu>
void launch_items(const Launch& L, int64_t groups, int rhs, bool wide, bool tiles, hipStream_t stream) {
  if (groups <= 0) return;
  if (groups > int64_t(0x7fffffff)) throw std::invalid_argument("schedule too large for one launch");
  if constexpr (kValu) {
    if (wide) throw std::invalid_argument("the VALU variant needs (min(rhs, 16) - 1) * K * 4 + 128 <= 0xfffffff0");
    launch_rhs<true, false>(L, groups, rhs, false, stream);
  } else {
    if (wide)
      launch_rhs<false, true>(L, groups, rhs, tiles, stream);
    else
      launch_rhs<false, false>(L, groups, rhs, tiles, stream);
  }
  check_hip(hipGetLastError(), "row_owned_mfma launch");
}

// Second pass of the split-row path: workgroup (i, j) sums the j-th run of
// kReduceThreads elements of block row i's slab over the row's partial slabs
// in part order, ((p0 + p1) + p2) + ..., and writes them to C.  Consecutive
// lanes take consecutive rows of one RHS column, so each part's reads and the
// C stores are contiguous; the loads of four parts are issued before their
// adds, so a lane waits for memory once per four parts.
constexpr int kReduceThreads = 256;

__global__ __launch_bounds__(kReduceThreads) void split_reduce_kernel(const SplitRowRec* rows, const float* w,
                                                                      int64_t ldw, float* c, int64_t ldc, int rhs) {
  const SplitRowRec r = rows[blockIdx.x];
  const int h = r.h;
  const int e = int(blockIdx.y) * kReduceThreads + int(threadIdx.x);
  if (e >= h * rhs) return;
  const int n = e / h;
  const int i = e - n * h;
  const float* part = w + r.w_off + i + int64_t(n) * ldw;
  float sum = part[0];
  int q = 1;
  for (; q + 3 < r.parts; q += 4) {
    const float v0 = part[int64_t(q) * h], v1 = part[int64_t(q + 1) * h];
    const float v2 = part[int64_t(q + 2) * h], v3 = part[int64_t(q + 3) * h];
    sum = (((sum + v0) + v1) + v2) + v3;
  }
  for (; q < r.parts; ++q) sum += part[int64_t(q) * h];
  c[r.c_off + i + int64_t(n) * ldc] = sum;
}

// The allocation-free split-row launcher's workspace: one static array per
// device, 16 MiB, set aside when the library's code object is loaded on the
// device and held until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host it names a stand-in, not device memory):
// it passes the device address that hipGetSymbolAddress returns for the
// current device, looked up once per device.
constexpr int64_t kScratchFloats = int64_t(4) << 20;
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};

float* scratch_for_current_device() {
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  if (device < 0 || device >= kMaxDevices) throw std::runtime_error("device ordinal beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device] == nullptr) {
    void* address = nullptr;
    check_hip(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (split-row scratch)");
    g_scratch[device] = static_cast<float*>(address);
  }
  return g_scratch[device];
}

}  // namespace

bool narrow_b_offsets(const vbsr_device_view& a, int rhs) {
  // 32-bit buffer offsets: a B tile's resource spans min(rhs, 16) - 1
  // columns of ld K plus one step, and must end at least 64 bytes below the
  // out-of-range offset (K <= 153,391,684 at RHS 8, 71,582,785 otherwise).
  const uint64_t span = uint64_t(rhs < 16 ? rhs - 1 : 15) * uint64_t(a.scalar_cols) * 4u + 64u;
  return span + 64u <= kOutOfRange;
}

namespace {

// wide_b: 64-bit B addressing even where 32-bit offsets would do.
template <bool kValu>
void launch_row_owned_math(const vbsr_device_view& a, const vbsr_row_schedule& s, const float* b, float* c, int rhs,
                           bool wide_b, hipStream_t stream) {
  if (!supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
  check_panels(a, b, c, rhs);
  const void* rows = rhs >= 32 && s.rows_wide != nullptr ? s.rows_wide : s.rows;
  int64_t groups = s.groups;
  const bool tiles = !kValu && rhs == 64 && s.rhs64_tiles != 0;
  if (tiles) {
    rows = s.rows_tile;
    groups = s.groups_tile;
  } else if (rhs == 64 && s.rows_rhs64 != nullptr) {
    rows = s.rows_rhs64;
    groups = s.groups_rhs64;
  }
  // A matrix with block rows has at least one workgroup in every order (empty
  // rows included), so a schedule whose chosen order is missing or empty
  // belongs to no matrix with rows: refuse it rather than launch nothing or
  // read through a null pointer.
  if (a.block_rows > 0 && (rows == nullptr || groups <= 0 || s.steps == nullptr))
    throw std::invalid_argument("schedule has no launch order for this matrix (take it from vbsr_matrix_row_schedule)");
  const Launch L{a, static_cast<const StepRec*>(s.steps), static_cast<const WaveItem*>(rows), s.step_limit, b, c,
                 a.scalar_rows};
  // At RHS 64 the schedule says which kernel runs: the split-k kernel or
  // the tile split (rhs64_tiles, set by the matrix's rule).
  launch_items<kValu>(L, groups, rhs, wide_b || !narrow_b_offsets(a, rhs), tiles, stream);
}

}  // namespace

void launch_row_owned(const vbsr_device_view& a, const vbsr_row_schedule& s, const float* b, float* c, int rhs,
                      hipStream_t stream) {
  launch_row_owned_math<false>(a, s, b, c, rhs, false, stream);
}

void launch_row_owned_wide_b(const vbsr_device_view& a, const vbsr_row_schedule& s, const float* b, float* c,
                             int rhs, hipStream_t stream) {
  launch_row_owned_math<false>(a, s, b, c, rhs, true, stream);
}

void launch_row_owned_valu(const vbsr_device_view& a, const vbsr_row_schedule& s, const float* b, float* c, int rhs,
                           hipStream_t stream) {
  launch_row_owned_math<true>(a, s, b, c, rhs, false, stream);
}

int64_t split_workspace_floats(const DeviceMatrix::Split& split, int rhs) { return split.virtual_rows * rhs; }

void launch_split_row(const vbsr_device_view& a, const vbsr_row_schedule& s, const DeviceMatrix::Split& split,
                      const float* b, float* c, int rhs, float* workspace, int64_t workspace_floats,
                      hipStream_t stream) {
  if (!supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
  check_panels(a, b, c, rhs);
  const int64_t needed = split_workspace_floats(split, rhs);
  if (needed > 0 && (workspace == nullptr || workspace_floats < needed))
    throw std::invalid_argument("split-row workspace too small");
  if (needed > 0) {
    // The workspace must not overlap B or C.
    check_panels(split.virtual_rows, a.scalar_cols, b, workspace, rhs);
    check_panels(split.virtual_rows, a.scalar_rows, c, workspace, rhs);
  }
  if (a.block_rows <= 0) return;
  const Launch L{a, static_cast<const StepRec*>(s.steps), split.items, s.step_limit, b, workspace,
                 split.virtual_rows};
  launch_items<false>(L, split.groups, rhs, !narrow_b_offsets(a, rhs), false, stream);
  // A row's slab holds at most 64 * rhs elements.
  const unsigned chunks = unsigned((64 * rhs + kReduceThreads - 1) / kReduceThreads);
  split_reduce_kernel<<<dim3(unsigned(a.block_rows), chunks), dim3(kReduceThreads), 0, stream>>>(
      split.rows, workspace, split.virtual_rows, c, a.scalar_rows, rhs);
  check_hip(hipGetLastError(), "split_reduce launch");
}

int64_t split_scratch_floats() { return kScratchFloats; }

void launch_split_row_static(const vbsr_device_view& a, const vbsr_row_schedule& s, const DeviceMatrix::Split& split,
                             const float* b, float* c, int rhs, hipStream_t stream) {
  if (!supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
  const int64_t needed = split_workspace_floats(split, rhs);
  if (needed > kScratchFloats)
    throw std::invalid_argument("split-row workspace of " + std::to_string(needed * 4) +
                                " bytes exceeds the static scratch (" + std::to_string(kScratchFloats * 4) +
                                " bytes); use vbsr_launch_split_row with a workspace");
  launch_split_row(a, s, split, b, c, rhs, scratch_for_current_device(), kScratchFloats, stream);
}

}  // namespace vbsr_amd
