// MFMA row-owned kernels: the MI355X counterpart of the reference's tuned
// row-owned family (src/kernels/row_owned.cu:47-310, dispatched at 397-423).
//
// One wave64 owns one block row of height h and computes its whole h x RHS
// output slab, so every C element has exactly one writer and no atomics or
// workspace are needed.  The row's product is a sum over its blocks of
// (h x w block) * (w x RHS slice of B), evaluated with
// v_mfma_f32_16x16x4_f32 on 16x16 tiles of the transposed output:
//
//   D[n][r] += sum_{g=0..3} Bop[n][g] * Aop[g][r]
//   lane = 16*g + x:  src0 = B[k(g), n0 + x]   (rhs column x of the tile)
//                     src1 = A[r0 + x, k(g)]   (local row x of the tile)
//   result lane 16*g' + x, register v:  C[r0 + x, n0 + 4*g' + v]
//
// Within a 16-wide k step, lane group g owns k = k0 + 4g + i for the four
// MFMAs i = 0..3, so one 16-byte load per lane fetches its four B values
// (consecutive rows of one B column) and the A operand of MFMA i is, across
// each 16-lane group, 16 consecutive floats (64 B) of block column
// k0 + 4g + i.  Block widths are multiples of 8: a trailing 8-wide step
// zeroes the operands of groups 2 and 3.  Rows are padded to 16-row tiles
// (h = 8, 24, 40, 56 zero the missing rows); RHS 8 fills half of one rhs
// tile.  Zeroed lanes never load, so no access leaves the block or B.
//
// Accumulation order is fixed by the row's block order and the MFMA
// sequence, so results are bit-identical from run to run.
#include <hip/hip_runtime.h>

#include "../internal.hpp"

namespace vbsr_amd {
namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kWavesPerGroup = 4;
constexpr int kGroupThreads = kWave * kWavesPerGroup;

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <int RHS, int TILES>
__device__ __forceinline__ void row_product(const vbsr_device_view& a, int row, int h,
                                            const float* __restrict__ b, float* __restrict__ c,
                                            int lane) {
  constexpr int kRhsTiles = RHS < 16 ? 1 : RHS / 16;
  const int group = lane >> 4;
  const int x = lane & 15;

  f32x4 acc[TILES][kRhsTiles];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int nt = 0; nt < kRhsTiles; ++nt) acc[t][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int first = a.row_ptr[row];
  const int last = a.row_ptr[row + 1];
  const int64_t ldb = a.scalar_cols;

  for (int blk = first; blk < last; ++blk) {
    const int col = a.block_col[blk];
    const int w = a.col_size[col];
    const float* a_blk = a.values + a.value_off[blk];
    const float* b_blk = b + a.col_scalar_off[col];

    for (int k0 = 0; k0 < w; k0 += 16) {
      const int k = k0 + 4 * group;
      const bool k_ok = k < w;

      f32x4 bq[kRhsTiles];
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt) {
        const int n = nt * 16 + x;
        bq[nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (k_ok && n < RHS) bq[nt] = *reinterpret_cast<const f32x4*>(b_blk + k + int64_t(n) * ldb);
      }

      float av[TILES][4];
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const int r = t * 16 + x;
#pragma unroll
        for (int i = 0; i < 4; ++i) av[t][i] = 0.0f;
        if (k_ok && r < h) {
          const float* p = a_blk + r + int64_t(k) * h;
#pragma unroll
          for (int i = 0; i < 4; ++i) av[t][i] = p[int64_t(i) * h];
        }
      }

#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
          for (int nt = 0; nt < kRhsTiles; ++nt)
            acc[t][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(bq[nt][i], av[t][i], acc[t][nt], 0, 0, 0);
    }
  }

  const int64_t ldc = a.scalar_rows;
  float* c_row = c + a.row_scalar_off[row];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int r = t * 16 + x;
    if (r < h) {
#pragma unroll
      for (int nt = 0; nt < kRhsTiles; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int n = nt * 16 + 4 * group + v;
          if (n < RHS) c_row[r + int64_t(n) * ldc] = acc[t][nt][v];
        }
    }
  }
}

template <int RHS>
__global__ __launch_bounds__(kGroupThreads) void row_owned_mfma_kernel(vbsr_device_view a,
                                                                       const int32_t* __restrict__ order,
                                                                       const float* __restrict__ b,
                                                                       float* __restrict__ c) {
  const int wave = wave_uniform(int(threadIdx.x) / kWave);
  const int lane = int(threadIdx.x) % kWave;
  const int slot = int(blockIdx.x) * kWavesPerGroup + wave;
  if (slot >= a.block_rows) return;
  const int row = wave_uniform(order ? order[slot] : slot);
  const int h = a.row_size[row];
  switch ((h + 15) / 16) {
  case 1: row_product<RHS, 1>(a, row, h, b, c, lane); break;
  case 2: row_product<RHS, 2>(a, row, h, b, c, lane); break;
  case 3: row_product<RHS, 3>(a, row, h, b, c, lane); break;
  default: row_product<RHS, 4>(a, row, h, b, c, lane); break;
  }
}

template <int RHS>
void launch(const vbsr_device_view& a, const int32_t* order, const float* b, float* c, hipStream_t stream) {
  const unsigned groups = unsigned((int64_t(a.block_rows) + kWavesPerGroup - 1) / kWavesPerGroup);
  row_owned_mfma_kernel<RHS><<<dim3(groups), dim3(kGroupThreads), 0, stream>>>(a, order, b, c);
}

}  // namespace

void launch_mfma(const vbsr_device_view& a, const int32_t* order, const float* b, float* c, int rhs,
                 hipStream_t stream) {
  if (!supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
  if (a.block_rows <= 0) return;
  switch (rhs) {
  case 8: launch<8>(a, order, b, c, stream); break;
  case 16: launch<16>(a, order, b, c, stream); break;
  case 32: launch<32>(a, order, b, c, stream); break;
  default: launch<64>(a, order, b, c, stream); break;
  }
  check_hip(hipGetLastError(), "row_owned_mfma launch");
}

}  // namespace vbsr_amd
