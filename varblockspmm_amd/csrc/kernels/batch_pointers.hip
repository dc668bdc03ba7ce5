// Per-call pointer arrays of the grouped-GEMM baseline (gemm_baseline.cpp):
// entry i points at B + b_offset[i] and C + c_offset[i].  The reference
// rebuilds these arrays on the host and copies them at every execute
// (src/baseline/slot_split.cu:118-131); here one small kernel writes them on
// the device from offsets uploaded once.
#include <hip/hip_runtime.h>

#include "../internal.hpp"

namespace vbsr_amd {
namespace {

__global__ void fill_batch_pointers_kernel(const int64_t* __restrict__ b_offset, const int64_t* __restrict__ c_offset,
                                           int64_t count, const float* b, float* c, const float** b_pointers,
                                           float** c_pointers) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
    b_pointers[i] = b + b_offset[i];
    c_pointers[i] = c + c_offset[i];
  }
}

}  // namespace

void fill_batch_pointers(const int64_t* b_offset, const int64_t* c_offset, int64_t count, const float* b, float* c,
                         const float** b_pointers, float** c_pointers, hipStream_t stream) {
  if (count <= 0) return;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 1024);
  fill_batch_pointers_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(b_offset, c_offset, count, b, c,
                                                                             b_pointers, c_pointers);
  check_hip(hipGetLastError(), "fill_batch_pointers launch");
}

}  // namespace vbsr_amd
