// read_ceiling: the read bandwidth an MI355X delivers to a streaming kernel,
// from each level a kernel's L2 misses can be served by.  The row-owned
// kernel's traffic (its L2 misses, counted by FETCH_SIZE) is compared with
// these rates to say what bounds it.
//
// Cases (one JSON line each, median of --reps timed launches):
//   dram      1 GiB read once per launch; a second 1 GiB buffer is read
//             between launches, so nothing of the first is cached in L2 or
//             in the 256 MB Infinity Cache (MALL).
//   mall      96 MiB read 4 times per launch, after a warm-up launch: each
//             XCD streams its eighth (12 MiB, three times its 4 MiB L2) in
//             order, so every access misses L2 and the Infinity Cache serves
//             it.
//   l2        16 MiB read 8 times per launch: each XCD's eighth (2 MiB) stays
//             in its L2.
//   dram_regions_48k / _8k
//             168 MiB (A at configuration 3) read once, cold, laid out as the
//             row-owned kernel reads A: one workgroup per contiguous 48 KiB
//             (about a block row's A) or 8 KiB region, which it reads and
//             leaves.
// Each case runs with plain and with non-temporal 16-byte loads.
//   mixed     the row-owned kernel's mix of L2 misses at configuration 3
//             (about equal bytes of each): one launch reads 168 MiB once,
//             cold, with non-temporal loads (as it reads A) and, interleaved
//             with those, an 84 MiB buffer twice with plain loads, which the
//             Infinity Cache holds and each XCD's L2 does not (as it reads
//             B's line misses).  The Infinity Cache buffer is read once before
//             each timed launch, after the flush.
//   mixed_segments
//             the same, with the warm reads shaped as the kernel's B loads:
//             a K x 32 column-major panel (K = 145,304, as at configuration
//             3), read in k steps of 16 rows at pseudo-random 8-row
//             offsets, four lanes per column and 16 columns per load, so
//             each load reads sixteen 64-byte segments that straddle
//             128-byte lines as B's do.
//   write     1 GiB of zeros written once with plain 16-byte stores, after
//             the flush.
//   mixed_write, mixed_write_half_lines, mixed_write_shared_lines
//             the mixed case plus 18.9 MB of stores (C's bytes at
//             configuration 3, RHS 32): into whole lines, into the first
//             halves of twice as many lines, or into lines whose halves two
//             workgroups on different XCDs write (as adjacent block rows
//             share the boundary lines of C's columns).
//
// Workgroup i runs on XCD i mod 8; the grid is a multiple of 8 and each
// workgroup reads 16 KiB chunks i, i + grid, ..., so each XCD reads one
// eighth of the buffer.
//
//   make -C varblockspmm_amd/bench read_ceiling && varblockspmm_amd/bench/read_ceiling
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 16-byte loads in flight per lane

void check(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(status));
    std::exit(1);
  }
}

template <bool kNonTemporal>
__global__ __launch_bounds__(kThreads) void read_kernel(const f32x4* __restrict__ data, int64_t count, int passes,
                                                        float* __restrict__ sink) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t chunk = int64_t(kThreads) * kUnroll;
  const int64_t stride = int64_t(gridDim.x) * chunk;
  for (int pass = 0; pass < passes; ++pass) {
    for (int64_t base = int64_t(blockIdx.x) * chunk + threadIdx.x; base < count; base += stride) {
      f32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t i = base + int64_t(u) * kThreads;
        if (i < count)
          v[u] = kNonTemporal ? __builtin_nontemporal_load(data + i) : data[i];
        else
          v[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc += v[u];
    }
  }
  // Keeps the loads live; the buffers hold zeros, so nothing is written.
  const float total = acc.x + acc.y + acc.z + acc.w;
  if (total != 0.0f) sink[blockIdx.x * kThreads + threadIdx.x] = total;
}

// The same reads laid out as the row-owned kernel reads A: workgroup b reads
// only its own contiguous region of `region` vectors (a block row's A), its
// four waves taking interleaved 1 KB pieces, kUnroll in flight per lane, and
// leaves; the grid covers the buffer once.
template <bool kNonTemporal>
__global__ __launch_bounds__(kThreads) void region_kernel(const f32x4* __restrict__ data, int64_t region,
                                                          float* __restrict__ sink) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4* base = data + int64_t(blockIdx.x) * region;
  const int64_t chunk = int64_t(kThreads) * kUnroll;
  for (int64_t i0 = threadIdx.x; i0 < region; i0 += chunk) {
    f32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + int64_t(u) * kThreads;
      if (i < region)
        v[u] = kNonTemporal ? __builtin_nontemporal_load(base + i) : base[i];
      else
        v[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc += v[u];
  }
  const float total = acc.x + acc.y + acc.z + acc.w;
  if (total != 0.0f) sink[threadIdx.x] = total;
}

// The mixed case: lane loads alternate between `cold` (non-temporal, read
// once) and `warm` (plain; index i mod warm_count, so it is swept
// cold_count / warm_count times), kUnroll of each in flight.  kWrite: on
// every odd iteration each lane also stores its running sum, 16 bytes, to
// `out`, which the workgroup's lanes fill with contiguous 4 KiB pieces
// (write bytes about 5% of the read bytes, as C is of the row-owned
// kernel's L2-miss reads at configuration 3).  kWrite 2 stores the same
// vectors to the first 64 bytes of twice as many 128-byte lines, and kWrite
// 3 shares those lines between workgroups 2p and 2p + 1 (on different XCDs):
// one writes each line's first 64 bytes, the other its last 64, as
// adjacent block rows share the boundary lines of C's columns.
template <int kWrite>
__global__ __launch_bounds__(kThreads) void mixed_kernel(const f32x4* __restrict__ cold, int64_t cold_count,
                                                         const f32x4* __restrict__ warm, int64_t warm_count,
                                                         float* __restrict__ sink, f32x4* __restrict__ out) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t chunk = int64_t(kThreads) * kUnroll;
  const int64_t stride = int64_t(gridDim.x) * chunk;
  int64_t iteration = 0;
  for (int64_t base = int64_t(blockIdx.x) * chunk + threadIdx.x; base < cold_count; base += stride, ++iteration) {
    if (kWrite != 0 && (iteration & 1)) {
      const int64_t t = threadIdx.x, half_line = (t / 4) * 8 + t % 4;
      if (kWrite == 1)
        out[((iteration >> 1) * gridDim.x + blockIdx.x) * kThreads + t] = acc;
      else if (kWrite == 2)
        out[((iteration >> 1) * gridDim.x + blockIdx.x) * 2 * kThreads + half_line] = acc;
      else
        out[((iteration >> 1) * (gridDim.x / 2) + blockIdx.x / 2) * 2 * kThreads + half_line + 4 * (blockIdx.x % 2)] =
            acc;
    }
    f32x4 v[2 * kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + int64_t(u) * kThreads;
      const bool in = i < cold_count;
      v[2 * u] = in ? __builtin_nontemporal_load(cold + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      v[2 * u + 1] = in ? warm[i % warm_count] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < 2 * kUnroll; ++u) acc += v[u];
  }
  const float total = acc.x + acc.y + acc.z + acc.w;
  if (total != 0.0f) sink[blockIdx.x * kThreads + threadIdx.x] = total;
}

// mixed_segments: lane loads alternate between `cold` (non-temporal, read
// once, contiguous) and the panel `b` (plain): load u of a lane reads
// B[k0 + 4 q .. k0 + 4 q + 3, n] with n = (lane / 4) + 16 (u % 2), q = lane % 4
// and k0 a pseudo-random multiple of 8 per (iteration, u / 2).
__global__ __launch_bounds__(kThreads) void mixed_segments_kernel(const f32x4* __restrict__ cold, int64_t cold_count,
                                                                  const float* __restrict__ b, int64_t k_rows,
                                                                  float* __restrict__ sink) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t chunk = int64_t(kThreads) * kUnroll;
  const int64_t stride = int64_t(gridDim.x) * chunk;
  const int lane = int(threadIdx.x) % 64;
  const int64_t steps = (k_rows - 16) / 8;
  for (int64_t base = int64_t(blockIdx.x) * chunk + threadIdx.x; base < cold_count; base += stride) {
    f32x4 v[2 * kUnroll];
    const uint64_t it = uint64_t(base / chunk);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + int64_t(u) * kThreads;
      const bool in = i < cold_count;
      v[2 * u] = in ? __builtin_nontemporal_load(cold + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const uint64_t h = (it * 2654435761u + uint64_t(threadIdx.x / 64) * 40503u + uint64_t(u / 2) * 977u) % uint64_t(steps);
      const int64_t k0 = int64_t(h) * 8;
      const int64_t n = (lane >> 2) + 16 * (u & 1);
      const float* p = b + n * k_rows + k0 + 4 * (lane & 3);
      // p is 16-byte aligned: K, k0 and 4 q are multiples of 4 floats.
      v[2 * u + 1] = in ? *reinterpret_cast<const f32x4*>(p) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < 2 * kUnroll; ++u) acc += v[u];
  }
  const float total = acc.x + acc.y + acc.z + acc.w;
  if (total != 0.0f) sink[blockIdx.x * kThreads + threadIdx.x] = total;
}

struct Result {
  double median_us, gbps;
};

// region_bytes == 0: the strided sweep (read_kernel); otherwise one
// workgroup per region of that many bytes (region_kernel, one pass).
template <bool kNonTemporal>
Result run(const float* buffer, int64_t bytes, int passes, const float* flush, int64_t flush_bytes, int reps,
           int grid, float* sink, hipStream_t stream, int64_t region_bytes = 0) {
  const int64_t count = bytes / 16;
  const auto launch = [&](const float* p, int64_t n, int k) {
    if (region_bytes > 0 && p == buffer)
      region_kernel<kNonTemporal><<<unsigned(n / (region_bytes / 16)), kThreads, 0, stream>>>(
          reinterpret_cast<const f32x4*>(p), region_bytes / 16, sink);
    else
      read_kernel<kNonTemporal><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(p), n, k, sink);
  };
  hipEvent_t start, stop;
  check(hipEventCreateWithFlags(&start, hipEventDisableSystemFence), "hipEventCreate");
  check(hipEventCreateWithFlags(&stop, hipEventDisableSystemFence), "hipEventCreate");
  launch(buffer, count, passes);  // warm-up (and, for mall/l2, fills the caches)
  check(hipStreamSynchronize(stream), "warm-up");
  std::vector<double> us;
  for (int r = 0; r < reps; ++r) {
    if (flush != nullptr) launch(flush, flush_bytes / 16, 1);
    check(hipEventRecord(start, stream), "record");
    launch(buffer, count, passes);
    check(hipEventRecord(stop, stream), "record");
    check(hipEventSynchronize(stop), "sync");
    float ms = 0;
    check(hipEventElapsedTime(&ms, start, stop), "elapsed");
    us.push_back(double(ms) * 1000.0);
  }
  check(hipGetLastError(), "launch");
  std::sort(us.begin(), us.end());
  const double median = us[us.size() / 2];
  check(hipEventDestroy(start), "destroy");
  check(hipEventDestroy(stop), "destroy");
  return {median, double(bytes) * passes / (median * 1e3)};
}

// Streaming writes of zeros, strided as read_kernel reads.
__global__ __launch_bounds__(kThreads) void write_kernel(f32x4* __restrict__ data, int64_t count) {
  const int64_t chunk = int64_t(kThreads) * kUnroll;
  const int64_t stride = int64_t(gridDim.x) * chunk;
  for (int64_t base = int64_t(blockIdx.x) * chunk + threadIdx.x; base < count; base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + int64_t(u) * kThreads;
      if (i < count) data[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
}

// segments_k > 0: the warm reads are mixed_segments_kernel's B-shaped
// segments of a segments_k x 32 panel at `warm`; the bytes counted are then
// the cold bytes plus the same number of warm bytes requested.  out != null:
// mixed_kernel<true>, which also writes to `out` (see there).
Result run_mixed(const float* cold, int64_t cold_bytes, const float* warm, int64_t warm_bytes, const float* flush,
                 int64_t flush_bytes, int reps, int grid, float* sink, hipStream_t stream, int64_t segments_k = 0,
                 float* out = nullptr, int write_mode = 1) {
  hipEvent_t start, stop;
  check(hipEventCreateWithFlags(&start, hipEventDisableSystemFence), "hipEventCreate");
  check(hipEventCreateWithFlags(&stop, hipEventDisableSystemFence), "hipEventCreate");
  std::vector<double> us;
  for (int r = 0; r < reps + 1; ++r) {  // the first launch is a warm-up
    // Plain reads allocate in L2 and the Infinity Cache, so the flush
    // evicts the cold buffer from both; then the warm buffer is loaded.
    read_kernel<false><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(flush), flush_bytes / 16, 1, sink);
    read_kernel<false><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(warm), warm_bytes / 16, 1, sink);
    check(hipEventRecord(start, stream), "record");
    if (segments_k > 0)
      mixed_segments_kernel<<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(cold), cold_bytes / 16, warm,
                                                           segments_k, sink);
    else if (out != nullptr && write_mode == 1)
      mixed_kernel<1><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(cold), cold_bytes / 16,
                                                     reinterpret_cast<const f32x4*>(warm), warm_bytes / 16, sink,
                                                     reinterpret_cast<f32x4*>(out));
    else if (out != nullptr && write_mode == 2)
      mixed_kernel<2><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(cold), cold_bytes / 16,
                                                     reinterpret_cast<const f32x4*>(warm), warm_bytes / 16, sink,
                                                     reinterpret_cast<f32x4*>(out));
    else if (out != nullptr)
      mixed_kernel<3><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(cold), cold_bytes / 16,
                                                     reinterpret_cast<const f32x4*>(warm), warm_bytes / 16, sink,
                                                     reinterpret_cast<f32x4*>(out));
    else
      mixed_kernel<0><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(cold), cold_bytes / 16,
                                                     reinterpret_cast<const f32x4*>(warm), warm_bytes / 16, sink,
                                                     nullptr);
    check(hipEventRecord(stop, stream), "record");
    check(hipEventSynchronize(stop), "sync");
    float ms = 0;
    check(hipEventElapsedTime(&ms, start, stop), "elapsed");
    if (r > 0) us.push_back(double(ms) * 1000.0);
  }
  check(hipGetLastError(), "launch");
  std::sort(us.begin(), us.end());
  const double median = us[us.size() / 2];
  check(hipEventDestroy(start), "destroy");
  check(hipEventDestroy(stop), "destroy");
  return {median, double(2 * cold_bytes) / (median * 1e3)};
}

}  // namespace

int main(int argc, char** argv) {
  int reps = 20;
  for (int i = 1; i < argc; ++i)
    if (std::strcmp(argv[i], "--reps") == 0 && i + 1 < argc) reps = std::max(1, std::atoi(argv[++i]));

  hipDeviceProp_t props;
  check(hipGetDeviceProperties(&props, 0), "hipGetDeviceProperties");
  const int grid = props.multiProcessorCount * 8;  // 8 workgroups per CU, a multiple of the 8 XCDs

  const int64_t GiB = int64_t(1) << 30, MiB = int64_t(1) << 20;
  float *dram = nullptr, *flush = nullptr, *sink = nullptr;
  check(hipMalloc(&dram, size_t(GiB)), "hipMalloc");
  check(hipMalloc(&flush, size_t(GiB)), "hipMalloc");
  check(hipMalloc(&sink, size_t(grid) * kThreads * sizeof(float)), "hipMalloc");
  check(hipMemset(dram, 0, size_t(GiB)), "hipMemset");
  check(hipMemset(flush, 0, size_t(GiB)), "hipMemset");
  hipStream_t stream;
  check(hipStreamCreate(&stream), "hipStreamCreate");

  struct Case {
    const char* name;
    int64_t bytes;
    int passes;
    bool flushed;
    int64_t region;  // bytes per workgroup (0: strided sweep)
  };
  const Case cases[] = {{"dram", GiB, 1, true, 0},
                        {"mall", 96 * MiB, 4, false, 0},
                        {"l2", 16 * MiB, 8, false, 0},
                        {"dram_regions_48k", 168 * MiB, 1, true, 48 * 1024},
                        {"dram_regions_8k", 168 * MiB, 1, true, 8 * 1024}};
  for (const Case& c : cases) {
    for (const bool nt : {false, true}) {
      const Result r = nt ? run<true>(dram, c.bytes, c.passes, c.flushed ? flush : nullptr, GiB, reps, grid, sink,
                                      stream, c.region)
                          : run<false>(dram, c.bytes, c.passes, c.flushed ? flush : nullptr, GiB, reps, grid, sink,
                                       stream, c.region);
      const int launched = c.region > 0 ? int(c.bytes / c.region) : grid;
      std::printf("{\"case\": \"%s\", \"loads\": \"%s\", \"bytes_per_pass\": %lld, \"passes\": %d, \"median_us\": "
                  "%.2f, \"GB_per_s\": %.1f, \"grid\": %d, \"reps\": %d}\n",
                  c.name, nt ? "nontemporal" : "plain", static_cast<long long>(c.bytes), c.passes, r.median_us,
                  r.gbps, launched, reps);
      std::fflush(stdout);
    }
  }
  {
    // Write ceiling: 1 GiB of zeros into `dram` (which holds zeros).
    hipEvent_t start, stop;
    check(hipEventCreate(&start), "hipEventCreate");
    check(hipEventCreate(&stop), "hipEventCreate");
    std::vector<double> us;
    for (int r = 0; r < reps + 1; ++r) {
      read_kernel<false><<<grid, kThreads, 0, stream>>>(reinterpret_cast<const f32x4*>(flush), GiB / 16, 1, sink);
      check(hipEventRecord(start, stream), "record");
      write_kernel<<<grid, kThreads, 0, stream>>>(reinterpret_cast<f32x4*>(dram), GiB / 16);
      check(hipEventRecord(stop, stream), "record");
      check(hipEventSynchronize(stop), "sync");
      float ms = 0;
      check(hipEventElapsedTime(&ms, start, stop), "elapsed");
      if (r > 0) us.push_back(double(ms) * 1000.0);
    }
    check(hipGetLastError(), "launch");
    std::sort(us.begin(), us.end());
    const double median = us[us.size() / 2];
    std::printf("{\"case\": \"write\", \"stores\": \"plain\", \"bytes_per_pass\": %lld, \"passes\": 1, "
                "\"median_us\": %.2f, \"GB_per_s\": %.1f, \"grid\": %d, \"reps\": %d}\n",
                static_cast<long long>(GiB), median, double(GiB) / (median * 1e3), grid, reps);
    std::fflush(stdout);
    check(hipEventDestroy(start), "destroy");
    check(hipEventDestroy(stop), "destroy");
  }
  {
    // The mixed case reads the first 168 MiB of `dram` cold and the last
    // 84 MiB of `flush` warm (the rest of `flush` is the flush); it counts
    // 2 x 168 MiB per launch.
    const int64_t cold_bytes = 168 * MiB, warm_bytes = 84 * MiB;
    const Result r = run_mixed(dram, cold_bytes, flush + (GiB - warm_bytes) / 4, warm_bytes, flush, GiB - warm_bytes,
                               reps, grid, sink, stream);
    std::printf("{\"case\": \"mixed\", \"loads\": \"nontemporal cold + plain warm\", \"bytes_per_pass\": %lld, "
                "\"passes\": 1, \"median_us\": %.2f, \"GB_per_s\": %.1f, \"grid\": %d, \"reps\": %d}\n",
                static_cast<long long>(2 * cold_bytes), r.median_us, r.gbps, grid, reps);
    std::fflush(stdout);
    // The same with stores on every odd iteration: a lane iterates at most
    // ceil(cold / stride) times, and its odd iterations write rows
    // 0 .. iterations / 2 of a grid x kThreads array of 16-byte vectors.
    const int64_t stride = int64_t(grid) * kThreads * kUnroll;
    const int64_t iterations = (cold_bytes / 16 + stride - 1) / stride;
    const int64_t out_vectors = (iterations / 2 + 1) * grid * 2 * kThreads;  // room for write modes 1-3
    int64_t written = 0;  // vectors stored: lanes whose odd iteration j runs
    for (int64_t j = 1; j < iterations; j += 2)
      for (int64_t b = 0; b < grid; ++b)
        written += std::clamp<int64_t>(cold_bytes / 16 - j * stride - b * kThreads * kUnroll, 0, kThreads);
    float* out = nullptr;
    check(hipMalloc(&out, size_t(out_vectors) * 16), "hipMalloc");
    const char* write_names[] = {"", "mixed_write", "mixed_write_half_lines", "mixed_write_shared_lines"};
    for (int mode = 1; mode <= 3; ++mode) {
      const Result w = run_mixed(dram, cold_bytes, flush + (GiB - warm_bytes) / 4, warm_bytes, flush,
                                 GiB - warm_bytes, reps, grid, sink, stream, 0, out, mode);
      std::printf("{\"case\": \"%s\", \"loads\": \"nontemporal cold + plain warm + plain stores\", "
                  "\"bytes_per_pass\": %lld, \"bytes_written\": %lld, \"passes\": 1, \"median_us\": %.2f, "
                  "\"GB_per_s\": %.1f, \"grid\": %d, \"reps\": %d}\n",
                  write_names[mode], static_cast<long long>(2 * cold_bytes), static_cast<long long>(written * 16),
                  w.median_us, w.gbps, grid, reps);
      std::fflush(stdout);
    }
    check(hipFree(out), "hipFree");
    // B-shaped warm reads: a 145,304 x 32 panel (18.6 MB) at the end of `flush`.
    const int64_t k_rows = 145304, panel_bytes = k_rows * 32 * 4;
    const Result s = run_mixed(dram, cold_bytes, flush + (GiB - panel_bytes) / 4, panel_bytes, flush,
                               GiB - panel_bytes - 4096, reps, grid, sink, stream, k_rows);
    std::printf("{\"case\": \"mixed_segments\", \"loads\": \"nontemporal cold + plain 64-byte B segments\", "
                "\"bytes_per_pass\": %lld, \"passes\": 1, \"median_us\": %.2f, \"GB_per_s\": %.1f, \"grid\": %d, "
                "\"reps\": %d}\n",
                static_cast<long long>(2 * cold_bytes), s.median_us, s.gbps, grid, reps);
    std::fflush(stdout);
  }
  check(hipStreamDestroy(stream), "hipStreamDestroy");
  check(hipFree(dram), "hipFree");
  check(hipFree(flush), "hipFree");
  check(hipFree(sink), "hipFree");
  return 0;
}
