// vbsr_benchmark: the counterpart of the reference benchmark executable
// (bench/benchmark.cpp).  It generates one matrix, times each method and
// prints one CSV row per method with the reference's columns, in the
// reference's order and meaning (benchmark.cpp:209-225):
//
//   gpu_median_ms / gpu_p95_ms   HIP events around each repetition, run back
//                                to back after the warmup (benchmark.cpp:148-183);
//   hot_median_ms / hot_p95_ms   host wall time of the same repetitions
//                                (record, run, record, wait);
//   useful_gflops                2 * rhs * sum(h * w) / gpu median
//                                (benchmark.cpp:197-207);
//   launches, workspace_bytes    kernels per run, bytes of workspace (the
//                                rocSPARSE plan's, and a split-row plan's).
//
// Columns appended after the reference's: the same repetitions with a 1 GiB
// read-only sweep before each one (inputs in HBM only), the algorithmic bytes
// of one run and the resulting rate, and whether C was bit-identical after
// every repetition.
//
// Timing events are created with hipEventDisableSystemFence: HIP's
// timing-only events, which leave out the system-scope cache writeback and
// invalidate that a default event adds around the kernel.  B is the constant
// 0.01 of the reference benchmark (benchmark.cpp:239) unless --input random
// asks for the reference test's uniform [-1, 1] stream.
//
// Methods: row_owned_hybrid (Plan::execute with Kernel::RowOwned, the
// reference's tuned path, or Kernel::Auto, the same kernel), split_row in its
// place for --kernel split_row, row_owned_scalar (launch_row_owned_scalar) and
// scalar_csr_rocsparse (ScalarCsrPlan, the counterpart of the reference's
// scalar_csr_cusparse row) and slot_grouped_rocblas (GroupedGemmPlan, the
// counterpart of slot_grouped_cublas).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <iomanip>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include <varblockspmm/vbsr.hpp>

namespace {

void hip_check(hipError_t status, const char* what) {
  if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

struct Arguments {
  int rows = 1024;
  int degree = 8;
  int rhs_width = 32;
  int repetitions = 50;
  int warmup_repetitions = 10;
  uint64_t seed = 1;
  std::string locality = "local";
  std::string distribution = "high";
  std::string input = "constant";
  std::string kernel = "row_owned";
  bool cold = true;
  bool header = true;
};

struct Distribution {
  const char* name;
  vbsr::Distribution value;
};
constexpr Distribution kDistributions[] = {
    {"uniform", vbsr::Distribution::Uniform},     {"low", vbsr::Distribution::LowVariance},
    {"high", vbsr::Distribution::HighVariance},   {"bimodal", vbsr::Distribution::Bimodal},
    {"bimodal8or64", vbsr::Distribution::Bimodal8or64}, {"tied8to64", vbsr::Distribution::Tied8to64},
};

vbsr::Distribution parse_distribution(const std::string& value) {
  for (const auto& d : kDistributions)
    if (value == d.name) return d.value;
  throw std::runtime_error("unknown distribution: " + value);
}

void usage() {
  std::cerr << "usage: vbsr_benchmark [--rows N] [--degree D] [--rhs 8|16|32|64] [--reps N] [--warmup N]\n"
               "                      [--seed S] [--locality local|random|clamped]\n"
               "                      [--distribution uniform|low|high|bimodal|bimodal8or64|tied8to64]\n"
               "                      [--input constant|random] [--kernel row_owned|auto|split_row]\n"
               "                      [--no-cold] [--no-header]\n";
}

Arguments parse_arguments(int argc, char** argv) {
  Arguments a;
  for (int i = 1; i < argc; ++i) {
    const std::string option = argv[i];
    auto value = [&]() -> std::string {
      if (++i >= argc) throw std::runtime_error("missing value for " + option);
      return argv[i];
    };
    if (option == "--rows") a.rows = std::stoi(value());
    else if (option == "--degree") a.degree = std::stoi(value());
    else if (option == "--rhs") a.rhs_width = std::stoi(value());
    else if (option == "--reps") a.repetitions = std::stoi(value());
    else if (option == "--warmup") a.warmup_repetitions = std::stoi(value());
    else if (option == "--seed") a.seed = std::stoull(value());
    else if (option == "--locality") a.locality = value();
    else if (option == "--distribution") a.distribution = value();
    else if (option == "--input") a.input = value();
    else if (option == "--kernel") a.kernel = value();
    else if (option == "--no-cold") a.cold = false;
    else if (option == "--no-header") a.header = false;
    else if (option == "--help") { usage(); std::exit(0); }
    else throw std::runtime_error("unknown argument: " + option);
  }
  if (a.repetitions < 1 || a.warmup_repetitions < 0) throw std::runtime_error("--reps must be >= 1, --warmup >= 0");
  if (a.locality != "local" && a.locality != "random" && a.locality != "clamped")
    throw std::runtime_error("unknown locality: " + a.locality);
  if (a.input != "constant" && a.input != "random") throw std::runtime_error("unknown input: " + a.input);
  if (a.kernel != "row_owned" && a.kernel != "auto" && a.kernel != "split_row")
    throw std::runtime_error("unknown kernel: " + a.kernel);
  parse_distribution(a.distribution);
  return a;
}

// Read-only sweep of a buffer larger than L2 and the Infinity Cache together;
// it writes nothing, so no dirty line is left to be written back while the
// next repetition is timed.
__global__ void read_sweep(const float4* __restrict__ p, size_t n, float* out) {
  float acc = 0.0f;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const float4 v = p[i];
    acc += v.x + v.y + v.z + v.w;
  }
  if (acc == 1234.5f) out[blockIdx.x] = acc;  // never true for the zero-filled buffer
}

double percentile_95(const std::vector<double>& sorted) {
  return sorted[std::min(sorted.size() - 1, size_t(double(sorted.size()) * 0.95))];
}

struct Timing {
  double gpu_median, gpu_p95, host_median, host_p95, cold_median, cold_p95;
  bool identical;
};

struct Bench {
  hipStream_t stream{};
  hipEvent_t begin{}, end{};
  float* flush{};
  float* flush_out{};
  size_t flush_vec4 = (size_t(1) << 30) / 16;

  Bench() {
    hip_check(hipStreamCreate(&stream), "hipStreamCreate");
    hip_check(hipEventCreateWithFlags(&begin, hipEventDisableSystemFence), "hipEventCreateWithFlags");
    hip_check(hipEventCreateWithFlags(&end, hipEventDisableSystemFence), "hipEventCreateWithFlags");
  }
  ~Bench() {
    (void)hipFree(flush);
    (void)hipFree(flush_out);
    (void)hipEventDestroy(begin);
    (void)hipEventDestroy(end);
    (void)hipStreamDestroy(stream);
  }
  void flush_caches() {
    if (!flush) {
      hip_check(hipMalloc(&flush, flush_vec4 * 16), "hipMalloc flush");
      hip_check(hipMalloc(&flush_out, 4096 * sizeof(float)), "hipMalloc flush_out");
      hip_check(hipMemset(flush, 0, flush_vec4 * 16), "hipMemset flush");
    }
    read_sweep<<<4096, 256, 0, stream>>>(reinterpret_cast<const float4*>(flush), flush_vec4, flush_out);
    hip_check(hipGetLastError(), "read_sweep launch");
  }

  Timing time(const std::function<void(hipStream_t)>& op, const Arguments& a, const float* c, size_t c_count) {
    for (int i = 0; i < a.warmup_repetitions; ++i) op(stream);
    hip_check(hipStreamSynchronize(stream), "warmup");
    std::vector<float> first(c_count), now(c_count);
    hip_check(hipMemcpy(first.data(), c, c_count * sizeof(float), hipMemcpyDeviceToHost), "copy C");
    bool identical = true;
    auto check = [&] {
      hip_check(hipMemcpy(now.data(), c, c_count * sizeof(float), hipMemcpyDeviceToHost), "copy C");
      identical = identical && std::memcmp(first.data(), now.data(), c_count * sizeof(float)) == 0;
    };
    std::vector<double> gpu, host, cold;
    for (int i = 0; i < a.repetitions; ++i) {
      const auto t0 = std::chrono::steady_clock::now();
      hip_check(hipEventRecord(begin, stream), "hipEventRecord");
      op(stream);
      hip_check(hipEventRecord(end, stream), "hipEventRecord");
      hip_check(hipEventSynchronize(end), "hipEventSynchronize");
      const auto t1 = std::chrono::steady_clock::now();
      float ms = 0.0f;
      hip_check(hipEventElapsedTime(&ms, begin, end), "hipEventElapsedTime");
      gpu.push_back(ms);
      host.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
    }
    check();
    if (a.cold) {
      for (int i = 0; i < a.repetitions; ++i) {
        flush_caches();
        hip_check(hipEventRecord(begin, stream), "hipEventRecord");
        op(stream);
        hip_check(hipEventRecord(end, stream), "hipEventRecord");
        hip_check(hipEventSynchronize(end), "hipEventSynchronize");
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, begin, end), "hipEventElapsedTime");
        cold.push_back(ms);
      }
      check();
    }
    std::sort(gpu.begin(), gpu.end());
    std::sort(host.begin(), host.end());
    std::sort(cold.begin(), cold.end());
    Timing t{};
    t.gpu_median = gpu[gpu.size() / 2];
    t.gpu_p95 = percentile_95(gpu);
    t.host_median = host[host.size() / 2];
    t.host_p95 = percentile_95(host);
    t.cold_median = cold.empty() ? 0.0 : cold[cold.size() / 2];
    t.cold_p95 = cold.empty() ? 0.0 : percentile_95(cold);
    t.identical = identical;
    return t;
  }
};

int run(const Arguments& a) {
  vbsr::GeneratorOptions options;
  options.block_rows = a.rows;
  options.block_cols = a.rows;  // square block grid, as the reference benchmark (benchmark.cpp:188)
  options.degree = a.degree;
  options.rhs_width = a.rhs_width;
  options.distribution = parse_distribution(a.distribution);
  options.local_columns = a.locality != "random";
  options.clamp_local_columns = a.locality == "clamped";
  options.seed = a.seed;
  const vbsr::HostMatrix host = vbsr::generate(options);
  vbsr::Matrix matrix(host);
  const int64_t k = matrix.scalar_cols(), m = matrix.scalar_rows();
  const size_t b_count = size_t(k) * size_t(a.rhs_width), c_count = size_t(m) * size_t(a.rhs_width);

  std::vector<float> input(b_count, 0.01f);
  if (a.input == "random" && b_count > 0)
    if (vbsr_make_random_input(int64_t(b_count), a.seed, input.data()) != VBSR_OK)
      throw std::runtime_error(vbsr_last_error());
  float *b = nullptr, *c = nullptr;
  hip_check(hipMalloc(&b, std::max<size_t>(b_count, 1) * sizeof(float)), "hipMalloc B");
  hip_check(hipMalloc(&c, std::max<size_t>(c_count, 1) * sizeof(float)), "hipMalloc C");
  hip_check(hipMemcpy(b, input.data(), b_count * sizeof(float), hipMemcpyHostToDevice), "copy B");

  double sum_hw = 0.0;  // useful flops / (2 rhs), benchmark.cpp:197-207
  for (int i = 0; i < host.block_rows; ++i)
    for (int blk = host.row_ptr[size_t(i)]; blk < host.row_ptr[size_t(i) + 1]; ++blk)
      sum_hw += double(host.row_size[size_t(i)]) * host.col_size[size_t(host.block_col[size_t(blk)])];
  const double useful_flops = 2.0 * sum_hw * a.rhs_width;
  const double meta = 4.0 * (host.block_rows + 1) + 4.0 * double(host.block_col.size()) + 4.0 * host.block_rows +
                      4.0 * host.block_cols + 8.0 * (host.block_rows + 1) + 8.0 * (host.block_cols + 1) +
                      8.0 * double(host.block_col.size() + 1);
  const double bytes = 4.0 * sum_hw + 4.0 * double(b_count) + 4.0 * double(c_count) + meta;

  const vbsr::Kernel kernel = a.kernel == "auto"        ? vbsr::Kernel::Auto
                              : a.kernel == "split_row" ? vbsr::Kernel::SplitRow
                                                        : vbsr::Kernel::RowOwned;
  vbsr::Plan plan(matrix, {a.rhs_width, kernel});
  const vbsr::DeviceMatrix view = matrix.device_view();
  Bench bench;
  if (a.header)
    std::cout << "method,block_rows,degree,distribution,locality,rhs,seed,"
                 "gpu_median_ms,gpu_p95_ms,hot_median_ms,hot_p95_ms,useful_gflops,"
                 "launches,workspace_bytes,cold_median_ms,cold_p95_ms,algorithmic_bytes,cold_gbs,identical\n";
  auto report = [&](const char* method, const Timing& t, int launches, size_t workspace) {
    std::cout << method << ',' << a.rows << ',' << a.degree << ',' << a.distribution << ',' << a.locality << ','
              << a.rhs_width << ',' << a.seed << ',' << std::fixed << std::setprecision(5) << t.gpu_median << ','
              << t.gpu_p95 << ',' << t.host_median << ',' << t.host_p95 << ','
              << useful_flops / (t.gpu_median * 1e6) << ',' << launches << ',' << workspace << ',' << t.cold_median << ','
              << t.cold_p95 << ',' << std::setprecision(0) << bytes << ',' << std::setprecision(2)
              << (t.cold_median > 0 ? bytes / (t.cold_median * 1e6) : 0.0) << ',' << (t.identical ? 1 : 0) << '\n'
              << std::flush;
  };
  // A split-row plan (two launches) owns the workspace the split-row path
  // needs, and is reported under a method name of its own, so that its rows
  // never mix into the reference's row_owned_hybrid column.
  const bool split_row = kernel == vbsr::Kernel::SplitRow;
  const size_t plan_workspace = split_row ? size_t(vbsr::split_row_workspace_bytes(matrix, a.rhs_width)) : 0;
  report(split_row ? "split_row" : "row_owned_hybrid",
         bench.time([&](hipStream_t s) { plan.execute(b, c, s); }, a, c, c_count), plan.launch_count(),
         plan_workspace);
  report("row_owned_scalar",
         bench.time([&](hipStream_t s) { vbsr::launch_row_owned_scalar(view, b, c, a.rhs_width, s); }, a, c,
                    c_count),
         1, 0);
  vbsr::ScalarCsrPlan csr(host, a.rhs_width);
  const Timing csr_timing = bench.time([&](hipStream_t s) { csr.execute(b, c, s); }, a, c, c_count);
  report("scalar_csr_rocsparse", csr_timing, 1, csr.workspace_bytes());
  vbsr::GroupedGemmPlan grouped(host, a.rhs_width);
  report("slot_grouped_rocblas", bench.time([&](hipStream_t s) { grouped.execute(b, c, s); }, a, c, c_count),
         grouped.launch_count(), 0);
  hip_check(hipFree(b), "hipFree");
  hip_check(hipFree(c), "hipFree");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return run(parse_arguments(argc, argv));
  } catch (const std::exception& error) {
    std::cerr << "error: " << error.what() << '\n';
    return 2;
  }
}
