// C++ API test: the reference's test program (tests/test_main.cpp) restated
// against this library's C++ API (include/varblockspmm/vbsr.hpp), with the
// gaps it leaves closed: outputs are poisoned with NaN before every run, the
// order-preserving kernel is checked bit for bit against the oracle's fmaf
// emulation, repeated runs must be bit-identical, and the stricter
// normwise/elementwise bounds are checked too.  The reference values come
// from the CPU oracle (oracle/vbsr_oracle.h).  Needs a GPU.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>
#include <functional>
#include <iostream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <varblockspmm/vbsr.hpp>

extern "C" {
#include "vbsr_oracle.h"
}

namespace {

void hip_ok(hipError_t status, const char* what) {
  if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

orc_view oracle_view(const vbsr::HostMatrix& m) {
  orc_view v{};
  v.block_rows = m.block_rows;
  v.block_cols = m.block_cols;
  v.row_ptr = m.row_ptr.data(); v.row_ptr_len = int64_t(m.row_ptr.size());
  v.block_col = m.block_col.data(); v.block_col_len = int64_t(m.block_col.size());
  v.row_size = m.row_size.data(); v.row_size_len = int64_t(m.row_size.size());
  v.col_size = m.col_size.data(); v.col_size_len = int64_t(m.col_size.size());
  v.row_scalar_off = m.row_scalar_off.data(); v.row_scalar_off_len = int64_t(m.row_scalar_off.size());
  v.col_scalar_off = m.col_scalar_off.data(); v.col_scalar_off_len = int64_t(m.col_scalar_off.size());
  v.value_off = m.value_off.data(); v.value_off_len = int64_t(m.value_off.size());
  v.values = m.values.data(); v.values_len = int64_t(m.values.size());
  return v;
}

struct DeviceBuffer {
  float* ptr{};
  size_t count{};
  explicit DeviceBuffer(size_t n) : count(n) { hip_ok(hipMalloc(&ptr, std::max<size_t>(n, 1) * sizeof(float)), "hipMalloc"); }
  ~DeviceBuffer() { (void)hipFree(ptr); }
  std::vector<float> read() const {
    std::vector<float> out(count);
    hip_ok(hipMemcpy(out.data(), ptr, count * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return out;
  }
  void poison() {
    std::vector<float> nan(count, std::nanf(""));
    hip_ok(hipMemcpy(ptr, nan.data(), count * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
};

// Reference tolerance (tests/test_main.cpp:14-40) plus the library's bounds.
void compare(const std::vector<float>& result, const std::vector<float>& reference,
             const std::vector<double>& bound, const std::string& name) {
  double max_err = 0, sq_err = 0, ref_norm = 0, ref_max = 0, bound_max = 0;
  for (size_t i = 0; i < result.size(); ++i) {
    if (!std::isfinite(result[i])) throw std::runtime_error(name + " produced NaN/Inf");
    const double e = double(result[i]) - reference[i];
    max_err = std::max(max_err, std::abs(e));
    sq_err += e * e;
    ref_norm += double(reference[i]) * reference[i];
    ref_max = std::max(ref_max, std::abs(double(reference[i])));
    bound_max = std::max(bound_max, bound[i]);
  }
  const double rel = std::sqrt(sq_err / (ref_norm + 1e-30));
  const double normwise = max_err / (ref_max + 1e-30);
  const double elementwise = max_err / (bound_max + 1e-30);
  if (max_err > 5e-4 || rel > 5e-5 || normwise > 1e-5 || elementwise > 1e-6)
    throw std::runtime_error(name + " mismatch: max=" + std::to_string(max_err) + " rel=" + std::to_string(rel) +
                             " normwise=" + std::to_string(normwise) + " elementwise=" + std::to_string(elementwise));
}

void expect_invalid_argument(const std::function<void()>& op, const char* failure) {
  try {
    op();
  } catch (const std::invalid_argument&) {
    return;
  }
  throw std::runtime_error(failure);
}

// tests/test_main.cpp:116-143
void run_negative_tests() {
  vbsr::GeneratorOptions options;
  options.block_rows = 4;
  options.block_cols = 4;
  options.degree = 2;
  const vbsr::HostMatrix valid = vbsr::generate(options);
  vbsr::HostMatrix bad = valid;
  bad.row_ptr.back()++;
  expect_invalid_argument([&] { bad.validate(); }, "malformed row_ptr accepted");
  bad = valid;
  bad.row_size[0] = 7;
  expect_invalid_argument([&] { bad.validate(); }, "unsupported block size accepted");
  expect_invalid_argument([&] { vbsr::Matrix m(bad); }, "Matrix accepted an invalid host matrix");
  vbsr::Matrix device(valid);
  expect_invalid_argument([&] { vbsr::Plan plan(device, {7, vbsr::Kernel::RowOwned}); }, "invalid RHS accepted");
  // Kernel::SplitRow, reserved and rejected in the reference (test_main.cpp:140), is the split-row path here;
  // kernels outside the enumeration are still rejected.
  if (vbsr::Plan(device, {8, vbsr::Kernel::SplitRow}).launch_count() != 2)
    throw std::runtime_error("split-row plan should take two launches");
  expect_invalid_argument([&] { vbsr::Plan plan(device, {8, static_cast<vbsr::Kernel>(3)}); }, "kernel 3 accepted");
  expect_invalid_argument([&] { vbsr::ScalarCsrPlan plan(valid, 12); }, "CSR plan accepted an invalid RHS");
  expect_invalid_argument([&] { vbsr::ScalarCsrPlan plan(bad, 8); }, "CSR plan accepted an invalid host matrix");
  expect_invalid_argument([&] { vbsr::GroupedGemmPlan plan(valid, 24); }, "grouped plan accepted an invalid RHS");
  expect_invalid_argument([&] { vbsr::GroupedGemmPlan plan(bad, 8); }, "grouped plan accepted an invalid matrix");
  options.degree = 5;
  expect_invalid_argument([&] { vbsr::generate(options); }, "degree > block_cols accepted");
}

// tests/test_main.cpp:61-105 for one case.
void run_case(vbsr::Distribution distribution, int degree, int rhs, bool local, uint64_t seed) {
  vbsr::GeneratorOptions options;
  options.block_rows = 9;
  options.block_cols = 17;
  options.degree = degree;
  options.distribution = distribution;
  options.local_columns = local;
  options.seed = seed;
  const vbsr::HostMatrix host = vbsr::generate(options);
  const orc_view ov = oracle_view(host);

  std::vector<float> input(size_t(host.scalar_cols() * rhs));
  orc_make_random_input(int64_t(input.size()), seed, input.data());
  std::vector<float> reference(size_t(host.scalar_rows() * rhs)), emulated(reference.size());
  std::vector<double> bound(reference.size());
  orc_cpu_reference(&ov, input.data(), int64_t(input.size()), rhs, reference.data());
  orc_fmaf_order(&ov, input.data(), int64_t(input.size()), rhs, emulated.data());
  orc_abs_product_sum(&ov, input.data(), int64_t(input.size()), rhs, bound.data());

  // The library's own cpu_reference, called as test_main.cpp:73 calls it:
  // the reference's arithmetic, so bit-identical to the oracle's.
  const std::vector<float> library_reference = vbsr::cpu_reference(host, input, rhs);
  if (library_reference.size() != reference.size() ||
      std::memcmp(library_reference.data(), reference.data(), reference.size() * sizeof(float)) != 0)
    throw std::runtime_error("vbsr::cpu_reference differs from the oracle (degree " + std::to_string(degree) +
                             ", rhs " + std::to_string(rhs) + ", seed " + std::to_string(seed) + ")");
  std::vector<float> short_input(input.begin(), input.end() - 1);
  expect_invalid_argument([&] { (void)vbsr::cpu_reference(host, short_input, rhs); },
                          "cpu_reference accepted a B of the wrong size");

  vbsr::Matrix device(host);
  DeviceBuffer b(input.size()), c(reference.size());
  hip_ok(hipMemcpy(b.ptr, input.data(), input.size() * sizeof(float), hipMemcpyHostToDevice), "upload B");
  hipStream_t stream;
  hip_ok(hipStreamCreate(&stream), "hipStreamCreate");

  const std::string tag = " (degree " + std::to_string(degree) + ", rhs " + std::to_string(rhs) + ", seed " +
                          std::to_string(seed) + ")";
  vbsr::Plan split(device, {rhs, vbsr::Kernel::SplitRow});
  c.poison();
  split.execute(b.ptr, c.ptr, stream);
  hip_ok(hipStreamSynchronize(stream), "sync");
  compare(c.read(), reference, bound, "split-row" + tag);
  vbsr::Plan plan(device, {rhs, vbsr::Kernel::RowOwned});
  if (plan.launch_count() != 1) throw std::runtime_error("launch_count != 1" + tag);
  c.poison();
  plan.execute(b.ptr, c.ptr, stream);
  hip_ok(hipStreamSynchronize(stream), "sync");
  const std::vector<float> first = c.read();
  compare(first, reference, bound, "row-owned MFMA" + tag);
  c.poison();
  plan.execute(b.ptr, c.ptr, stream);
  hip_ok(hipStreamSynchronize(stream), "sync");
  if (std::memcmp(first.data(), c.read().data(), first.size() * sizeof(float)) != 0)
    throw std::runtime_error("row-owned MFMA not bit-identical across runs" + tag);

  c.poison();
  vbsr::launch_row_owned_scalar(device.device_view(), b.ptr, c.ptr, rhs, stream);
  hip_ok(hipStreamSynchronize(stream), "sync");
  const std::vector<float> scalar = c.read();
  compare(scalar, reference, bound, "row-owned scalar" + tag);
  if (std::memcmp(scalar.data(), emulated.data(), scalar.size() * sizeof(float)) != 0)
    throw std::runtime_error("row-owned scalar differs from the fmaf-order emulation" + tag);

  // The library baseline, as test_main.cpp:96-97 runs the cuSPARSE plan.
  vbsr::ScalarCsrPlan csr(host, rhs);
  if (csr.workspace_bytes() != 0) throw std::runtime_error("workspace before the first execute" + tag);
  for (int run = 0; run < 2; ++run) {
    c.poison();
    csr.execute(b.ptr, c.ptr, stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    compare(c.read(), reference, bound, "rocSPARSE CSR" + tag);
  }
  vbsr::GroupedGemmPlan grouped(host, rhs);
  if (grouped.launch_count() != degree) throw std::runtime_error("grouped launch_count != degree" + tag);
  c.poison();
  grouped.execute(b.ptr, c.ptr, stream);
  hip_ok(hipStreamSynchronize(stream), "sync");
  compare(c.read(), reference, bound, "grouped rocBLAS" + tag);
  // The one-shot, synchronising forms (reference vbsr.hpp:163-168).
  c.poison();
  vbsr::cusparse_scalar_baseline(host, b.ptr, c.ptr, rhs, stream);
  compare(c.read(), reference, bound, "one-shot rocSPARSE" + tag);
  c.poison();
  vbsr::slot_split_baseline(host, b.ptr, c.ptr, rhs, stream);
  compare(c.read(), reference, bound, "one-shot grouped rocBLAS" + tag);

  hip_ok(hipStreamDestroy(stream), "hipStreamDestroy");
}

// Matrix is move-only (reference vbsr.cpp:128-162), and a Plan keeps a
// non-owning view of the device arrays (reference vbsr.hpp:114-116).  A move
// hands those arrays over without copying them, so a plan built before the
// move keeps working; the moved-from object holds nothing, rejects use with
// std::invalid_argument, and is destroyed harmlessly.  Move assignment frees
// the target's own arrays first; self-assignment keeps them.
void run_move_tests() {
  vbsr::GeneratorOptions options;
  options.block_rows = 9;
  options.block_cols = 17;
  options.degree = 4;
  options.seed = 5;
  const vbsr::HostMatrix host = vbsr::generate(options);
  options.seed = 6;
  const vbsr::HostMatrix other = vbsr::generate(options);
  const int rhs = 32;
  const orc_view ov = oracle_view(host);
  std::vector<float> input(size_t(host.scalar_cols() * rhs));
  orc_make_random_input(int64_t(input.size()), 5, input.data());
  std::vector<float> reference(size_t(host.scalar_rows() * rhs));
  std::vector<double> bound(reference.size());
  orc_cpu_reference(&ov, input.data(), int64_t(input.size()), rhs, reference.data());
  orc_abs_product_sum(&ov, input.data(), int64_t(input.size()), rhs, bound.data());
  DeviceBuffer b(input.size()), c(reference.size());
  hip_ok(hipMemcpy(b.ptr, input.data(), input.size() * sizeof(float), hipMemcpyHostToDevice), "upload B");

  const auto run = [&](const vbsr::Plan& plan, const char* name) {
    c.poison();
    plan.execute(b.ptr, c.ptr);
    hip_ok(hipDeviceSynchronize(), "sync");
    compare(c.read(), reference, bound, name);
  };
  const auto require = [](bool ok, const char* failure) {
    if (!ok) throw std::runtime_error(failure);
  };

  vbsr::Matrix first(host);
  const float* values = first.device_view().values;
  const vbsr::Plan before(first, {rhs, vbsr::Kernel::RowOwned});

  vbsr::Matrix second(std::move(first));
  require(first.handle() == nullptr, "moved-from Matrix still owns a handle");
  require(first.scalar_rows() == 0 && first.scalar_cols() == 0, "moved-from Matrix reports a shape");
  require(second.device_view().values == values, "move construction copied the device arrays");
  require(second.scalar_rows() == host.scalar_rows() && second.scalar_cols() == host.scalar_cols(),
          "moved-to Matrix lost its shape");
  expect_invalid_argument([&] { (void)first.device_view(); }, "moved-from Matrix gave a device view");
  expect_invalid_argument([&] { vbsr::Plan plan(first, {rhs, vbsr::Kernel::RowOwned}); },
                          "Plan accepted a moved-from Matrix");
  run(before, "plan built before a move construction");

  vbsr::Matrix third(other);
  third = std::move(second);
  require(second.handle() == nullptr, "move-assigned-from Matrix still owns a handle");
  require(third.device_view().values == values, "move assignment copied the device arrays");
  vbsr::Matrix& alias = third;
  third = std::move(alias);
  require(third.device_view().values == values, "self move assignment dropped the device arrays");
  run(before, "plan built before a move assignment");
  run(vbsr::Plan(third, {rhs, vbsr::Kernel::RowOwned}), "plan built on a move-assigned Matrix");

  first = std::move(third);  // a moved-from object can be assigned to again
  require(third.handle() == nullptr && first.device_view().values == values, "second move assignment failed");
  run(before, "plan built before two moves");
}

// Plan copies share one handle (vbsr::Plan holds a shared_ptr).  The
// reference's Plan is a stateless view (docs/design.md:15), so a default
// plan and a copy of it may execute at once on two streams.  The matrix is
// one where the split-row path would pay (32 block rows of degree 16), so a
// default plan that took it would share a workspace and race here.  An
// explicit SplitRow plan and its copy do share one: with an event after each
// execute that the other stream waits on, their results stay exact too.
void run_concurrent_copy_tests() {
  vbsr::GeneratorOptions options;
  options.block_rows = 32;
  options.block_cols = 32;
  options.degree = 16;
  options.distribution = vbsr::Distribution::HighVariance;
  options.local_columns = false;
  options.seed = 1;
  const vbsr::HostMatrix host = vbsr::generate(options);
  const int rhs = 64;
  const orc_view ov = oracle_view(host);
  vbsr::Matrix device(host);
  if (!vbsr::split_row_advised(device, rhs)) throw std::runtime_error("split-row not advised at 32 rows, degree 16");
  if (vbsr::split_row_advised(device, 8)) throw std::runtime_error("split-row advised at rhs 8");

  struct Side {
    std::vector<float> input, reference, serial;
    std::vector<double> bound;
    hipStream_t stream{};
  };
  Side sides[2];
  std::vector<std::unique_ptr<DeviceBuffer>> bs, cs;
  for (int i = 0; i < 2; ++i) {
    Side& s = sides[i];
    s.input.resize(size_t(host.scalar_cols() * rhs));
    orc_make_random_input(int64_t(s.input.size()), uint64_t(21 + i), s.input.data());
    s.reference.resize(size_t(host.scalar_rows() * rhs));
    s.bound.resize(s.reference.size());
    orc_cpu_reference(&ov, s.input.data(), int64_t(s.input.size()), rhs, s.reference.data());
    orc_abs_product_sum(&ov, s.input.data(), int64_t(s.input.size()), rhs, s.bound.data());
    bs.push_back(std::make_unique<DeviceBuffer>(s.input.size()));
    cs.push_back(std::make_unique<DeviceBuffer>(s.reference.size()));
    hip_ok(hipMemcpy(bs[i]->ptr, s.input.data(), s.input.size() * sizeof(float), hipMemcpyHostToDevice), "upload B");
    hip_ok(hipStreamCreate(&s.stream), "hipStreamCreate");
  }
  const auto check_plans = [&](const vbsr::Plan& plan, const vbsr::Plan& copy, bool with_events, const char* name) {
    const vbsr::Plan* plans[2] = {&plan, &copy};
    for (int i = 0; i < 2; ++i) {
      cs[i]->poison();
      plans[i]->execute(bs[i]->ptr, cs[i]->ptr, sides[i].stream);
      hip_ok(hipStreamSynchronize(sides[i].stream), "sync");
      sides[i].serial = cs[i]->read();
      compare(sides[i].serial, sides[i].reference, sides[i].bound, std::string(name) + " serial");
      cs[i]->poison();
    }
    hipEvent_t done[2];
    for (auto& e : done) hip_ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    for (int round = 0; round < 20; ++round)
      for (int i = 0; i < 2; ++i) {
        plans[i]->execute(bs[i]->ptr, cs[i]->ptr, sides[i].stream);
        if (with_events) {
          hip_ok(hipEventRecord(done[i], sides[i].stream), "hipEventRecord");
          hip_ok(hipStreamWaitEvent(sides[1 - i].stream, done[i], 0), "hipStreamWaitEvent");
        }
      }
    hip_ok(hipDeviceSynchronize(), "sync");
    for (auto& e : done) hip_ok(hipEventDestroy(e), "hipEventDestroy");
    for (int i = 0; i < 2; ++i) {
      const std::vector<float> out = cs[i]->read();
      if (std::memcmp(out.data(), sides[i].serial.data(), out.size() * sizeof(float)) != 0)
        throw std::runtime_error(std::string(name) + ": interleaved result differs from the serial run");
      compare(out, sides[i].reference, sides[i].bound, name);
    }
  };

  const vbsr::Plan plan(device, {rhs});  // Kernel::Auto
  const vbsr::Plan copy = plan;
  if (plan.launch_count() != 1 || copy.launch_count() != 1)
    throw std::runtime_error("a default plan should run the row-owned kernel (one launch)");
  check_plans(plan, copy, false, "default plan and its copy on two streams");
  const vbsr::Plan split(device, {rhs, vbsr::Kernel::SplitRow});
  const vbsr::Plan split_copy = split;
  if (split.launch_count() != 2) throw std::runtime_error("split-row plan should take two launches");
  check_plans(split, split_copy, true, "split-row plan and its copy, events between the streams");
  for (Side& s : sides) hip_ok(hipStreamDestroy(s.stream), "hipStreamDestroy");
}

// tests/test_main.cpp:145-161
int run_parameter_matrix() {
  const vbsr::Distribution distributions[] = {vbsr::Distribution::Uniform, vbsr::Distribution::LowVariance,
                                              vbsr::Distribution::HighVariance, vbsr::Distribution::Bimodal};
  const int degrees[] = {1, 4, 8, 16};
  const int widths[] = {8, 16, 32, 64};
  uint64_t seed = 11;
  int cases = 0;
  for (const auto distribution : distributions)
    for (const int degree : degrees)
      for (const int rhs : widths) {
        run_case(distribution, degree, rhs, (seed & 1) != 0, seed);
        ++seed;
        ++cases;
      }
  return cases;
}

}  // namespace

int main() {
  try {
    run_negative_tests();
    run_move_tests();
    run_concurrent_copy_tests();
    const int cases = run_parameter_matrix();
    std::cout << "PASS: negative tests + Matrix move and lifetime tests + concurrent plan copies + " << cases
              << " parameter cases (MFMA plan + order-preserving kernel + rocSPARSE CSR plan + grouped "
                 "rocBLAS plan, non-default stream, NaN-poisoned C, bit-identical repeats)\n";
    return 0;
  } catch (const std::exception& error) {
    std::cerr << "FAIL: " << error.what() << '\n';
    return 1;
  }
}
