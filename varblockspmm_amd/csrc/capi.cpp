// extern "C" boundary (include/vbsr.h).  Every entry point catches C++
// exceptions and maps them to status codes: std::invalid_argument ->
// VBSR_INVALID_ARGUMENT, anything else -> VBSR_RUNTIME_ERROR.  The message is
// kept per thread for vbsr_last_error().
#include <exception>
#include <new>

#include <hip/hip_runtime_api.h>

#include "internal.hpp"

struct vbsr_host_matrix {
  vbsr_amd::HostMatrix host;
};
struct vbsr_matrix {
  vbsr_amd::DeviceMatrix device;
  explicit vbsr_matrix(const vbsr_host_view& host) : device(host) {}
};
struct vbsr_plan {
  vbsr_amd::Plan plan;
};
struct vbsr_csr_plan {
  vbsr_amd::CsrPlan plan;
  vbsr_csr_plan(const vbsr_host_view& host, int rhs) : plan(host, rhs) {}
};
struct vbsr_gemm_plan {
  vbsr_amd::GemmPlan plan;
  vbsr_gemm_plan(const vbsr_host_view& host, int rhs) : plan(host, rhs) {}
};

namespace {

thread_local std::string g_last_error;

template <class F>
int guarded(F&& body) {
  try {
    body();
    g_last_error.clear();
    return VBSR_OK;
  } catch (const std::invalid_argument& e) {
    g_last_error = e.what();
    return VBSR_INVALID_ARGUMENT;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return VBSR_RUNTIME_ERROR;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return VBSR_RUNTIME_ERROR;
  } catch (...) {
    g_last_error = "unknown error";
    return VBSR_RUNTIME_ERROR;
  }
}

template <class T>
void require(const T* p, const char* name) {
  if (p == nullptr) throw std::invalid_argument(std::string(name) + " is null");
}

}  // namespace

extern "C" {

const char* vbsr_last_error(void) { return g_last_error.c_str(); }

int vbsr_validate(const vbsr_host_view* host) {
  return guarded([&] {
    require(host, "host");
    vbsr_amd::validate(*host);
  });
}

int vbsr_generate(const vbsr_generator_options* options, vbsr_host_matrix** out) {
  return guarded([&] {
    require(options, "options");
    require(out, "out");
    *out = nullptr;
    auto* m = new vbsr_host_matrix{vbsr_amd::generate(*options)};
    *out = m;
  });
}

int vbsr_host_matrix_view(const vbsr_host_matrix* matrix, vbsr_host_view* out) {
  return guarded([&] {
    require(matrix, "matrix");
    require(out, "out");
    *out = matrix->host.view();
  });
}

void vbsr_host_matrix_destroy(vbsr_host_matrix* matrix) { delete matrix; }

int vbsr_make_random_input(int64_t count, uint64_t seed, float* out) {
  return guarded([&] {
    if (count < 0) throw std::invalid_argument("negative count");
    if (count > 0) require(out, "out");
    vbsr_amd::make_random_input(count, seed, out);
  });
}

int vbsr_cpu_reference(const vbsr_host_view* host, const float* B, int64_t b_len, int32_t rhs, float* C,
                       int64_t c_len) {
  return guarded([&] {
    require(host, "host");
    vbsr_amd::cpu_reference(*host, B, b_len, rhs, C, c_len);
  });
}

int vbsr_matrix_create(const vbsr_host_view* host, vbsr_matrix** out) {
  return guarded([&] {
    require(host, "host");
    require(out, "out");
    *out = nullptr;
    *out = new vbsr_matrix(*host);
  });
}

void vbsr_matrix_destroy(vbsr_matrix* matrix) { delete matrix; }

int vbsr_matrix_device_view(const vbsr_matrix* matrix, vbsr_device_view* out) {
  return guarded([&] {
    require(matrix, "matrix");
    require(out, "out");
    *out = matrix->device.view();
  });
}

int64_t vbsr_matrix_scalar_rows(const vbsr_matrix* matrix) {
  return matrix ? matrix->device.view().scalar_rows : 0;
}

int64_t vbsr_matrix_scalar_cols(const vbsr_matrix* matrix) {
  return matrix ? matrix->device.view().scalar_cols : 0;
}

int vbsr_matrix_row_schedule(const vbsr_matrix* matrix, vbsr_row_schedule* out) {
  return guarded([&] {
    require(matrix, "matrix");
    require(out, "out");
    *out = matrix->device.schedule();
  });
}

int vbsr_plan_create(const vbsr_matrix* matrix, const vbsr_plan_options* options, vbsr_plan** out) {
  return guarded([&] {
    require(matrix, "matrix");
    require(options, "options");
    require(out, "out");
    *out = nullptr;
    *out = new vbsr_plan{vbsr_amd::Plan(matrix->device, *options)};
  });
}

void vbsr_plan_destroy(vbsr_plan* plan) { delete plan; }

int vbsr_plan_execute(const vbsr_plan* plan, const float* B, float* C, hipStream_t stream) {
  return guarded([&] {
    require(plan, "plan");
    plan->plan.execute(B, C, stream);
  });
}

int vbsr_plan_launch_count(const vbsr_plan* plan) { return plan ? plan->plan.launch_count() : 0; }

int vbsr_launch_row_owned(const vbsr_device_view* matrix, const vbsr_row_schedule* schedule,
                          const float* B, float* C, int32_t rhs, hipStream_t stream) {
  return guarded([&] {
    require(matrix, "matrix");
    require(schedule, "schedule");
    vbsr_amd::launch_row_owned(*matrix, *schedule, B, C, rhs, stream);
  });
}

int vbsr_launch_row_owned_wide_b(const vbsr_device_view* matrix, const vbsr_row_schedule* schedule,
                                 const float* B, float* C, int32_t rhs, hipStream_t stream) {
  return guarded([&] {
    require(matrix, "matrix");
    require(schedule, "schedule");
    vbsr_amd::launch_row_owned_wide_b(*matrix, *schedule, B, C, rhs, stream);
  });
}

int vbsr_split_row_workspace_bytes(const vbsr_matrix* matrix, int32_t rhs, int64_t* bytes) {
  return guarded([&] {
    require(matrix, "matrix");
    require(bytes, "bytes");
    if (!vbsr_amd::supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
    *bytes = vbsr_amd::split_workspace_floats(matrix->device.split(), rhs) * int64_t(sizeof(float));
  });
}

int vbsr_matrix_split_row_advised(const vbsr_matrix* matrix, int32_t rhs, int32_t* advised) {
  return guarded([&] {
    require(matrix, "matrix");
    require(advised, "advised");
    if (!vbsr_amd::supported_rhs(rhs)) throw std::invalid_argument("unsupported rhs width");
    *advised = vbsr_amd::split_row_advised(matrix->device.split(), rhs) ? 1 : 0;
  });
}

int vbsr_launch_split_row(const vbsr_matrix* matrix, const float* B, float* C, int32_t rhs, void* workspace,
                          int64_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    require(matrix, "matrix");
    if (workspace_bytes < 0) throw std::invalid_argument("negative workspace size");
    if (reinterpret_cast<uintptr_t>(workspace) % alignof(float) != 0)
      throw std::invalid_argument("workspace must be 4-byte aligned");
    vbsr_amd::launch_split_row(matrix->device.view(), matrix->device.schedule(), matrix->device.split(), B, C, rhs,
                               static_cast<float*>(workspace), workspace_bytes / int64_t(sizeof(float)), stream);
  });
}

int vbsr_launch_split_row_static(const vbsr_matrix* matrix, const float* B, float* C, int32_t rhs,
                                 hipStream_t stream) {
  return guarded([&] {
    require(matrix, "matrix");
    vbsr_amd::launch_split_row_static(matrix->device.view(), matrix->device.schedule(), matrix->device.split(), B, C,
                                      rhs, stream);
  });
}

int vbsr_launch_row_owned_valu(const vbsr_device_view* matrix, const vbsr_row_schedule* schedule, const float* B,
                               float* C, int32_t rhs, hipStream_t stream) {
  return guarded([&] {
    require(matrix, "matrix");
    require(schedule, "schedule");
    vbsr_amd::launch_row_owned_valu(*matrix, *schedule, B, C, rhs, stream);
  });
}

int vbsr_launch_row_owned_scalar(const vbsr_device_view* matrix, const float* B, float* C, int32_t rhs,
                                 hipStream_t stream) {
  return guarded([&] {
    require(matrix, "matrix");
    vbsr_amd::launch_scalar(*matrix, B, C, rhs, stream);
  });
}

int vbsr_csr_plan_create(const vbsr_host_view* host, int32_t rhs, vbsr_csr_plan** out) {
  return guarded([&] {
    require(host, "host");
    require(out, "out");
    *out = nullptr;
    *out = new vbsr_csr_plan(*host, rhs);
  });
}

void vbsr_csr_plan_destroy(vbsr_csr_plan* plan) { delete plan; }

int vbsr_csr_plan_execute(vbsr_csr_plan* plan, const float* B, float* C, hipStream_t stream) {
  return guarded([&] {
    require(plan, "plan");
    plan->plan.execute(B, C, stream);
  });
}

int64_t vbsr_csr_plan_workspace_bytes(const vbsr_csr_plan* plan) {
  return plan ? int64_t(plan->plan.workspace_bytes()) : 0;
}

int vbsr_gemm_plan_create(const vbsr_host_view* host, int32_t rhs, vbsr_gemm_plan** out) {
  return guarded([&] {
    require(host, "host");
    require(out, "out");
    *out = nullptr;
    *out = new vbsr_gemm_plan(*host, rhs);
  });
}

void vbsr_gemm_plan_destroy(vbsr_gemm_plan* plan) { delete plan; }

int vbsr_gemm_plan_execute(vbsr_gemm_plan* plan, const float* B, float* C, hipStream_t stream) {
  return guarded([&] {
    require(plan, "plan");
    plan->plan.execute(B, C, stream);
  });
}

int vbsr_gemm_plan_launch_count(const vbsr_gemm_plan* plan) { return plan ? plan->plan.launch_count() : 0; }

// The one-shot baselines build the plan, execute it and wait for the stream
// before the plan (and its device copies) is released, as the reference's
// do (cusparse_baseline.cu:183-188, slot_split.cu:147-152).
int vbsr_scalar_csr_baseline(const vbsr_host_view* host, const float* B, float* C, int32_t rhs, hipStream_t stream) {
  return guarded([&] {
    require(host, "host");
    vbsr_amd::CsrPlan plan(*host, rhs);
    plan.execute(B, C, stream);
    vbsr_amd::check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
  });
}

int vbsr_slot_split_baseline(const vbsr_host_view* host, const float* B, float* C, int32_t rhs, hipStream_t stream) {
  return guarded([&] {
    require(host, "host");
    vbsr_amd::GemmPlan plan(*host, rhs);
    plan.execute(B, C, stream);
    vbsr_amd::check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
  });
}

}  // extern "C"
