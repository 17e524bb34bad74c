// C-ABI entry points of the W8A8 (INT8 x INT8 -> INT32) linear; kernels in gemm_launch.h.
#include <cstdio>
#include <mutex>

#include "gemm_launch.h"

using namespace m5k;
using namespace m5k::gemm;
using namespace m5k::gemm::detail;

extern "C" int m5k_gemm_i8(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                           const float* a_scales, const float* b_scales, void* c, int c_dtype,
                           const float* bias, const int32_t* bias_row_map, const void* residual,
                           const void* gate, const int32_t* gate_row_map, void* stream) {
  clear_error();
  const char* name = "m5k_gemm_i8";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(a && b && c && a_scales && b_scales, "%s: null operand, scale or output pointer", name);
  M5K_REQUIRE(k <= 133144, "%s: K=%lld exceeds the INT32 worst-case bound 133144", name, (long long)k);
  M5K_REQUIRE(!bias_row_map || bias, "%s: bias_row_map requires bias", name);
  M5K_REQUIRE((residual == nullptr) == (gate == nullptr), "%s: residual and gate go together", name);
  M5K_REQUIRE(!gate_row_map || gate, "%s: gate_row_map requires gate", name);
  M5K_REQUIRE(!(bias && residual), "%s: bias and gated residual cannot be combined", name);
  M5K_REQUIRE(!residual || c_dtype == M5K_BF16, "%s: gated epilogue requires BF16 output", name);
  EpiParams p{a_scales, b_scales, c, bias, bias_row_map, static_cast<const uint16_t*>(residual),
              static_cast<const uint16_t*>(gate), gate_row_map};
  hipStream_t st = as_stream(stream);
  switch (c_dtype) {
    case M5K_BF16: return launch_i8<M5K_BF16>(a, b, m, n, k, p, st);
    case M5K_F16: return launch_i8<M5K_F16>(a, b, m, n, k, p, st);
    case M5K_F32: return launch_i8<M5K_F32>(a, b, m, n, k, p, st);
    default: set_error("%s: unsupported output dtype %d", name, c_dtype); return M5K_EINVAL;
  }
}

extern "C" int m5k_gemm_i8_acc(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                               int32_t* acc, void* stream) {
  clear_error();
  const char* name = "m5k_gemm_i8_acc";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(a && b && acc, "%s: null pointer", name);
  M5K_REQUIRE(k <= 133144, "%s: K exceeds the INT32 worst-case bound", name);
  EpiParams p{};
  p.c = acc;
  return launch<I8, M5K_I32, EPI_NONE, EPI_NONE, true>(a, b, m, n, k, p, as_stream(stream), name);
}

extern "C" int m5k_gemm_launch_plan(int ab_dtype, int64_t m, int64_t n, int cus, int* schedule,
                                    int64_t* full_tiles) {
  clear_error();
  const char* name = "m5k_gemm_launch_plan";
  M5K_REQUIRE(schedule != nullptr && full_tiles != nullptr, "%s: null output", name);
  if (int rc = check_shape(m, n, 1, name)) return rc;
  M5K_REQUIRE(cus > 0, "%s: cus must be positive", name);
  M5K_REQUIRE(ab_dtype == M5K_I8 || ab_dtype == M5K_U8 || ab_dtype == M5K_BF16 || ab_dtype == M5K_F16 ||
                  ab_dtype == M5K_F32,
              "%s: ab_dtype must be I8, U8 (FP8 codes), BF16, F16 or F32", name);
  const bool md16 = ab_dtype == M5K_I8 || ab_dtype == M5K_BF16 || ab_dtype == M5K_F16;
  *schedule = plan_schedule(md16, ab_dtype == M5K_I8, m, n, cus, *full_tiles);
  return M5K_OK;
}

extern "C" int m5k_gemm_set_schedule(int schedule, int* previous) {
  clear_error();
  M5K_REQUIRE(schedule >= -1 && schedule <= SCHED_QUAD, "m5k_gemm_set_schedule: schedule %d outside [-1, 3]",
              schedule);
  if (previous) *previous = g_thread_schedule;
  g_thread_schedule = schedule;
  return M5K_OK;
}

namespace {

// Split-K partials of m5k_gemm_i8_splitk_noalloc.  The name is a host-side stand-in: host code
// uses only the per-device address that hipGetSymbolAddress returns.
static __device__ __align__(256) int32_t scratch[M5K_SCRATCH_ELEMS];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch[kMaxDevices] = {};

// The copy of `scratch` on the device that `stream` belongs to (the current device for the null
// stream), looked up once per device with that device current and cached.
int scratch_of_stream_device(hipStream_t stream, int32_t** out, const char* name) {
  int current = -1;
  M5K_REQUIRE(hipGetDevice(&current) == hipSuccess && current >= 0, "%s: no current HIP device", name);
  int dev = current;
  if (stream != nullptr) {
    hipDevice_t sd = -1;
    const hipError_t e = hipStreamGetDevice(stream, &sd);
    M5K_REQUIRE(e == hipSuccess, "%s: hipStreamGetDevice failed: %s", name, hipGetErrorString(e));
    dev = static_cast<int>(sd);
  }
  M5K_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d outside the supported range", name, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    if (dev != current) M5K_REQUIRE(hipSetDevice(dev) == hipSuccess, "%s: hipSetDevice(%d) failed", name, dev);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != current) (void)hipSetDevice(current);
    M5K_REQUIRE(e == hipSuccess && ptr != nullptr, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name,
                dev, hipGetErrorString(e));
    g_scratch[dev] = static_cast<int32_t*>(ptr);
  }
  *out = g_scratch[dev];
  return M5K_OK;
}

}  // namespace

extern "C" int m5k_gemm_i8_splitk(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                                  const float* a_scales, const float* b_scales, void* c, int c_dtype,
                                  const float* bias, const int32_t* bias_row_map, const void* residual,
                                  const void* gate, const int32_t* gate_row_map, int splits, int32_t* workspace,
                                  int64_t workspace_elems, void* stream) {
  clear_error();
  const char* name = "m5k_gemm_i8_splitk";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(a && b && c && a_scales && b_scales && workspace, "%s: null operand, scale, output or workspace", name);
  M5K_REQUIRE(k <= 133144, "%s: K=%lld exceeds the INT32 worst-case bound 133144", name, (long long)k);
  M5K_REQUIRE(!bias_row_map || bias, "%s: bias_row_map requires bias", name);
  M5K_REQUIRE((residual == nullptr) == (gate == nullptr), "%s: residual and gate go together", name);
  M5K_REQUIRE(!gate_row_map || gate, "%s: gate_row_map requires gate", name);
  M5K_REQUIRE(!(bias && residual), "%s: bias and gated residual cannot be combined", name);
  M5K_REQUIRE(!residual || c_dtype == M5K_BF16, "%s: gated epilogue requires BF16 output", name);
  M5K_REQUIRE(splits >= 1 && splits <= 64, "%s: splits=%d outside [1,64]", name, splits);
  M5K_REQUIRE(dma_ok(a, b, k), "%s: split-K needs 16-byte aligned operands with K %% 16 == 0", name);
  M5K_REQUIRE(workspace_elems >= static_cast<int64_t>(splits) * m * n, "%s: workspace holds %lld INT32, needs %lld",
              name, (long long)workspace_elems, (long long)(static_cast<int64_t>(splits) * m * n));
  EpiParams p{a_scales, b_scales, c, bias, bias_row_map, static_cast<const uint16_t*>(residual),
              static_cast<const uint16_t*>(gate), gate_row_map};
  hipStream_t st = as_stream(stream);
  switch (c_dtype) {
    case M5K_BF16: return launch_i8_splitk<M5K_BF16>(a, b, m, n, k, p, splits, workspace, st, name);
    case M5K_F16: return launch_i8_splitk<M5K_F16>(a, b, m, n, k, p, splits, workspace, st, name);
    case M5K_F32: return launch_i8_splitk<M5K_F32>(a, b, m, n, k, p, splits, workspace, st, name);
    default: set_error("%s: unsupported output dtype %d", name, c_dtype); return M5K_EINVAL;
  }
}

extern "C" int m5k_gemm_i8_splitk_noalloc(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                                          const float* a_scales, const float* b_scales, void* c, int c_dtype,
                                          const float* bias, const int32_t* bias_row_map, const void* residual,
                                          const void* gate, const int32_t* gate_row_map, int splits, void* stream) {
  clear_error();
  const char* name = "m5k_gemm_i8_splitk_noalloc";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(splits >= 1 && splits <= 64, "%s: splits=%d outside [1,64]", name, splits);
  M5K_REQUIRE(static_cast<int64_t>(splits) * m * n <= M5K_SCRATCH_ELEMS,
              "%s: splits*m*n = %lld INT32 partials exceed the %d-element scratch array", name,
              (long long)(static_cast<int64_t>(splits) * m * n), M5K_SCRATCH_ELEMS);
  int32_t* ws = nullptr;
  if (int rc = scratch_of_stream_device(as_stream(stream), &ws, name)) return rc;
  // Every partial that the epilogue reads is written first by the split kernel, so the
  // array needs no clearing between calls.
  const int rc = m5k_gemm_i8_splitk(a, b, m, n, k, a_scales, b_scales, c, c_dtype, bias, bias_row_map, residual, gate,
                                    gate_row_map, splits, ws, M5K_SCRATCH_ELEMS, stream);
  if (rc != M5K_OK) {
    // Report the failure under this entry point's name.
    char detail[512];
    snprintf(detail, sizeof(detail), "%s", m5k_last_error());
    set_error("%s: %s", name, detail);
  }
  return rc;
}
