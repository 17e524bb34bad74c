// C-ABI entry point of the FP8 E4M3 linear (FP32 accumulation); kernels in gemm_launch.h.
#include "gemm_launch.h"

using namespace m5k;
using namespace m5k::gemm;
using namespace m5k::gemm::detail;

extern "C" int m5k_gemm_f8(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                           const float* a_scales, const float* b_scales, void* c, int c_dtype,
                           void* stream) {
  clear_error();
  const char* name = "m5k_gemm_f8";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(a && b && c && a_scales && b_scales, "%s: null pointer", name);
  M5K_REQUIRE(k % 128 == 0, "%s: K=%lld must be a multiple of 128", name, (long long)k);
  EpiParams p{a_scales, b_scales, c, nullptr, nullptr, nullptr, nullptr, nullptr};
  hipStream_t st = as_stream(stream);
  switch (c_dtype) {
    case M5K_BF16: return launch<F8, M5K_BF16, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
    case M5K_F16: return launch<F8, M5K_F16, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
    case M5K_F32: return launch<F8, M5K_F32, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
    default: set_error("%s: unsupported output dtype %d", name, c_dtype); return M5K_EINVAL;
  }
}


// Split-K FP8 linear for short M: `splits` K ranges per output tile, FP32 partials in
// workspace[splits][m][n] (workspace_elems floats at least), then one epilogue pass.
extern "C" int m5k_gemm_f8_splitk(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                                  const float* a_scales, const float* b_scales, void* c, int c_dtype, int splits,
                                  float* workspace, int64_t workspace_elems, void* stream) {
  clear_error();
  const char* name = "m5k_gemm_f8_splitk";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(a && b && c && a_scales && b_scales && workspace, "%s: null operand, scale, output or workspace", name);
  M5K_REQUIRE(k % 128 == 0, "%s: K=%lld must be a multiple of 128", name, (long long)k);
  M5K_REQUIRE(splits >= 1 && splits <= 64, "%s: splits=%d outside [1,64]", name, splits);
  M5K_REQUIRE(dma_ok(a, b, k), "%s: split-K needs 16-byte aligned operands", name);
  M5K_REQUIRE(workspace_elems >= static_cast<int64_t>(splits) * m * n, "%s: workspace holds %lld floats, needs %lld",
              name, (long long)workspace_elems, (long long)(static_cast<int64_t>(splits) * m * n));
  EpiParams p{a_scales, b_scales, c, nullptr, nullptr, nullptr, nullptr, nullptr};
  hipStream_t st = as_stream(stream);
  switch (c_dtype) {
    case M5K_BF16: return launch_f8_splitk<M5K_BF16>(a, b, m, n, k, p, splits, workspace, st, name);
    case M5K_F16: return launch_f8_splitk<M5K_F16>(a, b, m, n, k, p, splits, workspace, st, name);
    case M5K_F32: return launch_f8_splitk<M5K_F32>(a, b, m, n, k, p, splits, workspace, st, name);
    default: set_error("%s: unsupported output dtype %d", name, c_dtype); return M5K_EINVAL;
  }
}
