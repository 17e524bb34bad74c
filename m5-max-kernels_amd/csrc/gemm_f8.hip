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

