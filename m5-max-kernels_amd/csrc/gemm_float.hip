// C-ABI entry point of the BF16/FP16/FP32 linear (FP32 accumulation); kernels in gemm_launch.h.
#include "gemm_launch.h"

using namespace m5k;
using namespace m5k::gemm;
using namespace m5k::gemm::detail;

extern "C" int m5k_gemm_float(const void* a, const void* b, int ab_dtype, int64_t m, int64_t n, int64_t k,
                              void* c, int c_dtype, const void* residual, const void* gate,
                              const int32_t* gate_row_map, void* stream) {
  clear_error();
  const char* name = "m5k_gemm_float";
  if (int rc = check_shape(m, n, k, name)) return rc;
  M5K_REQUIRE(a && b && c, "%s: null pointer", name);
  M5K_REQUIRE((residual == nullptr) == (gate == nullptr), "%s: residual and gate go together", name);
  M5K_REQUIRE(!gate_row_map || gate, "%s: gate_row_map requires gate", name);
  M5K_REQUIRE(!residual || (c_dtype == M5K_BF16 && ab_dtype == M5K_BF16),
              "%s: gated epilogue requires BF16 operands and output", name);
  EpiParams p{nullptr, nullptr, c, nullptr, nullptr, static_cast<const uint16_t*>(residual),
              static_cast<const uint16_t*>(gate), gate_row_map};
  hipStream_t st = as_stream(stream);
  if (ab_dtype == M5K_BF16) {
    switch (c_dtype) {
      case M5K_BF16: return launch_plain<BF16, M5K_BF16>(a, b, m, n, k, p, st, name);
      case M5K_F16: return launch_plain<BF16, M5K_F16>(a, b, m, n, k, p, st, name);
      case M5K_F32: return launch_plain<BF16, M5K_F32>(a, b, m, n, k, p, st, name);
      default: break;
    }
  } else if (ab_dtype == M5K_F32 && !residual) {
    switch (c_dtype) {
      case M5K_BF16: return launch<F32, M5K_BF16, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
      case M5K_F16: return launch<F32, M5K_F16, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
      case M5K_F32: return launch<F32, M5K_F32, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
      default: break;
    }
  } else if (ab_dtype == M5K_F16) {
    switch (c_dtype) {
      case M5K_BF16: return launch<F16, M5K_BF16, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
      case M5K_F16: return launch<F16, M5K_F16, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
      case M5K_F32: return launch<F16, M5K_F32, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
      default: break;
    }
  }
  set_error("%s: unsupported dtypes operands=%d output=%d", name, ab_dtype, c_dtype);
  return M5K_EINVAL;
}
