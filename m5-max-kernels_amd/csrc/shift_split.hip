// Conditioning preparation of the shift-split projection (norm-shift-split backend,
// src/m5kernels/norm_hadamard_gemm.py:233-247,459-460 of the reference).
//
// With RMS factor r_i, gamma, and per-conditioning-row scale alpha_p and shift beta_p,
//   (r_i x_i c_p + beta_p) W^T = r_i ((x_i c_p) W^T) + beta_p W^T,   c_p = gamma (1 + alpha_p),
// so a conditioning row p needs two tables, built once per condition:
//   combined[p, j] = float(gamma[j]) * (1 + float(scale[p, j]))          (FP32, in this order)
//   bias[p, n]     = sum_j float(shift[p, j]) * float(W[n, j])            (FP32 accumulation)
// The online projection then quantizes (x c_p) D H with the RMS factor folded into the row
// scale and adds bias[p] in the W8A8 GEMM epilogue.
//
// The bias is P rows against the whole weight: HBM-bound on reading W once (2 N K bytes
// for BF16).  One wave owns one W row; each lane streams 8-element chunks (16-byte loads),
// multiplies them into up to kPB conditioning rows held in registers, and the wave sums its
// lanes with the fixed DPP tree.  Up to kPB rows this reads W once.  More conditioning rows
// make the projection a small GEMM, [P, K] x [N, K]^T, which runs on the BF16/F16/FP32 MFMA
// GEMM with FP32 output instead (W read once per 256-row tile of P).
#include "m5k_common.h"

namespace m5k {
namespace shift_split {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPB = 8;  // conditioning rows per pass

template <int PDT>
__global__ __launch_bounds__(kThreads) void combine_kernel(const void* __restrict__ gamma,
                                                           const void* __restrict__ scale, int64_t total, int64_t k,
                                                           float* __restrict__ combined) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
    combined[i] = load_elem<PDT>(gamma, i % k) * (1.0f + load_elem<PDT>(scale, i));
  }
}

// VEC: k % 8 == 0 and 16-byte aligned operands; otherwise one element per lane step.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void bias_project_kernel(const void* __restrict__ shift,
                                                                const void* __restrict__ w, int np, int64_t n,
                                                                int64_t k, float* __restrict__ bias) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + wave;
  if (row >= n) return;  // whole waves only; the kernel has no barrier
  float acc[kPB];
#pragma unroll
  for (int p = 0; p < kPB; ++p) acc[p] = 0.0f;
  if constexpr (VEC) {
    const int64_t chunks = k / 8;
#pragma unroll 4
    for (int64_t c = lane; c < chunks; c += 64) {
      float wv[8];
      load8<DT>(w, row * k + 8 * c, wv);
#pragma unroll
      for (int p = 0; p < kPB; ++p) {
        if (p < np) {
          float sv[8];
          load8<DT>(shift, p * k + 8 * c, sv);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[p] = __builtin_fmaf(sv[i], wv[i], acc[p]);
        }
      }
    }
  } else {
    for (int64_t j = lane; j < k; j += 64) {
      const float wv = load_elem<DT>(w, row * k + j);
#pragma unroll
      for (int p = 0; p < kPB; ++p)
        if (p < np) acc[p] = __builtin_fmaf(load_elem<DT>(shift, p * k + j), wv, acc[p]);
    }
  }
#pragma unroll
  for (int p = 0; p < kPB; ++p) {
    const float total = wave_sum(acc[p]);
    if (p < np && lane == 0) bias[p * n + row] = total;
  }
}

template <int DT>
int launch_bias(const void* shift, const void* w, int64_t p_rows, int64_t n, int64_t k, float* bias,
                hipStream_t st) {
  if (p_rows > kPB) return m5k_gemm_float(shift, w, DT, p_rows, n, k, bias, M5K_F32, nullptr, nullptr, nullptr, st);
  const int64_t blocks = (n + kWaves - 1) / kWaves;
  M5K_REQUIRE(blocks <= 0x7FFFFFFF, "m5k_shift_split_condition: too many weight rows");
  const int np = static_cast<int>(p_rows);
  const bool vec = k % 8 == 0 && aligned16(shift) && aligned16(w);
  if (vec)
    bias_project_kernel<DT, true>
        <<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st>>>(shift, w, np, n, k, bias);
  else
    bias_project_kernel<DT, false>
        <<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st>>>(shift, w, np, n, k, bias);
  return launch_status("m5k_shift_split_condition");
}

template <int PDT>
int launch_combine(const void* gamma, const void* scale, int64_t p_rows, int64_t k, float* combined,
                   hipStream_t st) {
  const int64_t total = p_rows * k;
  const int64_t want = (total + kThreads - 1) / kThreads;
  const unsigned blocks = static_cast<unsigned>(want < 4096 ? want : 4096);
  combine_kernel<PDT><<<dim3(blocks), dim3(kThreads), 0, st>>>(gamma, scale, total, k, combined);
  return launch_status("m5k_shift_split_condition");
}

}  // namespace
}  // namespace shift_split
}  // namespace m5k

using namespace m5k;
using namespace m5k::shift_split;

extern "C" int m5k_shift_split_condition(const void* gamma, const void* scale, int param_dtype, const void* shift,
                                         const void* w, int operand_dtype, int64_t p_rows, int64_t k, int64_t n,
                                         float* combined, float* bias, void* stream) {
  clear_error();
  const char* name = "m5k_shift_split_condition";
  M5K_REQUIRE(gamma && scale && shift && w && combined && bias, "%s: null pointer", name);
  M5K_REQUIRE(p_rows > 0 && k > 0 && n > 0, "%s: bad shape P=%lld K=%lld N=%lld", name, (long long)p_rows,
              (long long)k, (long long)n);
  M5K_REQUIRE(param_dtype == M5K_BF16 || param_dtype == M5K_F16 || param_dtype == M5K_F32,
              "%s: unsupported parameter dtype %d", name, param_dtype);
  M5K_REQUIRE(operand_dtype == M5K_BF16 || operand_dtype == M5K_F16 || operand_dtype == M5K_F32,
              "%s: unsupported operand dtype %d", name, operand_dtype);
  hipStream_t st = as_stream(stream);
  int rc = param_dtype == M5K_BF16  ? launch_combine<M5K_BF16>(gamma, scale, p_rows, k, combined, st)
           : param_dtype == M5K_F16 ? launch_combine<M5K_F16>(gamma, scale, p_rows, k, combined, st)
                                    : launch_combine<M5K_F32>(gamma, scale, p_rows, k, combined, st);
  if (rc) return rc;
  return operand_dtype == M5K_BF16  ? launch_bias<M5K_BF16>(shift, w, p_rows, n, k, bias, st)
         : operand_dtype == M5K_F16 ? launch_bias<M5K_F16>(shift, w, p_rows, n, k, bias, st)
                                    : launch_bias<M5K_F32>(shift, w, p_rows, n, k, bias, st);
}
