// Per-row symmetric INT8 / FP8-E4M3 activation quantizer for gfx950.
//
// Behaviour follows the reference contract quantize_reference
// (src/m5kernels/numerics.py:29-46) as realised by shaders/quantize.metal:1-38:
//   peak  = max |x|                        (FP32, order-independent => exact)
//   scale = peak == 0 ? 1 : peak / 127     (or / 448 for FP8), IEEE division
//   code  = clamp(rint_even(x / scale), -127, 127)   or  E4M3(x / scale)
// One workgroup of 4 wave64 owns one row.  The row is read once from HBM with
// 16-byte loads and held in VGPRs between the max reduction and the encode, so
// HBM traffic is exactly 2*K (bf16 in) + K (codes out) + 4 bytes per row.
#include "m5k_common.h"

namespace m5k {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// |x| maximum over one 16-byte chunk, as FP32.
template <int DT>
__device__ __forceinline__ float chunk_absmax(const uint4& v) {
  if constexpr (DT == M5K_F32) {
    float m = fabsf(__uint_as_float(v.x));
    m = fmaxf(m, fabsf(__uint_as_float(v.y)));
    m = fmaxf(m, fabsf(__uint_as_float(v.z)));
    return fmaxf(m, fabsf(__uint_as_float(v.w)));
  } else {
    // Non-negative 16-bit floats order like their magnitude bits: integer max is exact.
    uint32_t m = 0;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m = max(m, w[i] & 0x7FFFu);
      m = max(m, (w[i] >> 16) & 0x7FFFu);
    }
    return DT == M5K_BF16 ? bf16_bits_to_f32(m) : f16_bits_to_f32(m);
  }
}

// Encode one 16-byte chunk (8 halfs or 4 floats) and store its 8 or 4 code bytes.
template <int DT, int MODE>
__device__ __forceinline__ void encode_chunk(const uint4& v, float scale, uint8_t* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (DT == M5K_F32) {
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed |= quant_encode<MODE>(__uint_as_float(w[i]), scale) << (8 * i);
    *reinterpret_cast<uint32_t*>(out) = packed;
  } else {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e0 = DT == M5K_BF16 ? bf16_bits_to_f32(w[i] & 0xFFFFu) : f16_bits_to_f32(w[i] & 0xFFFFu);
      const float e1 = DT == M5K_BF16 ? bf16_bits_to_f32(w[i] >> 16) : f16_bits_to_f32(w[i] >> 16);
      const uint32_t pair = quant_encode<MODE>(e0, scale) | (quant_encode<MODE>(e1, scale) << 8);
      if (i < 2) lo |= pair << (16 * i);
      else hi |= pair << (16 * (i - 2));
    }
    *reinterpret_cast<uint2*>(out) = make_uint2(lo, hi);
  }
}

// Vector path: row bytes % 16 == 0 and 16-byte aligned bases.  CPT = 16-byte chunks
// per thread kept in registers; CPT == 0 re-reads the row (very wide rows).
template <int DT, int MODE, int CPT>
__global__ __launch_bounds__(kThreads) void quantize_rows_vec(const uint8_t* __restrict__ x,
                                                                int64_t k, uint8_t* __restrict__ q,
                                                                float* __restrict__ scales) {
  __shared__ float red[kWaves];
  constexpr int EPC = 16 / dtype_bytes<DT>();  // elements per chunk
  const int64_t row = blockIdx.x;
  const int64_t nchunks = k / EPC;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * k * dtype_bytes<DT>());
  uint8_t* qr = q + row * k;
  const int tid = threadIdx.x;

  float peak = 0.0f;
  if constexpr (CPT > 0) {
    uint4 v[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int64_t c = tid + (int64_t)i * kThreads;
      v[i] = c < nchunks ? xr[c] : make_uint4(0, 0, 0, 0);
      peak = fmaxf(peak, chunk_absmax<DT>(v[i]));
    }
    peak = block_max<kWaves>(peak, red);
    const float scale = quant_scale<MODE>(peak);
    if (tid == 0) scales[row] = scale;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int64_t c = tid + (int64_t)i * kThreads;
      if (c < nchunks) encode_chunk<DT, MODE>(v[i], scale, qr + c * EPC);
    }
  } else {
    for (int64_t c = tid; c < nchunks; c += kThreads) peak = fmaxf(peak, chunk_absmax<DT>(xr[c]));
    peak = block_max<kWaves>(peak, red);
    const float scale = quant_scale<MODE>(peak);
    if (tid == 0) scales[row] = scale;
    for (int64_t c = tid; c < nchunks; c += kThreads) encode_chunk<DT, MODE>(xr[c], scale, qr + c * EPC);
  }
}

// Scalar path for any K / alignment.
template <int DT, int MODE>
__global__ __launch_bounds__(kThreads) void quantize_rows_scalar(const void* __restrict__ x, int64_t k,
                                                                   uint8_t* __restrict__ q,
                                                                   float* __restrict__ scales) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const int64_t base = row * k;
  float peak = 0.0f;
  for (int64_t j = threadIdx.x; j < k; j += kThreads) peak = fmaxf(peak, fabsf(load_elem<DT>(x, base + j)));
  peak = block_max<kWaves>(peak, red);
  const float scale = quant_scale<MODE>(peak);
  if (threadIdx.x == 0) scales[row] = scale;
  for (int64_t j = threadIdx.x; j < k; j += kThreads)
    q[base + j] = static_cast<uint8_t>(quant_encode<MODE>(load_elem<DT>(x, base + j), scale));
}

template <int DT, int MODE>
int launch_quantize(const void* x, int64_t rows, int64_t k, void* q, float* s, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  const int64_t row_bytes = k * dtype_bytes<DT>();
  const bool vec = row_bytes % 16 == 0 && aligned16(x) && aligned16(q) && (k % 8 == 0 || DT == M5K_F32) &&
                   (k % 4 == 0);
  auto* xb = static_cast<const uint8_t*>(x);
  auto* qb = static_cast<uint8_t*>(q);
  if (vec) {
    const int64_t chunks = row_bytes / 16;
    if (chunks <= kThreads * 1) quantize_rows_vec<DT, MODE, 1><<<grid, block, 0, st>>>(xb, k, qb, s);
    else if (chunks <= kThreads * 2) quantize_rows_vec<DT, MODE, 2><<<grid, block, 0, st>>>(xb, k, qb, s);
    else if (chunks <= kThreads * 4) quantize_rows_vec<DT, MODE, 4><<<grid, block, 0, st>>>(xb, k, qb, s);
    else if (chunks <= kThreads * 8) quantize_rows_vec<DT, MODE, 8><<<grid, block, 0, st>>>(xb, k, qb, s);
    else if (chunks <= kThreads * 16) quantize_rows_vec<DT, MODE, 16><<<grid, block, 0, st>>>(xb, k, qb, s);
    else quantize_rows_vec<DT, MODE, 0><<<grid, block, 0, st>>>(xb, k, qb, s);
  } else {
    quantize_rows_scalar<DT, MODE><<<grid, block, 0, st>>>(x, k, qb, s);
  }
  return launch_status("m5k_quantize_rows");
}

template <int DT>
int dispatch_mode(int mode, const void* x, int64_t rows, int64_t k, void* q, float* s, hipStream_t st) {
  return mode == M5K_QUANT_FP8 ? launch_quantize<DT, M5K_QUANT_FP8>(x, rows, k, q, s, st)
                               : launch_quantize<DT, M5K_QUANT_INT8>(x, rows, k, q, s, st);
}

}  // namespace
}  // namespace m5k

extern "C" int m5k_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int mode, void* q,
                                 float* scales, void* stream) {
  using namespace m5k;
  clear_error();
  M5K_REQUIRE(x && q && scales, "m5k_quantize_rows: null pointer");
  M5K_REQUIRE(rows > 0 && k > 0, "m5k_quantize_rows: empty shape [%lld,%lld]", (long long)rows, (long long)k);
  M5K_REQUIRE(rows <= 0x7FFFFFFF, "m5k_quantize_rows: too many rows");
  M5K_REQUIRE(mode == M5K_QUANT_INT8 || mode == M5K_QUANT_FP8, "m5k_quantize_rows: unknown mode %d", mode);
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return dispatch_mode<M5K_BF16>(mode, x, rows, k, q, scales, st);
    case M5K_F16: return dispatch_mode<M5K_F16>(mode, x, rows, k, q, scales, st);
    case M5K_F32: return dispatch_mode<M5K_F32>(mode, x, rows, k, q, scales, st);
    default: set_error("m5k_quantize_rows: unsupported input dtype %d", x_dtype); return M5K_EINVAL;
  }
}
