// Per-row symmetric INT8 / FP8-E4M3 activation quantizer for gfx950.
//
// Behaviour follows the reference contract quantize_reference
// (src/m5kernels/numerics.py:29-46) as realised by shaders/quantize.metal:1-38:
//   peak  = max |x|, NaN ignored           (FP32, order-independent => exact)
//   scale = peak == 0 ? 1 : peak / 127     (or / 448 for FP8), IEEE division
//   code  = clamp(rint_even(x / scale), -127, 127)   or  E4M3(x / scale)
// INT8 codes come from a reciprocal multiply with a grouped exact fallback near rounding
// boundaries (encode_i8), bit-identical to the IEEE division.
//
// A row is read once from HBM with 16-byte loads and held in VGPRs between the max
// reduction and the encode, so HBM traffic is exactly 2*K (bf16 in) + K (codes out) + 4
// bytes per row.  Each row has its own workgroup of 4 wave64.  With the encode at about
// eight VALU ops per element the kernel runs within ~15% of a plain copy of the same bytes;
// a persistent grid with a one-row register prefetch measured no faster.
#include "m5k_common.h"

namespace m5k {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float half_to_f32(uint32_t bits16) {
  return DT == M5K_BF16 ? bf16_bits_to_f32(bits16) : f16_bits_to_f32(bits16);
}

// Largest |x| over a thread's CPT 16-byte chunks, as FP32, NaN ignored like the reference's
// max (quantize.metal:7).  16-bit inputs: non-negative halfs order like their magnitude bits,
// so one packed u16 max per word covers two elements; magnitude bits above infinity's mean a
// NaN, and that thread recomputes its maximum in FP32.
template <int DT, int CPT>
__device__ __forceinline__ float thread_absmax(const uint4 (&v)[CPT]) {
  if constexpr (DT == M5K_F32) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      m = fmaxf(m, fabsf(__uint_as_float(v[i].x)));
      m = fmaxf(m, fabsf(__uint_as_float(v[i].y)));
      m = fmaxf(m, fabsf(__uint_as_float(v[i].z)));
      m = fmaxf(m, fabsf(__uint_as_float(v[i].w)));
    }
    return m;
  } else {
    u16x2 acc = {0, 0};
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, w[j] & 0x7FFF7FFFu));
    }
    const uint32_t bits = acc.x > acc.y ? acc.x : acc.y;
    constexpr uint32_t kInfBits = DT == M5K_BF16 ? 0x7F80u : 0x7C00u;
    if (bits <= kInfBits) return half_to_f32<DT>(bits);
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m = fmaxf(m, fabsf(half_to_f32<DT>(w[j] & 0xFFFFu)));
        m = fmaxf(m, fabsf(half_to_f32<DT>(w[j] >> 16)));
      }
    }
    return m;
  }
}

// Encode one 16-byte chunk (8 halfs or 4 floats) and store its 8 or 4 code bytes.
template <int DT, int MODE>
__device__ __forceinline__ void encode_chunk(const uint4& v, const I8Scale& s, uint8_t* out) {
  constexpr int EPC = 16 / dtype_bytes<DT>();
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float f[EPC];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (DT == M5K_F32) {
      f[j] = __uint_as_float(w[j]);
    } else {
      f[2 * j] = half_to_f32<DT>(w[j] & 0xFFFFu);
      f[2 * j + 1] = half_to_f32<DT>(w[j] >> 16);
    }
  }
  uint32_t packed[EPC / 4];
  if constexpr (MODE == M5K_QUANT_INT8) {
    encode_i8<EPC>(f, s, packed);
  } else {
#pragma unroll
    for (int j = 0; j < EPC / 4; ++j) {
      packed[j] = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) packed[j] |= fp8_e4m3_encode(f[4 * j + b] / s.scale) << (8 * b);
    }
  }
  if constexpr (EPC == 8) *reinterpret_cast<uint2*>(out) = make_uint2(packed[0], packed[1]);
  else *reinterpret_cast<uint32_t*>(out) = packed[0];
}

// Load a row's chunks tid, tid + 256, ... into registers; chunks past the row read as zero.
template <int CPT>
__device__ __forceinline__ void load_row(const uint4* __restrict__ xr, int64_t nchunks, int tid, uint4 (&v)[CPT]) {
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = tid + (int64_t)i * kThreads;
    v[i] = c < nchunks ? xr[c] : make_uint4(0, 0, 0, 0);
  }
}

template <int DT, int MODE, int CPT>
__device__ __forceinline__ void store_row(const uint4 (&v)[CPT], const I8Scale& s, int64_t nchunks, int tid,
                                          uint8_t* __restrict__ qr) {
  constexpr int EPC = 16 / dtype_bytes<DT>();
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = tid + (int64_t)i * kThreads;
    if (c < nchunks) encode_chunk<DT, MODE>(v[i], s, qr + c * EPC);
  }
}

// One workgroup per row: row bytes % 16 == 0 and 16-byte aligned bases.  CPT = 16-byte
// chunks per thread kept in registers.
template <int DT, int MODE, int CPT>
__global__ __launch_bounds__(kThreads) void quantize_rows_vec(const uint8_t* __restrict__ x, int64_t k,
                                                                uint8_t* __restrict__ q,
                                                                float* __restrict__ scales) {
  __shared__ float red[kWaves];
  constexpr int EPC = 16 / dtype_bytes<DT>();
  const int64_t row = blockIdx.x;
  const int64_t nchunks = k / EPC;
  const int tid = threadIdx.x;
  uint4 v[CPT];
  load_row<CPT>(reinterpret_cast<const uint4*>(x + row * k * dtype_bytes<DT>()), nchunks, tid, v);
  const float peak = block_max<kWaves>(thread_absmax<DT, CPT>(v), red);
  const I8Scale s = i8_scale(quant_scale<MODE>(peak));
  if (tid == 0) scales[row] = s.scale;
  store_row<DT, MODE, CPT>(v, s, nchunks, tid, q + row * k);
}

// Rows wider than 16 chunks per thread: two passes, the second re-reading the row.
template <int DT, int MODE>
__global__ __launch_bounds__(kThreads) void quantize_rows_wide(const uint8_t* __restrict__ x, int64_t k,
                                                                 uint8_t* __restrict__ q,
                                                                 float* __restrict__ scales) {
  __shared__ float red[kWaves];
  constexpr int EPC = 16 / dtype_bytes<DT>();
  const int64_t row = blockIdx.x;
  const int64_t nchunks = k / EPC;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * k * dtype_bytes<DT>());
  uint8_t* qr = q + row * k;
  float peak = 0.0f;
  for (int64_t c = threadIdx.x; c < nchunks; c += kThreads) {
    const uint4 v[1] = {xr[c]};
    peak = fmaxf(peak, thread_absmax<DT, 1>(v));
  }
  peak = block_max<kWaves>(peak, red);
  const I8Scale s = i8_scale(quant_scale<MODE>(peak));
  if (threadIdx.x == 0) scales[row] = s.scale;
  for (int64_t c = threadIdx.x; c < nchunks; c += kThreads) encode_chunk<DT, MODE>(xr[c], s, qr + c * EPC);
}

// Scalar path for any K / alignment: IEEE division per element.
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

template <int DT, int MODE, int CPT>
void launch_vec(const uint8_t* x, int64_t rows, int64_t k, uint8_t* q, float* s, hipStream_t st) {
  quantize_rows_vec<DT, MODE, CPT><<<dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st>>>(x, k, q, s);
}

template <int DT, int MODE>
int launch_quantize(const void* x, int64_t rows, int64_t k, void* q, float* s, hipStream_t st) {
  const int64_t row_bytes = k * dtype_bytes<DT>();
  const bool vec = row_bytes % 16 == 0 && aligned16(x) && aligned16(q);
  auto* xb = static_cast<const uint8_t*>(x);
  auto* qb = static_cast<uint8_t*>(q);
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  const int64_t chunks = row_bytes / 16;
  if (!vec) quantize_rows_scalar<DT, MODE><<<grid, block, 0, st>>>(x, k, qb, s);
  else if (chunks <= kThreads * 1) launch_vec<DT, MODE, 1>(xb, rows, k, qb, s, st);
  else if (chunks <= kThreads * 2) launch_vec<DT, MODE, 2>(xb, rows, k, qb, s, st);
  else if (chunks <= kThreads * 4) launch_vec<DT, MODE, 4>(xb, rows, k, qb, s, st);
  else if (chunks <= kThreads * 8) launch_vec<DT, MODE, 8>(xb, rows, k, qb, s, st);
  else if (chunks <= kThreads * 16) launch_vec<DT, MODE, 16>(xb, rows, k, qb, s, st);
  else quantize_rows_wide<DT, MODE><<<grid, block, 0, st>>>(xb, k, qb, s);
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
