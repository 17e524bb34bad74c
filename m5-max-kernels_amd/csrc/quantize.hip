// Per-row symmetric INT8 / FP8-E4M3 activation quantizer for gfx950.
//
// Behaviour follows the reference contract quantize_reference
// (src/m5kernels/numerics.py:29-46) as realised by shaders/quantize.metal:1-38:
//   peak  = max |x|, NaN ignored           (FP32, order-independent => exact)
//   scale = peak == 0 ? 1 : peak / 127     (or / 448 for FP8), IEEE division
//   code  = clamp(rint_even(x / scale), -127, 127)   or  E4M3(x / scale)
// INT8 codes come from two fused multiply-adds that bracket the quotient, with a grouped
// exact fallback near rounding boundaries (encode_i8), bit-identical to the IEEE division.
//
// A row is read once from HBM with 16-byte loads and held in VGPRs between the max
// reduction and the encode, so HBM traffic is exactly 2*K (bf16 in) + K (codes out) + 4
// bytes per row.  Each row has its own workgroup of 256, 512 or 1024 threads, as many as
// give each thread about two 16-byte chunks (see launch_quantize).  At [4096, 16384] the
// kernel takes ~30 us where the same traffic with no arithmetic streams in 26 us: a row's
// time is its loads, one block reduction, then its encode, and a wider workgroup shortens
// the last two.  A persistent grid with a one-row register prefetch, and a variant at 8
// waves per SIMD, measured no faster with 256 threads per row.  Nor did four rows per
// workgroup, unrolled so that each row's loads stay in flight across the previous row's
// reduction (an LDS-only barrier, exact vmcnt waits): 40.6 us against 37.9 us for INT8, the
// halved occupancy (118 VGPRs) costing more than the overlap gains.  Giving each thread two
// adjacent chunks, so that its codes leave in one 16-byte store, measured 10% slower for INT8
// (4% faster for FP8).
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
  if constexpr (MODE == M5K_QUANT_INT8) encode_i8_div<EPC>(f, s, packed);
  else encode_fp8<EPC>(f, s, packed);
  if constexpr (EPC == 8) *reinterpret_cast<uint2*>(out) = make_uint2(packed[0], packed[1]);
  else *reinterpret_cast<uint32_t*>(out) = packed[0];
}

// Load a row's chunks tid, tid + KT, ... into registers; chunks past the row read as zero.
template <int CPT, int KT>
__device__ __forceinline__ void load_row(const uint4* __restrict__ xr, int64_t nchunks, int tid, uint4 (&v)[CPT]) {
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = tid + (int64_t)i * KT;
    v[i] = c < nchunks ? xr[c] : make_uint4(0, 0, 0, 0);
  }
}

template <int DT, int MODE, int CPT, int KT>
__device__ __forceinline__ void store_row(const uint4 (&v)[CPT], const I8Scale& s, int64_t nchunks, int tid,
                                          uint8_t* __restrict__ qr) {
  constexpr int EPC = 16 / dtype_bytes<DT>();
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = tid + (int64_t)i * KT;
    if (c < nchunks) encode_chunk<DT, MODE>(v[i], s, qr + c * EPC);
  }
}

// One workgroup of KT threads per row: row bytes % 16 == 0 and 16-byte aligned bases.  CPT =
// 16-byte chunks per thread kept in registers.
template <int DT, int MODE, int CPT, int KT>
__global__ __launch_bounds__(KT) void quantize_rows_vec(const uint8_t* __restrict__ x, int64_t k,
                                                          uint8_t* __restrict__ q,
                                                          float* __restrict__ scales) {
  __shared__ float red[KT / 64];
  constexpr int EPC = 16 / dtype_bytes<DT>();
  const int64_t row = blockIdx.x;
  const int64_t nchunks = k / EPC;
  const int tid = threadIdx.x;
  uint4 v[CPT];
  load_row<CPT, KT>(reinterpret_cast<const uint4*>(x + row * k * dtype_bytes<DT>()), nchunks, tid, v);
  const float peak = block_max<KT / 64>(thread_absmax<DT, CPT>(v), red);
  const I8Scale s = i8_scale(quant_scale<MODE>(peak));
  if (tid == 0) scales[row] = s.scale;
  store_row<DT, MODE, CPT, KT>(v, s, nchunks, tid, q + row * k);
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

// ---- MXINT8 (32-element blocks with a shared power-of-two scale) ----------------------------
// numerics.py:33-41 and quantize.metal's block mode: per block, e = 0 for an all-zero block,
// else clamp(floor(log2(peak)) - 6, -127, 127) with log2 rounded to FP32 before the floor (a
// peak just below 2^k gives k, as the reference's float32 log2 does); code =
// clamp(rint(x / 2^e), -127, 127); exponent byte e + 127.  Four lanes own a block, 8 elements
// each; the quad reduces its peak with DPP.  Division by 2^e is exact scaling, so
// ldexp(x, -e) rounds to the same value.
template <int DT>
__global__ __launch_bounds__(kThreads) void quantize_mx_kernel(const uint8_t* __restrict__ x, int64_t blocks,
                                                               int8_t* __restrict__ q, uint8_t* __restrict__ s) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if ((t >> 2) >= blocks) return;  // whole quads leave together
  constexpr int EB = dtype_bytes<DT>();
  const uint4* p = reinterpret_cast<const uint4*>(x + t * 8 * EB);
  float v[8];
  if constexpr (DT == M5K_F32) {
    const uint4 a = p[0], b = p[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
  } else {
    const uint4 a = p[0];
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = half_to_f32<DT>(w[i] & 0xFFFFu);
      v[2 * i + 1] = half_to_f32<DT>(w[i] >> 16);
    }
  }
  float peak = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) peak = fmaxf(peak, fabsf(v[i]));
  peak = fmaxf(peak, dpp_move<0xB1>(peak));  // quad_perm [1,0,3,2]
  peak = fmaxf(peak, dpp_move<0x4E>(peak));  // quad_perm [2,3,0,1]
  int e = 0;
  if (peak > 0.0f) {
    const float l = static_cast<float>(log2(static_cast<double>(peak)));
    e = min(max(static_cast<int>(floorf(l)) - 6, -127), 127);
  }
  uint32_t code[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) code[i] = i8_clamp_code(rintf(ldexpf(v[i], -e)));
  *reinterpret_cast<uint2*>(q + t * 8) =
      make_uint2(code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24),
                 code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24));
  if ((t & 3) == 0) s[t >> 2] = static_cast<uint8_t>(e + 127);
}

// MXINT8 codes to BF16 values code * 2^(e - 127): exact (|code| <= 127 fits the BF16
// significand), 8 elements per thread.
__global__ __launch_bounds__(kThreads) void mx_to_bf16_kernel(const int8_t* __restrict__ q,
                                                              const uint8_t* __restrict__ s, int64_t groups,
                                                              uint16_t* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= groups) return;
  const uint2 w = *reinterpret_cast<const uint2*>(q + t * 8);
  const int e = static_cast<int>(s[t >> 2]) - 127;
  uint32_t out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = i < 2 ? w.x : w.y;
    const int sh = 16 * (i & 1);
    const float lo = ldexpf(static_cast<float>(static_cast<int8_t>((word >> sh) & 0xFFu)), e);
    const float hi = ldexpf(static_cast<float>(static_cast<int8_t>((word >> (sh + 8)) & 0xFFu)), e);
    out[i] = f32x2_to_bf16x2(lo, hi);
  }
  *reinterpret_cast<uint4*>(y + t * 8) = make_uint4(out[0], out[1], out[2], out[3]);
}

template <int DT, int MODE, int KT, int CPT>
void launch_vec(const uint8_t* x, int64_t rows, int64_t k, uint8_t* q, float* s, hipStream_t st) {
  launch_kernel(quantize_rows_vec<DT, MODE, CPT, KT>, dim3(static_cast<unsigned>(rows)), dim3(KT), st, x, k, q, s);
}

template <int DT, int MODE>
int launch_quantize(const void* x, int64_t rows, int64_t k, void* q, float* s, hipStream_t st) {
  const int64_t row_bytes = k * dtype_bytes<DT>();
  const bool vec = row_bytes % 16 == 0 && aligned16(x) && aligned16(q);
  auto* xb = static_cast<const uint8_t*>(x);
  auto* qb = static_cast<uint8_t*>(q);
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  const int64_t chunks = row_bytes / 16;
  // Workgroup width: rows of more than 512 chunks take 512 or 1024 threads with two (or more)
  // chunks each.  A wider workgroup finishes its row sooner, and at FFN-down ([4096, 16384]
  // BF16, 2048 chunks) 1024 threads x 2 chunks measured 29.4 us against 30.2 us for 512 x 4
  // and 32.0-32.7 us for 256 x 8; at K 4096 (512 chunks) 256 x 2 measured 9.3 us against 15.7
  // us for 512 x 1.  FP8 rows of up to 2048 chunks take 512 x 4: inside the FP8 online step
  // (quantize + FP8 GEMM, FFN-down) it measured 232.3 us against 234.5 us for 1024 x 2.  The row
  // peak is order-independent, so codes and scales do not depend on the width.
  if (!vec) quantize_rows_scalar<DT, MODE><<<grid, block, 0, st>>>(x, k, qb, s);
  else if (chunks <= 256) launch_vec<DT, MODE, 256, 1>(xb, rows, k, qb, s, st);
  else if (chunks <= 512) launch_vec<DT, MODE, 256, 2>(xb, rows, k, qb, s, st);
  else if (chunks <= 1024) launch_vec<DT, MODE, 512, 2>(xb, rows, k, qb, s, st);
  else if (chunks <= 2048) {
    if constexpr (MODE == M5K_QUANT_FP8) launch_vec<DT, MODE, 512, 4>(xb, rows, k, qb, s, st);
    else launch_vec<DT, MODE, 1024, 2>(xb, rows, k, qb, s, st);
  }
  else if (chunks <= 4096) launch_vec<DT, MODE, 1024, 4>(xb, rows, k, qb, s, st);
  else if (chunks <= 8192) launch_vec<DT, MODE, 1024, 8>(xb, rows, k, qb, s, st);
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

extern "C" int m5k_quantize_mxint8(const void* x, int x_dtype, int64_t rows, int64_t k, int8_t* q,
                                   uint8_t* exponents, void* stream) {
  using namespace m5k;
  clear_error();
  const char* name = "m5k_quantize_mxint8";
  M5K_REQUIRE(x && q && exponents, "%s: null pointer", name);
  M5K_REQUIRE(rows > 0 && k > 0 && k % 32 == 0, "%s: shape [%lld,%lld] needs K a positive multiple of 32", name,
              (long long)rows, (long long)k);
  M5K_REQUIRE(aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0, "%s: misaligned buffers", name);
  const int64_t blocks = rows * (k / 32);
  const int64_t groups = (blocks * 4 + kThreads - 1) / kThreads;
  M5K_REQUIRE(groups <= 0x7FFFFFFF, "%s: input too large", name);
  const dim3 grid(static_cast<unsigned>(groups)), block(kThreads);
  hipStream_t st = as_stream(stream);
  auto* xb = static_cast<const uint8_t*>(x);
  switch (x_dtype) {
    case M5K_BF16: quantize_mx_kernel<M5K_BF16><<<grid, block, 0, st>>>(xb, blocks, q, exponents); break;
    case M5K_F16: quantize_mx_kernel<M5K_F16><<<grid, block, 0, st>>>(xb, blocks, q, exponents); break;
    case M5K_F32: quantize_mx_kernel<M5K_F32><<<grid, block, 0, st>>>(xb, blocks, q, exponents); break;
    default: set_error("%s: unsupported input dtype %d", name, x_dtype); return M5K_EINVAL;
  }
  return launch_status(name);
}

extern "C" int m5k_mxint8_to_bf16(const int8_t* q, const uint8_t* exponents, int64_t rows, int64_t k, void* y,
                                  void* stream) {
  using namespace m5k;
  clear_error();
  const char* name = "m5k_mxint8_to_bf16";
  M5K_REQUIRE(q && exponents && y, "%s: null pointer", name);
  M5K_REQUIRE(rows > 0 && k > 0 && k % 32 == 0, "%s: shape [%lld,%lld] needs K a positive multiple of 32", name,
              (long long)rows, (long long)k);
  M5K_REQUIRE((reinterpret_cast<uintptr_t>(q) & 7u) == 0 && aligned16(y), "%s: misaligned buffers", name);
  const int64_t groups = rows * k / 8;
  const int64_t blocks = (groups + kThreads - 1) / kThreads;
  M5K_REQUIRE(blocks <= 0x7FFFFFFF, "%s: input too large", name);
  mx_to_bf16_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, as_stream(stream)>>>(
      q, exponents, groups, static_cast<uint16_t*>(y));
  return launch_status(name);
}
