// Shared device helpers and host-side error plumbing for libm5k.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "m5k.h"

namespace m5k {

// ---- host-side status --------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
// Translate a launch's hipGetLastError() into the ABI status.
int launch_status(const char* what);
// Compute units of the current device (cached per device; 0 if the query fails).
int device_cus();

#define M5K_REQUIRE(cond, ...)          \
  do {                                  \
    if (!(cond)) {                      \
      ::m5k::set_error(__VA_ARGS__);    \
      return M5K_EINVAL;                \
    }                                   \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- element conversions (device) --------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// FP32 -> BF16 round to nearest even, the producer-side cast of the reference
// (qk_rope_reference.py:37-42: (u + 0x7FFF + ((u >> 16) & 1)) >> 16 on finite inputs).
// gfx950's v_cvt_pk_bf16_f32 computes exactly that for every finite FP32 bit pattern,
// denormals included (checked exhaustively on MI355X), one instruction per pair.
typedef __bf16 m5k_bf16x2 __attribute__((ext_vector_type(2)));
typedef float m5k_f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two values to packed BF16 (lo in bits 0-15).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  const m5k_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, m5k_bf16x2));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16)));
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Round an FP32 value through a storage dtype and back (the "O(...)" boundary).
template <int DT>
__device__ __forceinline__ float round_through(float v) {
  if constexpr (DT == M5K_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  else if constexpr (DT == M5K_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  else return v;
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t i) {
  if constexpr (DT == M5K_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[i]);
  else if constexpr (DT == M5K_F16) return f16_bits_to_f32(static_cast<const uint16_t*>(base)[i]);
  else return static_cast<const float*>(base)[i];
}

template <int DT>
__device__ __forceinline__ void store_elem(void* base, int64_t i, float v) {
  if constexpr (DT == M5K_BF16) static_cast<uint16_t*>(base)[i] = (uint16_t)f32_to_bf16_bits(v);
  else if constexpr (DT == M5K_F16) static_cast<uint16_t*>(base)[i] = (uint16_t)f32_to_f16_bits(v);
  else static_cast<float*>(base)[i] = v;
}

template <int DT>
constexpr int dtype_bytes() {
  return DT == M5K_F32 ? 4 : 2;
}

// Load 8 consecutive elements of dtype DT at element index e (16-byte aligned for 2-byte
// types, 32-byte for FP32).
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t e, float (&v)[8]) {
  const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(base) + e * dtype_bytes<DT>());
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
      if constexpr (DT == M5K_BF16) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      } else {
        v[2 * i] = f16_bits_to_f32(w[i] & 0xFFFFu);
        v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
      }
    }
  }
}

// OCP FP8 E4M3 ("fn") encoder: nearest finite code, ties to even code,
// saturating to 448 (code 126), sign taken from the sign bit.  Restates
// numerics.fp8_encode (src/m5kernels/numerics.py:17-26) with exponent-field
// extraction instead of a codebook search.  Finite input only.
__device__ __forceinline__ uint32_t fp8_e4m3_encode(float v) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = __uint_as_float(u & 0x7FFFFFFFu);
  uint32_t bits;
  if (!(a < 448.0f)) {
    bits = 126u;
  } else if (a < 0.015625f) {  // below 2^-6: subnormal grid m * 2^-9, exact scaling
    bits = static_cast<uint32_t>(rintf(a * 512.0f));
  } else {
    int e = static_cast<int>((u >> 23) & 0xFFu) - 127;  // floor(log2 a), a normal
    float scaled = __uint_as_float(static_cast<uint32_t>(127 + 3 - e) << 23);  // 2^(3-e)
    int qm = static_cast<int>(rintf(a * scaled));                              // in [8,16]
    if (qm == 16) { qm = 8; ++e; }
    bits = static_cast<uint32_t>(((e + 7) << 3) + (qm - 8));
    bits = bits > 126u ? 126u : bits;
  }
  return sign | bits;
}

// Per-row quantization of one value given the row scale (IEEE FP32 division, then
// round-half-even and clamp for INT8; E4M3 encode for FP8).
template <int MODE>
__device__ __forceinline__ uint32_t quant_encode(float x, float scale) {
  const float z = x / scale;
  if constexpr (MODE == M5K_QUANT_FP8) {
    return fp8_e4m3_encode(z);
  } else {
    const float r = fminf(fmaxf(rintf(z), -127.0f), 127.0f);
    return static_cast<uint32_t>(static_cast<int>(r)) & 0xFFu;
  }
}

// Row-constant INT8 encoder state: the scale, its correctly rounded reciprocal, and `exact`
// when the reciprocal is unsafe (scale below 2^-100, where 1/scale may overflow): then every
// element takes the IEEE division.
struct I8Scale {
  float scale;
  float inv;
  bool exact;
};

__device__ __forceinline__ I8Scale i8_scale(float scale) {
  return I8Scale{scale, 1.0f / scale, scale < 0x1p-100f};
}

__device__ __forceinline__ uint32_t i8_clamp_code(float r) {
  const float c = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<uint32_t>(static_cast<int>(c)) & 0xFFu;
}

// INT8 codes of N values (N % 4 == 0) packed 4 per word, bit-identical to
// clamp(rint_even(fl(x / scale)), -127, 127) for every x of a row whose |x| <= peak.
// Fast path: q0 = fl(x * inv).  With scale = fl(peak / 127), |x / scale| <= 127.01, and
// |q0 - x/scale| <= 127.01 * (2^-23 + 2^-48) < 2^-16, so rint(q0) == rint(x/scale) unless a
// rounding boundary n + 1/2 lies within 2^-16 of q0.  Clamping to [-127, 127] before the
// rounding gives the same code.  Adding 1.5 * 2^23 rounds the clamped value to an integer
// (round-half-even) and leaves its two's-complement low byte in the low byte of the sum's
// bits.  If any element of the group lies within 2^-15 of a rounding boundary
// (|qc - rint(qc)| >= 1/2 - 2^-15, exact ties included) the whole group takes the IEEE
// division instead; one branch per group keeps the common path at about six VALU ops.
template <int N>
__device__ __forceinline__ void encode_i8(const float (&x)[N], const I8Scale& s, uint32_t (&out)[N / 4]) {
  constexpr float kRound = 0x1.8p23f;
  uint32_t t[N];
  float dev = s.exact ? 1.0f : 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float qc = fminf(fmaxf(x[i] * s.inv, -127.0f), 127.0f);
    const float biased = qc + kRound;
    dev = fmaxf(dev, fabsf(qc - (biased - kRound)));
    t[i] = __float_as_uint(biased);
  }
  if (dev >= 0.5f - 0x1p-15f) {
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = __float_as_uint(fminf(fmaxf(rintf(x[i] / s.scale), -127.0f), 127.0f) + kRound);
  }
#pragma unroll
  for (int w = 0; w < N / 4; ++w) {
    // v_perm_b32 picks byte 0 of each operand: selector bytes 0 and 4 address src1.b0 and src0.b0,
    // 0x0C yields zero.
    const uint32_t lo = __builtin_amdgcn_perm(t[4 * w + 1], t[4 * w], 0x0C0C0400u);
    const uint32_t hi = __builtin_amdgcn_perm(t[4 * w + 3], t[4 * w + 2], 0x04000C0Cu);
    out[w] = lo | hi;
  }
}

// FP8 E4M3 codes of N values (N % 4 == 0) packed 4 per word, bit-identical to
// fp8_e4m3_encode(fl(x / scale)) for every x of a row whose |x| <= peak, scale = fl(peak / 448).
// Fast path: y = fl(x * inv) clamped to [-448, 448] and converted by v_cvt_pk_fp8_f32, which
// equals fp8_e4m3_encode on every finite f32 of magnitude below 464 (all 2.28e9 of them
// compared on MI355X) and rounds monotonically in the magnitude.  y and fl(x / scale) differ by
// at most 3 ulp(y) (the reciprocal and the product each round once), i.e. at most 6 ulps of
// the binade below; so when the magnitudes 8 ulps below and above |y| convert to the same code,
// fl(x / scale) converts to that code too.  Otherwise the group takes the IEEE division and the
// software encoder.
template <int N>
__device__ __forceinline__ void encode_fp8(const float (&x)[N], const I8Scale& s, uint32_t (&out)[N / 4]) {
  bool ok = !s.exact;
#pragma unroll
  for (int w = 0; w < N / 4; ++w) {
    float y[4], below[4], above[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      y[b] = fminf(fmaxf(x[4 * w + b] * s.inv, -448.0f), 448.0f);
      const uint32_t a = __float_as_uint(y[b]) & 0x7FFFFFFFu;
      below[b] = __uint_as_float(a > 8u ? a - 8u : 0u);
      above[b] = __uint_as_float(a + 8u);
    }
    // word_sel false writes bits [15:0] (first operand in the low byte), true bits [31:16].
    int word = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    word = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], word, true);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(below[0], below[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(below[2], below[3], lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(above[0], above[1], 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(above[2], above[3], hi, true);
    ok = ok && lo == hi;
    out[w] = static_cast<uint32_t>(word);
  }
  if (!ok) {
#pragma unroll
    for (int w = 0; w < N / 4; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) word |= fp8_e4m3_encode(x[4 * w + b] / s.scale) << (8 * b);
      out[w] = word;
    }
  }
}

template <int MODE>
__device__ __forceinline__ float quant_scale(float peak) {
  return peak == 0.0f ? 1.0f : peak / (MODE == M5K_QUANT_FP8 ? 448.0f : 127.0f);
}

// ---- wave64 reductions -------------------------------------------------------------------
// DPP lane movement of v (0 where the row mask leaves a lane unwritten).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes, the result in every lane.  Fixed tree: lane pairs (xor 1), pairs
// of pairs (xor 2), quads across each half-row (row_half_mirror), halves across each row
// (row_mirror); then row 1 += row 0 and row 3 += row 2 (row_bcast15), row 3 += rows 0-1
// (row_bcast31); lane 63 holds (r2 + r3) + (r0 + r1).  One DPP add per step.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  v += dpp_move<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
  v += dpp_move<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum over the 64 lanes of non-negative values (absolute peaks), same movement pattern;
// lanes a row mask leaves unwritten contribute 0.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  v = fmaxf(v, dpp_move<0x142, 0xA>(v));
  v = fmaxf(v, dpp_move<0x143, 0xC>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Block-wide reductions over NWAVES waves through the NWAVES-float LDS slot `lds`; every
// thread gets the result.  One barrier: each reduction in a workgroup needs its own slot.
template <int NWAVES>
__device__ __forceinline__ float block_max(float v, float* lds) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int w = 1; w < NWAVES; ++w) r = fmaxf(r, lds[w]);
  return r;
}

template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float* lds) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int w = 1; w < NWAVES; ++w) r += lds[w];
  return r;
}

}  // namespace m5k
