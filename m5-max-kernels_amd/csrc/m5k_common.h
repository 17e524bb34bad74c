// Shared device helpers and host-side error plumbing for libm5k.so (gfx950 only).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
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

template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t st, Args&&... args) {
  kernel<<<grid, block, 0, st>>>(static_cast<KArgs>(args)...);
}

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

// Streaming stores (non-temporal: global_store ... nt) for large outputs that the kernel writes
// once and does not read back.  A normal store allocates its lines in the caches; right after a
// kernel that streamed a few hundred MB (the activation quantizer before the GEMM), writing the
// GEMM's 32 MB BF16 output that way took 26 us instead of 3 us (FFN-down, MI355X), while the
// non-temporal form took the same time in either order.  Bits are unaffected.
typedef unsigned int m5k_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int m5k_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_stream16(void* p, uint4 w) {
  __builtin_nontemporal_store(m5k_u32x4{w.x, w.y, w.z, w.w}, static_cast<m5k_u32x4*>(p));
}
__device__ __forceinline__ void store_stream8(void* p, uint2 w) {
  __builtin_nontemporal_store(m5k_u32x2{w.x, w.y}, static_cast<m5k_u32x2*>(p));
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

// INT8 code of one value as the low byte of a word, from the row's exact chain:
// clamp(rint_even(v), -127, 127) for the chain's FP32 result v.
__device__ __forceinline__ uint32_t i8_code_of(float v) {
  return i8_clamp_code(rintf(v));
}

// Row-constant INT8 encoder for codes clamp(rint_even(v(x)), -127, 127), where v(x) is the
// row's chain of correctly rounded FP32 operations on x whose exact value is x * m for a row
// constant m >= 0 (fl(x / scale): m = 1/scale; fl(fl(x * c) / scale): m = c/scale; ...).
//
// Fast path: t = fma(x, mult, 1.5 * 2^23) rounds x * mult to an integer once (the sum lies in
// [2^23, 2^24), where the FP32 spacing is 1, and 1.5 * 2^23 is even, so ties go to the even
// integer) and leaves its two's-complement low byte in the low byte of t's bits.  lo and hi
// are 8 representable steps below and above m~, an FP32 estimate of m with at most two
// roundings (|m~/m - 1| <= 2^-23 + 2^-48); 8 steps move m~ by more than 2^-21 (1 - 2^-20) of
// itself, so lo <= m (1 - 2^-22) and hi >= m (1 + 2^-22).  A chain of at most three roundings
// keeps v(x) / (x * m) within [1 - 3 * 2^-24, 1 + 3 * 2^-24 + 2^-46] of 1.  Then
// x * lo <= v(x) <= x * hi (x >= 0; reversed for x < 0), and rounding to an integer is
// monotone, so equal results of the two fused multiply-adds are rint(v(x)).  They are within
// [-127, 127] whenever |x| <= the row peak the scale was derived from (|v| <= 127.0001), so
// the clamp is inactive; m~ = 0 (an infinite scale, a zero peak) gives code 0 for every finite
// x, as the chain does.  Otherwise (a half-integer between the two products, a NaN, or `exact`
// set for a scale whose reciprocal is out of range) the call's N values take the chain itself,
// on every lane of the wave.
struct I8Bracket {
  float lo, hi;
  bool exact;  // every element takes the chain
};

// m_est is m~ (>= 0), exact forces the chain for the whole row.
__device__ __forceinline__ I8Bracket i8_bracket(float m_est, bool exact) {
  if (m_est == 0.0f) return I8Bracket{0.0f, 0.0f, exact};
  const bool in_range = m_est >= 0x1p-100f && m_est <= 0x1p100f;
  const uint32_t b = __float_as_uint(m_est);
  return I8Bracket{__uint_as_float(b - 8u), __uint_as_float(b + 8u), exact || !in_range};
}

// N values (N % 4 == 0) to N INT8 codes packed 4 per word.  chain(x) returns the code of x
// through the row's exact chain (a low byte), for groups the fast path cannot settle.
template <int N, class Chain>
__device__ __forceinline__ void encode_i8(const float (&x)[N], const I8Bracket& e, Chain chain,
                                          uint32_t (&out)[N / 4]) {
  constexpr float kRound = 0x1.8p23f;
  uint32_t t[N];
  // Lanes whose products disagree (or are NaN), gathered as wave masks: one v_cmp per value and
  // a scalar OR, instead of a per-lane boolean.  When any lane of the wave needs the chain, the
  // whole wave takes it: on the other lanes it yields the fast path's codes again.
  uint64_t unsettled = e.exact ? ~0ull : 0ull;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float lo = __builtin_fmaf(x[i], e.lo, kRound), hi = __builtin_fmaf(x[i], e.hi, kRound);
    unsettled |= __builtin_amdgcn_ballot_w64(!(lo == hi));
    t[i] = __float_as_uint(hi);
  }
  if (unsettled) {
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = chain(x[i]);
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

// The plain per-row quantizer's encoder: v(x) = fl(x / scale), m~ = fl(1 / scale).
__device__ __forceinline__ I8Bracket i8_div_bracket(const I8Scale& s) { return i8_bracket(s.inv, s.exact); }

template <int N>
__device__ __forceinline__ void encode_i8_div(const float (&x)[N], const I8Scale& s, uint32_t (&out)[N / 4]) {
  const float scale = s.scale;
  encode_i8<N>(x, i8_div_bracket(s), [scale](float v) { return i8_code_of(v / scale); }, out);
}

// FP8 E4M3 codes of N values (N % 4 == 0) packed 4 per word, bit-identical to
// fp8_e4m3_encode(fl(x / scale)) for every finite x of a row whose |x| <= peak,
// scale = fl(peak / 448).  The products fl(x * lo) and fl(x * hi), with lo and hi the
// multipliers of i8_bracket(fl(1 / scale)), bracket fl(x / scale): the multipliers sit more than
// 2^-22 of 1/scale away from it, each product and the quotient round once (2^-24).
// v_cvt_pk_fp8_f32 equals fp8_e4m3_encode on every finite f32 of magnitude below 464 (all
// 2.28e9 of them compared on MI355X; |x * hi| <= 448.001 here) and is monotone in the value, so
// when both products give the same code, fl(x / scale) gives it too.  Otherwise (or for an
// out-of-range reciprocal) the value takes the IEEE division and the same conversion of the
// quotient; quotients at or above 448 in magnitude saturate first as fp8_e4m3_encode does.
// Exact ties of fl(x / scale) are common for 16-bit inputs (an E4M3 midpoint has 4
// significant bits), so the exact chain is taken per byte position of a word, on every lane
// of the wave at once, only for positions unsettled on some lane.
template <int N>
__device__ __forceinline__ void encode_fp8(const float (&x)[N], const I8Scale& s, uint32_t (&out)[N / 4]) {
  const I8Bracket e = i8_bracket(s.inv, s.exact);
#pragma unroll
  for (int w = 0; w < N / 4; ++w) {
    // word_sel false writes bits [15:0] (first operand in the low byte), true bits [31:16].
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w] * e.lo, x[4 * w + 1] * e.lo, 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w + 2] * e.lo, x[4 * w + 3] * e.lo, lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w] * e.hi, x[4 * w + 1] * e.hi, 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w + 2] * e.hi, x[4 * w + 3] * e.hi, hi, true);
    uint32_t word = static_cast<uint32_t>(hi);
    if (e.exact || __builtin_amdgcn_ballot_w64(lo != hi)) {
      // Some lane of the wave has an unsettled value in this word: each byte position that is
      // unsettled on any lane takes the exact chain on every lane (on a settled lane it gives
      // the fast code again).  The exact chain is the IEEE quotient through the same
      // conversion; a quotient of magnitude 448 or more, infinite or NaN enters as 448 with its
      // sign bit, which converts to the software encoder's saturated code (126 and the sign).
      const uint32_t diff = static_cast<uint32_t>(lo ^ hi);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (e.exact || __builtin_amdgcn_ballot_w64(((diff >> (8 * b)) & 0xFFu) != 0)) {
          const float z = x[4 * w + b] / s.scale;
          const float q = fabsf(z) < 448.0f ? z : copysignf(448.0f, z);
          const uint32_t code = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q, q, 0, false)) & 0xFFu;
          word = (word & ~(0xFFu << (8 * b))) | (code << (8 * b));
        }
      }
    }
    out[w] = word;
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
