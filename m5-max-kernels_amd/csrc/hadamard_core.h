// Signed block-Hadamard butterflies on wave64 register tiles.
//
// Transform (hadamard.py:33-45, shaders/hadamard.metal:6-26): for each block of B
// consecutive elements of a row, v = x * sign, then log2(B) natural-order Sylvester
// stages; at stride s the pair (i, i+s) (bit s of i clear) becomes (a+b, a-b), then
// every value is multiplied once by the FP32 constant 1/sqrt(B).
//
// Register layout: a lane holds EPC = max(8, B/64) consecutive elements of a block, so
// one block spans LPB = B/EPC <= 64 consecutive lanes.  Strides below EPC stay inside
// a lane's registers; strides EPC..B/2 are lane-xor exchanges within the LPB-lane group
// (the upper lane of a pair computes lower - upper, as an FMA with -1).  Partners within 32
// lanes come through ds_swizzle in its bit-mask mode, the partner 32 lanes away through
// v_permlane32_swap (one pass leaves the lower half's value in one register and the upper
// half's in the other on every lane).  With ds_bpermute, which reads an address per lane, the
// B = 256 RMS-quantize row kernel took 1.5x as long.  Each stage output
// is one correctly rounded FP32 sum or difference of its two inputs, so the result is
// independent of which lane does the work and bit-identical to a sequential FP32
// evaluation of the same stages.
#pragma once

#include "m5k_common.h"

namespace m5k {
namespace hadamard {

template <int B>
struct Shape {
  static_assert(B >= 32 && B <= 1024 && (B & (B - 1)) == 0, "block must be a power of two in [32,1024]");
  static constexpr int EPC = B / 64 > 8 ? B / 64 : 8;  // elements per lane
  static constexpr int LPB = B / EPC;                  // lanes per block
};

// FP32 nearest value of 1/sqrt(B) (the double 1/sqrt(B) rounded to float).
template <int B>
__device__ __forceinline__ constexpr float inv_sqrt_block() {
  return B == 32    ? 0x1.6a09e6p-3f
         : B == 64  ? 0x1.0p-3f
         : B == 128 ? 0x1.6a09e6p-4f
         : B == 256 ? 0x1.0p-4f
         : B == 512 ? 0x1.6a09e6p-5f
                    : 0x1.0p-5f;
}

// Lane-xor stages M, 2M, ..., LPB/2 of the transform.  fma(+-1, v, peer) is the single
// rounding of v + peer (lower lane) or peer - v (upper lane): the same bits as the add or
// subtract, in one VALU op instead of add, sub, select.
template <int M, int LPB, int EPC>
__device__ __forceinline__ void cross_stages(float (&v)[EPC], int lane) {
  if constexpr (M < LPB) {
    const float sgn = (lane & M) ? -1.0f : 1.0f;
#pragma unroll
    for (int r = 0; r < EPC; ++r) {
      if constexpr (M < 32) {
        // Bit-mask swizzle within 32 lanes: and 0x1F, or 0, xor M.
        const float peer = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v[r]), 0x1F | (M << 10)));
        v[r] = __builtin_fmaf(sgn, v[r], peer);
      } else {
        // Both operands v: afterwards the first holds lanes 0-31's value and the second lanes
        // 32-63's, on every lane; lower + upper or lower - upper is fma(sgn, upper, lower).
        const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[r]), __float_as_uint(v[r]), false, false);
        v[r] = __builtin_fmaf(sgn, __uint_as_float(halves[1]), __uint_as_float(halves[0]));
      }
    }
    cross_stages<2 * M, LPB>(v, lane);
  }
}

// In-place transform of v[EPC] for the calling lane (all lanes of a block must call).
// SCALED = false leaves out the final multiply by 1/sqrt(B); FoldedI8 applies it inside the
// quantizer's encode instead.
template <int B, bool SCALED = true>
__device__ __forceinline__ void butterflies(float (&v)[Shape<B>::EPC]) {
  constexpr int EPC = Shape<B>::EPC, LPB = Shape<B>::LPB;
#pragma unroll
  for (int s = 1; s < EPC; s <<= 1) {
#pragma unroll
    for (int base = 0; base < EPC; base += 2 * s) {
#pragma unroll
      for (int j = 0; j < s; ++j) {
        const float a = v[base + j], c = v[base + j + s];
        v[base + j] = a + c;
        v[base + j + s] = a - c;
      }
    }
  }
  cross_stages<1, LPB>(v, static_cast<int>(threadIdx.x & 63));
  if constexpr (SCALED) {
    constexpr float inv = inv_sqrt_block<B>();
#pragma unroll
    for (int r = 0; r < EPC; ++r) v[r] = v[r] * inv;
  }
}

// Grouped lane tiles for the streaming rotation: a lane holds G = max(1, B/256) groups of 4
// consecutive elements, group t at block offset 256t + 4 * (lane mod B/4), so every group of a
// wave is 1 KiB of contiguous FP32 output.  Strides 1 and 2 stay inside a group, strides
// 4 .. min(B, 256)/2 are lane exchanges, strides 256 .. B/2 pair group t with group t + s in
// the same lane: the stride order is the natural one, as in butterflies().
template <int B>
struct Grouped {
  static constexpr int G = B > 256 ? B / 256 : 1;
  static constexpr int LPB = B > 256 ? 64 : B / 4;
};

template <int B>
__device__ __forceinline__ void butterflies_grouped(float (&v)[4 * Grouped<B>::G]) {
  constexpr int G = Grouped<B>::G;
#pragma unroll
  for (int t = 0; t < G; ++t) {
    float* w = v + 4 * t;
    const float a0 = w[0] + w[1], a1 = w[0] - w[1], a2 = w[2] + w[3], a3 = w[2] - w[3];
    w[0] = a0 + a2;
    w[1] = a1 + a3;
    w[2] = a0 - a2;
    w[3] = a1 - a3;
  }
  cross_stages<1, Grouped<B>::LPB>(v, static_cast<int>(threadIdx.x & 63));
#pragma unroll
  for (int s = 1; s < G; s <<= 1) {
#pragma unroll
    for (int t = 0; t < G; ++t) {
      if ((t & s) == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = v[4 * t + r], c = v[4 * (t + s) + r];
          v[4 * t + r] = a + c;
          v[4 * (t + s) + r] = a - c;
        }
      }
    }
  }
  constexpr float inv = inv_sqrt_block<B>();
#pragma unroll
  for (int r = 0; r < 4 * G; ++r) v[r] = v[r] * inv;
}

// Per-row INT8 encoder for butterflies<B, false> output z': the reference's rotated value is
// z = fl(z' * c), c = 1/sqrt(B) in FP32, and its code clamp(rint(fl(z / scale))).  Rounding
// is monotone, so the row peak max |z| = fl(max |z'| * c); the bracket multipliers come from
// m~ = fl(c * fl(1 / scale)) (two roundings of c / scale) against the two-rounding chain.
template <int B>
struct FoldedI8 {
  float scale;
  I8Bracket bracket;
  FoldedI8() = default;
  __device__ __forceinline__ FoldedI8(float scale_, const I8Bracket& bracket_) : scale(scale_), bracket(bracket_) {}
  __device__ __forceinline__ explicit FoldedI8(float peak_unscaled) {
    constexpr float c = inv_sqrt_block<B>();
    const I8Scale s = i8_scale(quant_scale<M5K_QUANT_INT8>(peak_unscaled * c));
    scale = s.scale;
    bracket = i8_bracket(c * s.inv, s.exact);
  }
  template <int N>
  __device__ __forceinline__ void encode(const float (&zu)[N], uint32_t (&out)[N / 4]) const {
    const float sc = scale;
    encode_i8<N>(zu, bracket, [sc](float z) { return i8_code_of((z * inv_sqrt_block<B>()) / sc); }, out);
  }
};

// Raw 16-byte words of 8 elements of dtype DT (one word for 2-byte types, two for FP32).
template <int DT>
struct Raw8 {
  uint4 w[dtype_bytes<DT>() / 2];
};

template <int DT>
__device__ __forceinline__ Raw8<DT> fetch8(const void* base, int64_t e) {
  const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(base) + e * dtype_bytes<DT>());
  Raw8<DT> r;
#pragma unroll
  for (int i = 0; i < dtype_bytes<DT>() / 2; ++i) r.w[i] = p[i];
  return r;
}

template <int DT>
__device__ __forceinline__ void decode8(const Raw8<DT>& r, float (&v)[8]) {
  if constexpr (DT == M5K_F32) {
    const uint32_t w[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w, r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
  } else {
    const uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
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

// 8 elements at column `col` of a row whose base address is uniform (a 32-bit lane offset).
template <int DT>
__device__ __forceinline__ Raw8<DT> fetch8_at(const uint8_t* row_base, uint32_t col) {
  const uint4* q = reinterpret_cast<const uint4*>(row_base + col * static_cast<uint32_t>(dtype_bytes<DT>()));
  Raw8<DT> r;
#pragma unroll
  for (int i = 0; i < dtype_bytes<DT>() / 2; ++i) r.w[i] = q[i];
  return r;
}

// Sign-bit masks of 8 columns for their 16-byte words of dtype DT (BF16/FP16 words hold elements
// 2i and 2i + 1 in bits 0-15 and 16-31; FP32 words one element each): XOR flips the sign of each
// column whose int8 sign is negative, the exact product with +-1.  v_perm_b32 moves sign bytes 2i and 2i + 1 to bytes 1 and 3 (selector
// 0x0C yields zero), the AND keeps their top bits.
template <int PDT>
struct SignMask8 {
  uint32_t m[PDT == M5K_F32 ? 8 : 4];
  __device__ __forceinline__ explicit SignMask8(const uint2& s) {
    if constexpr (PDT == M5K_F32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) m[i] = ((i < 4 ? s.x : s.y) << (24 - 8 * (i & 3))) & 0x80000000u;
    } else {
      m[0] = __builtin_amdgcn_perm(0u, s.x, 0x010C000Cu) & 0x80008000u;
      m[1] = __builtin_amdgcn_perm(0u, s.x, 0x030C020Cu) & 0x80008000u;
      m[2] = __builtin_amdgcn_perm(0u, s.y, 0x010C000Cu) & 0x80008000u;
      m[3] = __builtin_amdgcn_perm(0u, s.y, 0x030C020Cu) & 0x80008000u;
    }
  }
  __device__ __forceinline__ Raw8<PDT> apply(Raw8<PDT> r) const {
    if constexpr (PDT == M5K_F32) {
      r.w[0].x ^= m[0]; r.w[0].y ^= m[1]; r.w[0].z ^= m[2]; r.w[0].w ^= m[3];
      r.w[1].x ^= m[4]; r.w[1].y ^= m[5]; r.w[1].z ^= m[6]; r.w[1].w ^= m[7];
    } else {
      r.w[0].x ^= m[0]; r.w[0].y ^= m[1]; r.w[0].z ^= m[2]; r.w[0].w ^= m[3];
    }
    return r;
  }
};

// Parameter tables of the prep kernels (gamma, scale, shift, gate), 8 columns at a time.
// Tables<M5K_BF16> reads every table as BF16 (compile-time layout).  Tables<M5K_PMIX> reads each
// table in its own dtype, given at run time (BF16, FP16 or FP32; wave-uniform, so the choice is a
// scalar branch), into FP32-sized storage.  Every decode to FP32 is exact, so the FP32 arithmetic
// that follows sees the same values whatever dtype a table has.
constexpr int M5K_PMIX = 8;  // template code for per-table run-time dtypes (not an element dtype)

template <int PDT>
struct Tables;

template <>
struct Tables<M5K_BF16> {
  using raw = Raw8<M5K_BF16>;
  __device__ static raw fetch(const void* base, int64_t e, int) { return fetch8<M5K_BF16>(base, e); }
  __device__ static void decode(const raw& r, int, float (&v)[8]) { decode8<M5K_BF16>(r, v); }
  __device__ static raw sign(const raw& r, const uint2& s, int) { return SignMask8<M5K_BF16>(s).apply(r); }
  __device__ static void load(const void* base, int64_t e, int, float (&v)[8]) { decode8<M5K_BF16>(fetch8<M5K_BF16>(base, e), v); }
};

template <>
struct Tables<M5K_PMIX> {
  using raw = Raw8<M5K_F32>;  // FP32: both words; BF16 / FP16: the first word
  __device__ static raw fetch(const void* base, int64_t e, int dt) {
    if (dt == M5K_F32) return fetch8<M5K_F32>(base, e);
    raw r;
    r.w[0] = fetch8<M5K_BF16>(base, e).w[0];  // 8 two-byte elements
    r.w[1] = make_uint4(0u, 0u, 0u, 0u);
    return r;
  }
  __device__ static void decode(const raw& r, int dt, float (&v)[8]) {
    if (dt == M5K_F32) {
      decode8<M5K_F32>(r, v);
    } else if (dt == M5K_BF16) {
      Raw8<M5K_BF16> h;
      h.w[0] = r.w[0];
      decode8<M5K_BF16>(h, v);
    } else {
      Raw8<M5K_F16> h;
      h.w[0] = r.w[0];
      decode8<M5K_F16>(h, v);
    }
  }
  // BF16 and FP16 keep their sign bits in the same positions (bits 15 and 31 of each word).
  __device__ static raw sign(const raw& r, const uint2& s, int dt) {
    if (dt == M5K_F32) return SignMask8<M5K_F32>(s).apply(r);
    Raw8<M5K_BF16> h;
    h.w[0] = r.w[0];
    raw out = r;
    out.w[0] = SignMask8<M5K_BF16>(s).apply(h).w[0];
    return out;
  }
  __device__ static void load(const void* base, int64_t e, int dt, float (&v)[8]) { decode(fetch(base, e, dt), dt, v); }
};

}  // namespace hadamard
}  // namespace m5k
