// Block-Hadamard rotation (FP32 output) and fused rotation + per-row INT8 quantizer.
//
// rotate:  Y = (X * signs) blockdiag(H_B) in FP32 (hadamard.py:33-77).  Streaming
//          kernel: every lane owns groups of 4 consecutive elements, 2 (bf16) or 4 (fp32)
//          bytes in and 4 bytes out per element, no LDS.
// fused:   codes/scales of quantize(rotate(X), "int8") (hadamard_gemm.py:27-69 online
//          path) with one workgroup per row; the rotated row stays in VGPRs between
//          the row-peak reduction and the encode, so HBM sees 2K + K + 4 bytes per row.
//          Codes equal the two-kernel composition bit for bit (same FP32 values).
#include <type_traits>

#include "hadamard_core.h"

namespace m5k {
namespace hadamard {
namespace {

constexpr int kThreads = 256;

// Streaming rotation in grouped lane tiles (see Grouped<B>): each thread owns CPT lane tiles,
// tile g = (blockIdx.x * CPT + i) * kThreads + threadIdx.x, wave unit g / 64.  Every load and
// every 16-byte FP32 store of a wave is contiguous over its lanes; with 8 consecutive elements
// per lane the two stores of a lane's 32 bytes are half-dense (a plain BF16 -> FP32 conversion
// with that store pattern runs 71.1 us at [4096, 16384], 66.8 us with contiguous lane stores).
// All loads are issued before the first butterfly; the signs (+-1) enter as sign-bit flips of
// the packed words.  Lanes past the end rotate zeros (every lane takes part in the exchanges)
// and store nothing.
template <int DT>
using Word4 = typename std::conditional<DT == M5K_F32, uint4, uint2>::type;

template <int DT, int B, int CPT>
__global__ __launch_bounds__(kThreads) void rotate_kernel(const void* __restrict__ x, int64_t total_tiles, int64_t k,
                                                          const int8_t* __restrict__ signs, float* __restrict__ y) {
  constexpr int G = Grouped<B>::G;
  Word4<DT> xr[CPT][G];
  uint32_t sr[CPT][G];
  bool live[CPT];
  int64_t e[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t g = (static_cast<int64_t>(blockIdx.x) * CPT + i) * kThreads + threadIdx.x;
    live[i] = g < total_tiles;
    const int64_t gl = live[i] ? g : 0;
    // G = 1: tile g is elements 4g..4g+3; G > 1: unit gl / 64 is block gl / 64 of B elements.
    e[i] = G == 1 ? gl * 4 : (gl >> 6) * B + 4 * (gl & 63);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      const int64_t et = e[i] + 256 * t;
      xr[i][t] = *reinterpret_cast<const Word4<DT>*>(static_cast<const uint8_t*>(x) + et * dtype_bytes<DT>());
      sr[i][t] = *reinterpret_cast<const uint32_t*>(signs + et % k);
    }
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    float v[4 * G];
#pragma unroll
    for (int t = 0; t < G; ++t) {
      const uint32_t s = sr[i][t];
      const Word4<DT> w = xr[i][t];
      float* f = v + 4 * t;
      if constexpr (DT == M5K_F32) {
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) f[r] = __uint_as_float(u[r] ^ ((s << (24 - 8 * r)) & 0x80000000u));
      } else {
        // Sign bytes 0, 1 (2, 3) to the top bits of the two halves of the first (second) word.
        const uint32_t u[2] = {w.x ^ (__builtin_amdgcn_perm(0u, s, 0x010C000Cu) & 0x80008000u),
                               w.y ^ (__builtin_amdgcn_perm(0u, s, 0x030C020Cu) & 0x80008000u)};
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          if constexpr (DT == M5K_BF16) {
            f[2 * r] = __uint_as_float(u[r] << 16);
            f[2 * r + 1] = __uint_as_float(u[r] & 0xFFFF0000u);
          } else {
            f[2 * r] = f16_bits_to_f32(u[r] & 0xFFFFu);
            f[2 * r + 1] = f16_bits_to_f32(u[r] >> 16);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) f[r] = live[i] ? f[r] : 0.0f;
    }
    butterflies_grouped<B>(v);  // every lane participates in the exchanges
    if (live[i]) {
#pragma unroll
      for (int t = 0; t < G; ++t)
        *reinterpret_cast<float4*>(y + e[i] + 256 * t) = make_float4(v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]);
    }
  }
}

// One row per workgroup.  Every load of the row (x and signs of all CPT chunks) is issued
// before the first wait; a chunk past the row end (only when nchunks is not a multiple of the
// workgroup width, a uniform test) reads chunk 0, which is in bounds, and is zeroed.  The signs
// (+-1) enter as sign-bit flips of the packed words, the exact product with +-1.
template <int DT, int B, int CPT, int KT>
__global__ __launch_bounds__(KT) void rotate_quant_kernel(const void* __restrict__ x, int64_t k,
                                                          const int8_t* __restrict__ signs,
                                                          int8_t* __restrict__ q, float* __restrict__ scales) {
  __shared__ float red[KT / 64];
  constexpr int EPC = Shape<B>::EPC;
  constexpr int G = EPC / 8;  // 8-element groups per chunk
  const int64_t row = blockIdx.x;
  const int64_t nchunks = k / EPC;
  const bool ragged = nchunks < static_cast<int64_t>(CPT) * KT;
  const uint8_t* xrow = static_cast<const uint8_t*>(x) + row * k * dtype_bytes<DT>();
  Raw8<DT> xr[CPT][G];
  uint2 sr[CPT][G];
  bool live[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(i) * KT;
    live[i] = c < nchunks;
    const uint32_t j0 = static_cast<uint32_t>((live[i] ? c : 0) * EPC);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      xr[i][t] = fetch8_at<DT>(xrow, j0 + 8 * t);
      sr[i][t] = *reinterpret_cast<const uint2*>(signs + j0 + 8 * t);
    }
  }
  float v[CPT][EPC];
  float peak = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
#pragma unroll
    for (int t = 0; t < G; ++t) {
      float f[8];
      decode8<DT>(SignMask8<DT>(sr[i][t]).apply(xr[i][t]), f);
#pragma unroll
      for (int b = 0; b < 8; ++b) v[i][8 * t + b] = f[b];
    }
    if (ragged && !live[i]) {
#pragma unroll
      for (int r = 0; r < EPC; ++r) v[i][r] = 0.0f;
    }
    butterflies<B, false>(v[i]);
#pragma unroll
    for (int r = 0; r < EPC; r += 2) peak = fmaxf(peak, fmaxf(fabsf(v[i][r]), fabsf(v[i][r + 1])));
  }
  const FoldedI8<B> enc(block_max<KT / 64>(peak, red));
  if (threadIdx.x == 0) scales[row] = enc.scale;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    if (live[i]) {
      const int64_t c = threadIdx.x + static_cast<int64_t>(i) * KT;
      uint2* out = reinterpret_cast<uint2*>(q + row * k + c * EPC);
#pragma unroll
      for (int t = 0; t < G; ++t) {
        float g[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) g[b] = v[i][8 * t + b];
        uint32_t w[2];
        enc.template encode<8>(g, w);
        out[t] = make_uint2(w[0], w[1]);
      }
    }
  }
}

template <int DT, int B>
int launch_rotate(const void* x, int64_t rows, int64_t k, const int8_t* signs, float* y, hipStream_t st) {
  // Two tiles per thread for 2-byte inputs; FP32 tiles are already 16-byte loads, and one tile
  // per thread measured 85.4 us against 91.4 us for two at [4096, 16384] H128.
  constexpr int CPT = DT == M5K_F32 ? 1 : 2;
  const int64_t total = rows * k / 4 / Grouped<B>::G;
  const int64_t blocks = (total + CPT * kThreads - 1) / (CPT * kThreads);
  M5K_REQUIRE(blocks <= 0x7FFFFFFF, "m5k_hadamard_rotate: input too large");
  rotate_kernel<DT, B, CPT><<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st>>>(x, total, k, signs, y);
  return launch_status("m5k_hadamard_rotate");
}

template <int DT, int B, int CPT, int KT>
void rq_launch(dim3 grid, const void* x, int64_t k, const int8_t* signs, int8_t* q, float* s, hipStream_t st) {
  rotate_quant_kernel<DT, B, CPT, KT><<<grid, dim3(KT), 0, st>>>(x, k, signs, q, s);
}

template <int DT, int B>
int launch_rotate_quant(const void* x, int64_t rows, int64_t k, const int8_t* signs, int8_t* q, float* s,
                        hipStream_t st) {
  // One workgroup per row, as wide as leaves each thread about 32 values: 4 chunks of 8 (256
  // or 512 threads) or 2 chunks of 16 (B = 1024).  At [4096, 16384] H128 512 x 4 measured
  // 34.3 us against 38.0 us for 1024 x 2 and 39.8 us for 256 x 8; at K 8192, 256 x 4 19.9 us
  // against 20.9 us for 512 x 2.  A block's LPB lanes stay inside one wave at every width
  // (chunk c sits on thread c mod KT, and LPB divides 64).  The row peak is
  // order-independent, so the codes do not depend on the width.
  const int64_t chunks = k / Shape<B>::EPC;
  const dim3 grid(static_cast<unsigned>(rows));
  constexpr bool WIDE = Shape<B>::EPC >= 16;
  if (chunks <= 256) rq_launch<DT, B, 1, 256>(grid, x, k, signs, q, s, st);
  else if (chunks <= 512) rq_launch<DT, B, 2, 256>(grid, x, k, signs, q, s, st);
  else if (chunks <= 768) rq_launch<DT, B, 3, 256>(grid, x, k, signs, q, s, st);
  else if (chunks <= 1024) {
    if constexpr (WIDE) rq_launch<DT, B, 2, 512>(grid, x, k, signs, q, s, st);
    else rq_launch<DT, B, 4, 256>(grid, x, k, signs, q, s, st);
  } else if (chunks <= 2048) {
    if constexpr (WIDE) rq_launch<DT, B, 2, 1024>(grid, x, k, signs, q, s, st);
    else rq_launch<DT, B, 4, 512>(grid, x, k, signs, q, s, st);
  } else if (chunks <= 4096) rq_launch<DT, B, 4, 1024>(grid, x, k, signs, q, s, st);
  else {
    set_error("m5k_hadamard_quantize_rows: K=%lld exceeds the register-resident row limit %d", (long long)k,
              4 * 1024 * Shape<B>::EPC);
    return M5K_EINVAL;
  }
  return launch_status("m5k_hadamard_quantize_rows");
}

template <int DT, template <int, int> class Launcher, class... Args>
int by_block(int block, Args... args) {
  switch (block) {
    case 32: return Launcher<DT, 32>::run(args...);
    case 64: return Launcher<DT, 64>::run(args...);
    case 128: return Launcher<DT, 128>::run(args...);
    case 256: return Launcher<DT, 256>::run(args...);
    case 512: return Launcher<DT, 512>::run(args...);
    case 1024: return Launcher<DT, 1024>::run(args...);
    default: set_error("unsupported Hadamard block %d", block); return M5K_EINVAL;
  }
}

template <int DT, int B>
struct RotateL {
  static int run(const void* x, int64_t rows, int64_t k, const int8_t* signs, float* y, hipStream_t st) {
    return launch_rotate<DT, B>(x, rows, k, signs, y, st);
  }
};

template <int DT, int B>
struct RotateQuantL {
  static int run(const void* x, int64_t rows, int64_t k, const int8_t* signs, int8_t* q, float* s,
                 hipStream_t st) {
    return launch_rotate_quant<DT, B>(x, rows, k, signs, q, s, st);
  }
};

int check_args(const void* x, int x_dtype, int64_t rows, int64_t k, int block, const int8_t* signs,
               const char* name) {
  M5K_REQUIRE(x && signs, "%s: null pointer", name);
  M5K_REQUIRE(rows > 0 && k > 0, "%s: empty shape", name);
  M5K_REQUIRE(block >= 32 && block <= 1024 && (block & (block - 1)) == 0, "%s: block %d not in {32..1024}", name,
              block);
  M5K_REQUIRE(k % block == 0, "%s: K=%lld not divisible by block %d", name, (long long)k, block);
  M5K_REQUIRE(x_dtype == M5K_BF16 || x_dtype == M5K_F16 || x_dtype == M5K_F32, "%s: unsupported dtype %d", name,
              x_dtype);
  M5K_REQUIRE(aligned16(x) && (reinterpret_cast<uintptr_t>(signs) & 7u) == 0,
              "%s: x must be 16-byte and signs 8-byte aligned", name);
  return M5K_OK;
}

}  // namespace
}  // namespace hadamard
}  // namespace m5k

using namespace m5k;
using namespace m5k::hadamard;

extern "C" int m5k_hadamard_rotate(const void* x, int x_dtype, int64_t rows, int64_t k, int block,
                                   const int8_t* signs, float* y, void* stream) {
  clear_error();
  const char* name = "m5k_hadamard_rotate";
  if (int rc = check_args(x, x_dtype, rows, k, block, signs, name)) return rc;
  M5K_REQUIRE(y && aligned16(y), "%s: y must be a 16-byte aligned pointer", name);
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return by_block<M5K_BF16, RotateL>(block, x, rows, k, signs, y, st);
    case M5K_F16: return by_block<M5K_F16, RotateL>(block, x, rows, k, signs, y, st);
    default: return by_block<M5K_F32, RotateL>(block, x, rows, k, signs, y, st);
  }
}

extern "C" int m5k_hadamard_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int block,
                                          const int8_t* signs, int8_t* q, float* scales, void* stream) {
  clear_error();
  const char* name = "m5k_hadamard_quantize_rows";
  if (int rc = check_args(x, x_dtype, rows, k, block, signs, name)) return rc;
  M5K_REQUIRE(q && scales && (reinterpret_cast<uintptr_t>(q) & 7u) == 0, "%s: q must be 8-byte aligned", name);
  M5K_REQUIRE(rows <= 0x7FFFFFFF, "%s: too many rows", name);
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return by_block<M5K_BF16, RotateQuantL>(block, x, rows, k, signs, q, scales, st);
    case M5K_F16: return by_block<M5K_F16, RotateQuantL>(block, x, rows, k, signs, q, scales, st);
    default: return by_block<M5K_F32, RotateQuantL>(block, x, rows, k, signs, q, scales, st);
  }
}
