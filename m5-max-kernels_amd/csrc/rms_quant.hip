// RMS dynamic INT8 quantization with the inverse RMS folded into the row scales.
//
// Contract: rms_quant.py:41-117 with the arithmetic of shaders/rms_quant.metal:1-97.  For a
// row x[K], FP32 gamma[K] and +-1 signs[K]:
//   ss    = sum x^2 (the original input);  inv = 1 / sqrt(ss / K + eps)
//   v     = fold ? (x * gamma) * s : ((x * inv) * gamma) * s
//   z     = blockdiag(H_B) v for B >= 32 (natural-order Sylvester, FP32, * 1/sqrt(B)); z = v for B = 1
//   peak  = max |z|;  scale = peak == 0 ? 1 : (peak * (fold ? inv : 1)) / 127
//   code  = peak == 0 ? 0 : clamp(rint((z / peak) * 127), -127, 127)
// There is no additive shift and no reduced-precision intermediate, so the positive inverse
// RMS moves only the scales (fold = true) and the row peak and statistics can share one
// barrier.  One workgroup of 4 wave64 per row; for B >= 32 a lane holds NCH chunks of EPC
// consecutive elements in VGPRs, for B = 1 (any K) the row is read through the cache per pass.
#include "hadamard_core.h"

namespace m5k {
namespace rmsq {
namespace {

using hadamard::Shape;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct RmsParams {
  const void* x;
  const float* gamma;
  const int8_t* signs;
  int8_t* q;
  float* scales;
  int64_t k;
  float eps;
};

template <int DT>
__device__ __forceinline__ void load8x(const void* base, int64_t e, float (&v)[8]) {
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
      v[2 * i] = DT == M5K_BF16 ? __uint_as_float(w[i] << 16) : f16_bits_to_f32(w[i] & 0xFFFFu);
      v[2 * i + 1] = DT == M5K_BF16 ? __uint_as_float(w[i] & 0xFFFF0000u) : f16_bits_to_f32(w[i] >> 16);
    }
  }
}

__device__ __forceinline__ uint32_t rms_code(float z, float peak) {
  return peak == 0.0f ? 0u : i8_clamp_code(rintf((z / peak) * 127.0f));
}

// Workgroup max of m and sum of s through one barrier: the same wave reductions and the same
// in-order combination of the wave partials as block_max and block_sum.
__device__ __forceinline__ float2 block_max_sum(float m, float s, float2* lds) {
  m = wave_max(m);
  s = wave_sum(s);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = make_float2(m, s);
  __syncthreads();
  float2 r = lds[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    r.x = fmaxf(r.x, lds[w].x);
    r.y += lds[w].y;
  }
  return r;
}

// Block-Hadamard variant (B >= 32, K % B == 0).
template <int XDT, int B, int NCH, bool FOLD>
__global__ __launch_bounds__(kThreads) void rms_quant_block_kernel(RmsParams p) {
  __shared__ float red[2 * kWaves];  // unfolded: statistics, then peak
  __shared__ float2 red2[kWaves];    // folded: peak and sum of squares
  constexpr int EPC = Shape<B>::EPC;
  constexpr int NV = NCH * EPC;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t nchunks = p.k / EPC;
  const float kf = static_cast<float>(p.k);
  // Every load of the row (x, gamma and signs of all chunks) is issued before any value is
  // used, so their latencies overlap.  A lane whose chunk lies past the row end reads chunk 0
  // (in bounds) and zeroes what it read; rows with no such chunk (nchunks a multiple of the
  // workgroup width, uniform) skip the selects.
  const bool ragged = nchunks < static_cast<int64_t>(NCH) * kThreads;
  float v[NV], g[NV];
  uint2 sg[NV / 8];
  bool live[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * kThreads;
    live[i] = c < nchunks;
    const int64_t j0 = (live[i] ? c : 0) * EPC;
#pragma unroll
    for (int h = 0; h < EPC / 8; ++h) {
      const int64_t j = j0 + 8 * h;
      float t[8];
      load8x<XDT>(p.x, row * p.k + j, t);
      const float4 g0 = *reinterpret_cast<const float4*>(p.gamma + j);
      const float4 g1 = *reinterpret_cast<const float4*>(p.gamma + j + 4);
      const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      sg[(i * EPC) / 8 + h] = *reinterpret_cast<const uint2*>(p.signs + j);
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        v[i * EPC + 8 * h + r] = t[r];
        g[i * EPC + 8 * h + r] = gg[r];
      }
    }
  }
  if (ragged) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
#pragma unroll
      for (int r = 0; r < EPC; ++r) {
        v[i * EPC + r] = live[i] ? v[i * EPC + r] : 0.0f;
        g[i * EPC + r] = live[i] ? g[i * EPC + r] : 0.0f;
      }
    }
  }
  // The statistics feed only the inverse RMS; the sum of squares takes one fma per element
  // (its order is this kernel's own either way).
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < NV; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
  float inv = 1.0f;
  if constexpr (!FOLD) inv = 1.0f / sqrtf(block_sum<kWaves>(ss, red) / kf + p.eps);
  float peak = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    float z[EPC];
#pragma unroll
    for (int h = 0; h < EPC / 8; ++h) {
      const uint2 sw = sg[(i * EPC) / 8 + h];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float s = static_cast<float>(static_cast<int8_t>(((r < 4 ? sw.x : sw.y) >> (8 * (r & 3))) & 0xFFu));
        const float x = v[i * EPC + 8 * h + r];
        const float gr = g[i * EPC + 8 * h + r];
        z[8 * h + r] = FOLD ? (x * gr) * s : ((x * inv) * gr) * s;
      }
    }
    hadamard::butterflies<B, false>(z);
#pragma unroll
    for (int r = 0; r < EPC; r += 2) {
      v[i * EPC + r] = z[r];
      v[i * EPC + r + 1] = z[r + 1];
      peak = fmaxf(peak, fmaxf(fabsf(z[r]), fabsf(z[r + 1])));
    }
  }
  // The butterflies leave out the 1/sqrt(B) multiply: the reference's z is fl(z' * c), whose
  // row peak is fl(max |z'| * c) (rounding is monotone), and its code
  // rint(fl(fl(z / peak) * 127)), three roundings of z' * m for m = 127 c / peak, bracketed
  // by the estimate m~ = fl(c * fl(127 / peak)) (two roundings; 0 for a zero or infinite peak,
  // where every finite z codes to 0).
  constexpr float c = hadamard::inv_sqrt_block<B>();
  if constexpr (FOLD) {
    // Peak and sum of squares share one barrier; only the lane that writes the scale needs
    // the inverse RMS.
    const float2 ps = block_max_sum(peak, ss, red2);
    peak = ps.x * c;
    if (tid == 0) p.scales[row] = peak == 0.0f ? 1.0f : (peak * (1.0f / sqrtf(ps.y / kf + p.eps))) / 127.0f;
  } else {
    peak = block_max<kWaves>(peak, red + kWaves) * c;
    if (tid == 0) p.scales[row] = peak == 0.0f ? 1.0f : peak / 127.0f;
  }
  const I8Bracket enc = i8_bracket(peak == 0.0f ? 0.0f : c * (127.0f / peak), false);
  const auto chain = [peak](float zu) { return rms_code(zu * c, peak); };
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (live[i]) {
      const int64_t col = (tid + static_cast<int64_t>(i) * kThreads) * EPC;
#pragma unroll
      for (int h = 0; h < EPC / 8; ++h) {
        float t[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) t[r] = v[i * EPC + 8 * h + r];
        uint32_t w[2];
        encode_i8<8>(t, enc, chain, w);
        *reinterpret_cast<uint2*>(p.q + row * p.k + col + 8 * h) = make_uint2(w[0], w[1]);
      }
    }
  }
}

// B = 1 (no transform, any K): three passes over the cached row.
template <int XDT, bool FOLD>
__global__ __launch_bounds__(kThreads) void rms_quant_plain_kernel(RmsParams p) {
  __shared__ float red[3 * kWaves];
  const int64_t row = blockIdx.x;
  const int64_t base = row * p.k;
  const float kf = static_cast<float>(p.k);
  float ss = 0.0f, peak = 0.0f;
  for (int64_t j = threadIdx.x; j < p.k; j += kThreads) {
    const float x = load_elem<XDT>(p.x, base + j);
    ss += x * x;
    if constexpr (FOLD) peak = fmaxf(peak, fabsf((x * p.gamma[j]) * static_cast<float>(p.signs[j])));
  }
  float inv = 1.0f;
  if constexpr (!FOLD) {
    inv = 1.0f / sqrtf(block_sum<kWaves>(ss, red) / kf + p.eps);
    for (int64_t j = threadIdx.x; j < p.k; j += kThreads) {
      const float x = load_elem<XDT>(p.x, base + j);
      peak = fmaxf(peak, fabsf(((x * inv) * p.gamma[j]) * static_cast<float>(p.signs[j])));
    }
  }
  peak = block_max<kWaves>(peak, red + kWaves);
  if constexpr (FOLD) inv = 1.0f / sqrtf(block_sum<kWaves>(ss, red + 2 * kWaves) / kf + p.eps);
  if (threadIdx.x == 0) p.scales[row] = peak == 0.0f ? 1.0f : (FOLD ? peak * inv : peak) / 127.0f;
  for (int64_t j = threadIdx.x; j < p.k; j += kThreads) {
    const float x = load_elem<XDT>(p.x, base + j);
    const float s = static_cast<float>(p.signs[j]);
    const float z = FOLD ? (x * p.gamma[j]) * s : ((x * inv) * p.gamma[j]) * s;
    p.q[base + j] = static_cast<int8_t>(rms_code(z, peak));
  }
}

template <int XDT, int B, bool FOLD>
int launch_block(const RmsParams& p, int64_t rows, hipStream_t st) {
  const int64_t per_thread = (p.k / Shape<B>::EPC + kThreads - 1) / kThreads;
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  if (per_thread <= 1) rms_quant_block_kernel<XDT, B, 1, FOLD><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 2) rms_quant_block_kernel<XDT, B, 2, FOLD><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 3) rms_quant_block_kernel<XDT, B, 3, FOLD><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 4) rms_quant_block_kernel<XDT, B, 4, FOLD><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 8) rms_quant_block_kernel<XDT, B, 8, FOLD><<<grid, block, 0, st>>>(p);
  else {
    set_error("m5k_rms_quantize: K=%lld exceeds the register-resident row limit %d", (long long)p.k,
              8 * kThreads * Shape<B>::EPC);
    return M5K_EINVAL;
  }
  return launch_status("m5k_rms_quantize");
}

template <int XDT, bool FOLD>
int by_block(int block, const RmsParams& p, int64_t rows, hipStream_t st) {
  switch (block) {
    case 1: rms_quant_plain_kernel<XDT, FOLD><<<dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st>>>(p);
            return launch_status("m5k_rms_quantize");
    case 32: return launch_block<XDT, 32, FOLD>(p, rows, st);
    case 64: return launch_block<XDT, 64, FOLD>(p, rows, st);
    case 128: return launch_block<XDT, 128, FOLD>(p, rows, st);
    case 256: return launch_block<XDT, 256, FOLD>(p, rows, st);
    case 512: return launch_block<XDT, 512, FOLD>(p, rows, st);
    case 1024: return launch_block<XDT, 1024, FOLD>(p, rows, st);
    default: set_error("m5k_rms_quantize: unsupported block %d", block); return M5K_EINVAL;
  }
}

template <int XDT>
int by_fold(int fold, int block, const RmsParams& p, int64_t rows, hipStream_t st) {
  return fold ? by_block<XDT, true>(block, p, rows, st) : by_block<XDT, false>(block, p, rows, st);
}

}  // namespace
}  // namespace rmsq
}  // namespace m5k

using namespace m5k;
using namespace m5k::rmsq;

extern "C" int m5k_rms_quantize(const void* x, int x_dtype, int64_t rows, int64_t k, const float* gamma,
                                const int8_t* signs, int block, int fold_scale, float epsilon, int8_t* q,
                                float* scales, void* stream) {
  clear_error();
  const char* name = "m5k_rms_quantize";
  M5K_REQUIRE(x && gamma && signs && q && scales, "%s: null pointer", name);
  M5K_REQUIRE(rows > 0 && k > 0 && rows <= 0x7FFFFFFF, "%s: bad shape [%lld,%lld]", name, (long long)rows,
              (long long)k);
  M5K_REQUIRE(block == 1 || (block >= 32 && block <= 1024 && (block & (block - 1)) == 0 && k % block == 0),
              "%s: block %d must be 1 or a power of two in [32,1024] dividing K", name, block);
  M5K_REQUIRE(epsilon > 0.0f, "%s: epsilon must be positive", name);
  M5K_REQUIRE(block == 1 || (aligned16(x) && aligned16(gamma) && (reinterpret_cast<uintptr_t>(signs) & 7u) == 0 &&
                             (reinterpret_cast<uintptr_t>(q) & 7u) == 0),
              "%s: misaligned buffers", name);
  const RmsParams p{x, gamma, signs, q, scales, k, epsilon};
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return by_fold<M5K_BF16>(fold_scale, block, p, rows, st);
    case M5K_F16: return by_fold<M5K_F16>(fold_scale, block, p, rows, st);
    case M5K_F32: return by_fold<M5K_F32>(fold_scale, block, p, rows, st);
    default: set_error("%s: unsupported input dtype %d", name, x_dtype); return M5K_EINVAL;
  }
}
