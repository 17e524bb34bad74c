// Fused row preparation for the W8A8 projection (one dispatch per activation matrix):
//
//   [gated]  r = R(float(X) + float(Branch) * float(Gate[g + j]))   -> written once as R_next
//   stats    RMS: var = sum(r^2)/K            LayerNorm: mean = sum(r)/K, var = sum((r-mean)^2)/K
//            inv = 1 / sqrt(var + eps)         (IEEE division and square root)
//   modulate y = O(((r - mean) * inv * gamma[j]) * (1 + scale[t + j]) + shift[t + j])
//   rotate   z = blockdiag(H_B) (y * signs)   (natural-order Sylvester, FP32, * 1/sqrt(B))
//   quantize s = max|z| / 127 (1 if 0); q = clamp(rint_even(z / s), -127, 127)
//
// Contract: norm_hadamard.py:122-265 with the arithmetic of shaders/norm_hadamard.metal:19-118
// (R/O are the residual dtype and the round_output dtype; t and g are row-map table offsets).
// The staged comparators gated_residual_add (gated_residual.metal) and norm_modulate
// (norm_modulate.metal) run the same per-element arithmetic and the same reduction tree, so
// staged rotate(quantize(...)) reproduces the fused codes bit for bit (blocks <= 512).
//
// Layout: one workgroup (4 wave64) per row; a lane owns CPT chunks of EPC consecutive
// elements (chunk c = tid + 256*i), the whole row stays in VGPRs: HBM traffic is the
// minimum 2K (+2K branch, +2K R_next) + K + 4 bytes per row plus the parameter tables.
#include "hadamard_core.h"

namespace m5k {
namespace prep {
namespace {

using hadamard::Shape;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct PrepParams {
  const void* x;          // residual or X [rows, k] (XDT)
  const void* branch;     // [rows, k] (XDT) or null: ungated
  const void* gate;       // [k] or [P, k] (PDT)
  const int32_t* gate_map;
  const void* gamma;      // [k] (PDT)
  const void* scale;      // [k] or [P, k] (PDT)
  const void* shift;      // [k] or [P, k] (PDT)
  const int32_t* row_map;
  const int8_t* signs;    // [k]
  int8_t* q;              // [rows, k]
  float* scales;          // [rows]
  void* r_next;           // [rows, k] (XDT), gated only
  void* y;                // staged norm output [rows, k] (round dtype)
  int64_t k;
  float eps;
  int layer;              // 1: LayerNorm, 0: RMS
  int round_input;        // 1: O = XDT, 0: O = FP32
};

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
      v[2 * i] = DT == M5K_BF16 ? bf16_bits_to_f32(w[i] & 0xFFFFu) : f16_bits_to_f32(w[i] & 0xFFFFu);
      v[2 * i + 1] = DT == M5K_BF16 ? bf16_bits_to_f32(w[i] >> 16) : f16_bits_to_f32(w[i] >> 16);
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t e, const float (&v)[8]) {
  uint4* p = reinterpret_cast<uint4*>(static_cast<uint8_t*>(base) + e * dtype_bytes<DT>());
  if constexpr (DT == M5K_F32) {
    p[0] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
    p[1] = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7]));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = DT == M5K_BF16 ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
      const uint32_t hi = DT == M5K_BF16 ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
      w[i] = lo | (hi << 16);
    }
    p[0] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Row input for chunk c (8 elements at column j = 8c): X, or the gated residual update,
// rounded to the residual dtype and written to R_next.
template <int XDT, int PDT, bool GATED>
__device__ __forceinline__ void load_row_chunk(const PrepParams& p, int64_t row, int64_t j, float (&v)[8]) {
  const int64_t e = row * p.k + j;
  load8<XDT>(p.x, e, v);
  if constexpr (GATED) {
    float b[8], g[8];
    load8<XDT>(p.branch, e, b);
    const int64_t goff = p.gate_map ? static_cast<int64_t>(p.gate_map[row]) * p.k : 0;
    load8<PDT>(p.gate, goff + j, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_through<XDT>(v[i] + b[i] * g[i]);
    store8<XDT>(p.r_next, e, v);
  }
}

// Row statistics over the register-resident row: (mean, inv).  The reduction tree (lane
// partials in chunk order, wave xor-butterfly, waves summed in order) is shared by the fused
// and staged kernels.
template <int NV>
__device__ __forceinline__ void row_stats(const float (&v)[NV], const bool (&live)[NV / 8], int64_t k, int layer,
                                          float eps, float* red, float& mean, float& inv) {
  const float kf = static_cast<float>(k);
  float first = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) first += layer ? v[i] : v[i] * v[i];
  first = block_sum<kWaves>(first, red) / kf;
  mean = layer ? first : 0.0f;
  float var = first;
  if (layer) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float c = live[i / 8] ? v[i] - mean : 0.0f;
      acc += c * c;
    }
    var = block_sum<kWaves>(acc, red) / kf;
  }
  inv = 1.0f / sqrtf(var + eps);
}

// Modulation of 8 values of chunk j, then the O(...) cast.
template <int PDT>
__device__ __forceinline__ void modulate8(const PrepParams& p, int64_t row, int64_t j, float mean, float inv,
                                          int round_dt, float (&v)[8]) {
  float g[8], sc[8], sh[8];
  const int64_t toff = p.row_map ? static_cast<int64_t>(p.row_map[row]) * p.k : 0;
  load8<PDT>(p.gamma, j, g);
  load8<PDT>(p.scale, toff + j, sc);
  load8<PDT>(p.shift, toff + j, sh);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float normalized = (v[i] - mean) * inv * g[i];
    const float modulated = normalized * (1.0f + sc[i]) + sh[i];
    v[i] = round_dt == M5K_BF16 ? round_through<M5K_BF16>(modulated)
           : round_dt == M5K_F16 ? round_through<M5K_F16>(modulated)
                                 : modulated;
  }
}

// Fused kernel.  CPT chunks of EPC elements per lane.
template <int XDT, int PDT, int B, int CPT, bool GATED>
__global__ __launch_bounds__(kThreads) void fused_prep_kernel(PrepParams p) {
  __shared__ float red[kWaves];
  constexpr int EPC = Shape<B>::EPC;
  constexpr int NV = CPT * EPC;
  const int64_t row = blockIdx.x;
  const int64_t nchunks = p.k / EPC;
  float v[NV];
  bool live[NV / 8];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(i) * kThreads;
#pragma unroll
    for (int h = 0; h < EPC / 8; ++h) {
      float t[8];
      live[i * (EPC / 8) + h] = c < nchunks;
      if (c < nchunks) {
        load_row_chunk<XDT, PDT, GATED>(p, row, c * EPC + 8 * h, t);
      } else {
#pragma unroll
        for (int r = 0; r < 8; ++r) t[r] = 0.0f;
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) v[i * EPC + 8 * h + r] = t[r];
    }
  }
  float mean, inv;
  row_stats<NV>(v, live, p.k, p.layer, p.eps, red, mean, inv);
  const int round_dt = p.round_input ? XDT : M5K_F32;
  float peak = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(i) * kThreads;
    float z[EPC];
#pragma unroll
    for (int h = 0; h < EPC / 8; ++h) {
      float t[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) t[r] = v[i * EPC + 8 * h + r];
      if (c < nchunks) {
        const int64_t j = c * EPC + 8 * h;
        modulate8<PDT>(p, row, j, mean, inv, round_dt, t);
        const uint2 sg = *reinterpret_cast<const uint2*>(p.signs + j);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const uint32_t byte = ((r < 4 ? sg.x : sg.y) >> (8 * (r & 3))) & 0xFFu;
          t[r] = t[r] * static_cast<float>(static_cast<int8_t>(byte));
        }
      } else {
#pragma unroll
        for (int r = 0; r < 8; ++r) t[r] = 0.0f;
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) z[8 * h + r] = t[r];
    }
    hadamard::butterflies<B>(z);
#pragma unroll
    for (int r = 0; r < EPC; ++r) {
      v[i * EPC + r] = z[r];
      peak = fmaxf(peak, fabsf(z[r]));
    }
  }
  peak = block_max<kWaves>(peak, red);
  const I8Scale enc = i8_scale(quant_scale<M5K_QUANT_INT8>(peak));
  if (threadIdx.x == 0) p.scales[row] = enc.scale;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(i) * kThreads;
    if (c < nchunks) {
      uint2* out = reinterpret_cast<uint2*>(p.q + row * p.k + c * EPC);
#pragma unroll
      for (int t = 0; t < EPC / 8; ++t) {
        float g[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) g[b] = v[i * EPC + 8 * t + b];
        uint32_t w[2];
        encode_i8<8>(g, enc, w);
        out[t] = make_uint2(w[0], w[1]);
      }
    }
  }
}

// Staged norm + modulation (norm_modulate.metal): the fused kernel's EPC = 8 chunking and
// reduction tree, output in the round dtype.
template <int XDT, int PDT, int CPT>
__global__ __launch_bounds__(kThreads) void norm_modulate_kernel(PrepParams p) {
  __shared__ float red[kWaves];
  constexpr int NV = CPT * 8;
  const int64_t row = blockIdx.x;
  const int64_t nchunks = p.k / 8;
  float v[NV];
  bool live[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(i) * kThreads;
    float t[8];
    live[i] = c < nchunks;
    if (c < nchunks) {
      load8<XDT>(p.x, row * p.k + c * 8, t);
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) t[r] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) v[8 * i + r] = t[r];
  }
  float mean, inv;
  row_stats<NV>(v, live, p.k, p.layer, p.eps, red, mean, inv);
  const int round_dt = p.round_input ? XDT : M5K_F32;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(i) * kThreads;
    if (c < nchunks) {
      float t[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) t[r] = v[8 * i + r];
      modulate8<PDT>(p, row, c * 8, mean, inv, round_dt, t);
      if (p.round_input) store8<XDT>(p.y, row * p.k + c * 8, t);
      else store8<M5K_F32>(p.y, row * p.k + c * 8, t);
    }
  }
}

// Staged gated residual add (gated_residual.metal): 8 elements per thread.
template <int XDT, int PDT>
__global__ __launch_bounds__(kThreads) void gated_residual_kernel(PrepParams p, int64_t total_chunks) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= total_chunks) return;
  const int64_t e = c * 8;
  const int64_t row = e / p.k, j = e - row * p.k;
  float v[8];
  load_row_chunk<XDT, PDT, true>(p, row, j, v);  // writes R_next
}

template <int XDT, int PDT, int B, bool GATED>
int launch_fused(const PrepParams& p, int64_t rows, hipStream_t st) {
  const int64_t per_thread = (p.k / Shape<B>::EPC + kThreads - 1) / kThreads;
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  if (per_thread <= 1) fused_prep_kernel<XDT, PDT, B, 1, GATED><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 2) fused_prep_kernel<XDT, PDT, B, 2, GATED><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 4) fused_prep_kernel<XDT, PDT, B, 4, GATED><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 8) fused_prep_kernel<XDT, PDT, B, 8, GATED><<<grid, block, 0, st>>>(p);
  else {
    set_error("m5k_norm_hadamard_quantize: K=%lld exceeds the register-resident row limit %d", (long long)p.k,
              8 * kThreads * Shape<B>::EPC);
    return M5K_EINVAL;
  }
  return launch_status("m5k_norm_hadamard_quantize");
}

template <int XDT, int PDT, bool GATED>
int fused_by_block(int block, const PrepParams& p, int64_t rows, hipStream_t st) {
  switch (block) {
    case 32: return launch_fused<XDT, PDT, 32, GATED>(p, rows, st);
    case 64: return launch_fused<XDT, PDT, 64, GATED>(p, rows, st);
    case 128: return launch_fused<XDT, PDT, 128, GATED>(p, rows, st);
    case 256: return launch_fused<XDT, PDT, 256, GATED>(p, rows, st);
    case 512: return launch_fused<XDT, PDT, 512, GATED>(p, rows, st);
    case 1024: return launch_fused<XDT, PDT, 1024, GATED>(p, rows, st);
    default: set_error("m5k_norm_hadamard_quantize: unsupported block %d", block); return M5K_EINVAL;
  }
}

template <int XDT, int PDT>
int fused_dispatch(int block, const PrepParams& p, int64_t rows, hipStream_t st) {
  return p.branch ? fused_by_block<XDT, PDT, true>(block, p, rows, st)
                  : fused_by_block<XDT, PDT, false>(block, p, rows, st);
}

template <int XDT>
int fused_by_param(int pdt, int block, const PrepParams& p, int64_t rows, hipStream_t st) {
  return pdt == M5K_BF16 ? fused_dispatch<XDT, M5K_BF16>(block, p, rows, st)
                         : fused_dispatch<XDT, M5K_F32>(block, p, rows, st);
}

template <int XDT, int PDT>
int launch_norm(const PrepParams& p, int64_t rows, hipStream_t st) {
  const int64_t per_thread = (p.k / 8 + kThreads - 1) / kThreads;
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  if (per_thread <= 1) norm_modulate_kernel<XDT, PDT, 1><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 2) norm_modulate_kernel<XDT, PDT, 2><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 4) norm_modulate_kernel<XDT, PDT, 4><<<grid, block, 0, st>>>(p);
  else if (per_thread <= 8) norm_modulate_kernel<XDT, PDT, 8><<<grid, block, 0, st>>>(p);
  else {
    set_error("m5k_norm_modulate: K=%lld exceeds the register-resident row limit %d", (long long)p.k, 8 * kThreads * 8);
    return M5K_EINVAL;
  }
  return launch_status("m5k_norm_modulate");
}

template <int XDT>
int norm_by_param(int pdt, const PrepParams& p, int64_t rows, hipStream_t st) {
  return pdt == M5K_BF16 ? launch_norm<XDT, M5K_BF16>(p, rows, st) : launch_norm<XDT, M5K_F32>(p, rows, st);
}

template <int XDT, int PDT>
int launch_gate(const PrepParams& p, int64_t rows, hipStream_t st) {
  const int64_t chunks = rows * p.k / 8;
  const int64_t blocks = (chunks + kThreads - 1) / kThreads;
  M5K_REQUIRE(blocks <= 0x7FFFFFFF, "m5k_gated_residual_add: input too large");
  gated_residual_kernel<XDT, PDT><<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st>>>(p, chunks);
  return launch_status("m5k_gated_residual_add");
}

template <int XDT>
int gate_by_param(int pdt, const PrepParams& p, int64_t rows, hipStream_t st) {
  return pdt == M5K_BF16 ? launch_gate<XDT, M5K_BF16>(p, rows, st) : launch_gate<XDT, M5K_F32>(p, rows, st);
}

bool a16(const void* ptr) { return ptr == nullptr || aligned16(ptr); }

int check_common(const void* x, int x_dtype, int64_t rows, int64_t k, int param_dtype, const char* name) {
  M5K_REQUIRE(x, "%s: null input", name);
  M5K_REQUIRE(rows > 0 && k > 0 && rows <= 0x7FFFFFFF, "%s: bad shape [%lld,%lld]", name, (long long)rows,
              (long long)k);
  M5K_REQUIRE(k % 8 == 0, "%s: K=%lld must be a multiple of 8", name, (long long)k);
  M5K_REQUIRE(x_dtype == M5K_BF16 || x_dtype == M5K_F16 || x_dtype == M5K_F32, "%s: unsupported input dtype %d",
              name, x_dtype);
  M5K_REQUIRE(param_dtype == M5K_BF16 || param_dtype == M5K_F32, "%s: parameter dtype must be BF16 or F32", name);
  return M5K_OK;
}

}  // namespace
}  // namespace prep
}  // namespace m5k

using namespace m5k;
using namespace m5k::prep;

extern "C" int m5k_norm_hadamard_quantize(const void* x, int x_dtype, int64_t rows, int64_t k, const void* branch,
                                          const void* gate, const int32_t* gate_row_map, const void* gamma,
                                          const void* scale, const void* shift, int param_dtype,
                                          const int32_t* row_map, const int8_t* signs, int block, int norm,
                                          float epsilon, int round_to_input, int8_t* q, float* scales,
                                          void* residual_out, void* stream) {
  clear_error();
  const char* name = "m5k_norm_hadamard_quantize";
  if (int rc = check_common(x, x_dtype, rows, k, param_dtype, name)) return rc;
  M5K_REQUIRE(gamma && scale && shift && signs && q && scales, "%s: null pointer", name);
  M5K_REQUIRE(block >= 32 && block <= 1024 && (block & (block - 1)) == 0 && k % block == 0,
              "%s: block %d must be a power of two in [32,1024] dividing K", name, block);
  M5K_REQUIRE(!branch || (gate && residual_out), "%s: gated prep needs gate and residual_out", name);
  M5K_REQUIRE(epsilon > 0.0f, "%s: epsilon must be positive", name);
  M5K_REQUIRE(a16(x) && a16(branch) && a16(gate) && a16(gamma) && a16(scale) && a16(shift) && a16(residual_out) &&
                  (reinterpret_cast<uintptr_t>(signs) & 7u) == 0 && (reinterpret_cast<uintptr_t>(q) & 7u) == 0,
              "%s: misaligned buffers", name);
  PrepParams p{x,     branch, gate, gate_row_map, gamma,  scale, shift, row_map, signs, q, scales, residual_out,
               nullptr, k, epsilon, norm == M5K_NORM_LAYER ? 1 : 0, round_to_input ? 1 : 0};
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return fused_by_param<M5K_BF16>(param_dtype, block, p, rows, st);
    case M5K_F16: return fused_by_param<M5K_F16>(param_dtype, block, p, rows, st);
    default: return fused_by_param<M5K_F32>(param_dtype, block, p, rows, st);
  }
}

extern "C" int m5k_norm_modulate(const void* x, int x_dtype, int64_t rows, int64_t k, const void* gamma,
                                 const void* scale, const void* shift, int param_dtype, const int32_t* row_map,
                                 int norm, float epsilon, int round_to_input, void* y, void* stream) {
  clear_error();
  const char* name = "m5k_norm_modulate";
  if (int rc = check_common(x, x_dtype, rows, k, param_dtype, name)) return rc;
  M5K_REQUIRE(gamma && scale && shift && y, "%s: null pointer", name);
  M5K_REQUIRE(epsilon > 0.0f, "%s: epsilon must be positive", name);
  M5K_REQUIRE(a16(x) && a16(gamma) && a16(scale) && a16(shift) && a16(y), "%s: misaligned buffers", name);
  PrepParams p{x,       nullptr, nullptr, nullptr, gamma, scale, shift, row_map, nullptr, nullptr, nullptr, nullptr,
               y,       k,       epsilon, norm == M5K_NORM_LAYER ? 1 : 0, round_to_input ? 1 : 0};
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return norm_by_param<M5K_BF16>(param_dtype, p, rows, st);
    case M5K_F16: return norm_by_param<M5K_F16>(param_dtype, p, rows, st);
    default: return norm_by_param<M5K_F32>(param_dtype, p, rows, st);
  }
}

extern "C" int m5k_gated_residual_add(const void* residual, int dtype, int64_t rows, int64_t k, const void* branch,
                                      const void* gate, int gate_dtype, const int32_t* gate_row_map, void* out,
                                      void* stream) {
  clear_error();
  const char* name = "m5k_gated_residual_add";
  if (int rc = check_common(residual, dtype, rows, k, gate_dtype, name)) return rc;
  M5K_REQUIRE(branch && gate && out, "%s: null pointer", name);
  M5K_REQUIRE(a16(residual) && a16(branch) && a16(gate) && a16(out), "%s: misaligned buffers", name);
  PrepParams p{residual, branch, gate, gate_row_map, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
               out,      nullptr, k,   1.0f,         0,       0};
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case M5K_BF16: return gate_by_param<M5K_BF16>(gate_dtype, p, rows, st);
    case M5K_F16: return gate_by_param<M5K_F16>(gate_dtype, p, rows, st);
    default: return gate_by_param<M5K_F32>(gate_dtype, p, rows, st);
  }
}
