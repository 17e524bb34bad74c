// Fused row preparation for the W8A8 projection (one dispatch per activation matrix):
//
//   [gated]  r = R(float(X) + float(Branch) * float(Gate[g + j]))   -> written once as R_next
//   stats    RMS: var = sum(r^2)/K            LayerNorm: mean = sum(r)/K, var = sum((r-mean)^2)/K
//            inv = 1 / sqrt(var + eps)         (IEEE division and square root)
//   modulate y = O(((r - mean) * inv * gamma[j]) * (1 + scale[t + j]) + shift[t + j])
// The squares are accumulated and the last multiply-add of the modulation is evaluated as
// fused multiply-adds (one rounding each), the contraction the reference's Metal build
// applies by default; the reference pins these stages only to +-1 code.
//   rotate   z = blockdiag(H_B) (y * signs)   (natural-order Sylvester, FP32, * 1/sqrt(B))
//   quantize s = max|z| / 127 (1 if 0); q = clamp(rint_even(z / s), -127, 127)
//
// Contract: norm_hadamard.py:122-265 with the arithmetic of shaders/norm_hadamard.metal:19-118
// (R/O are the residual dtype and the round_output dtype; t and g are row-map table offsets).
// The staged comparators gated_residual_add (gated_residual.metal) and norm_modulate
// (norm_modulate.metal) run the same per-element arithmetic and the same reduction tree, so
// staged rotate(quantize(...)) reproduces the fused codes bit for bit (blocks <= 512).
//
// Layout: one workgroup of 4 wave64 per row.  A lane owns NCH chunks of EPC consecutive
// elements (chunk c = tid + 256*i) and the whole row stays in VGPRs: HBM traffic is the
// minimum 2K (+2K branch, +2K R_next) + K + 4 bytes per row plus the parameter tables.  At
// K = 4096 a lane holds 16 values, which keeps register use low enough for 7 resident
// workgroups per CU; a one-wave-per-row layout (64 values per lane) measured slower for lack
// of resident waves.  So did variants that decode the column parameters once for several
// rows (two rows per workgroup; or a contiguous range of rows per workgroup with the decoded
// parameters held in VGPRs and the next row prefetched): they execute 10-20% fewer VALU
// instructions per element but keep fewer rows' loads in flight per CU.
#include <cmath>

#include "hadamard_core.h"

namespace m5k {
namespace prep {
namespace {

using hadamard::decode8;
using hadamard::fetch8;
using hadamard::fetch8_at;
using hadamard::Raw8;
using hadamard::Shape;
using hadamard::M5K_PMIX;
using hadamard::Tables;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct PrepParams {
  const void* x;          // residual or X [rows, k] (XDT)
  const void* branch;     // [rows, k] (BDT) or null: ungated
  const void* gate;       // [k] or [P, k] (dt_gate)
  const int32_t* gate_map;
  const void* gamma;      // [k] (dt_gamma)
  const void* scale;      // [k] or [P, k] (dt_scale)
  const void* shift;      // [k] or [P, k] (dt_shift)
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
  float inv_k;            // 1/K when K is a power of two (exact), else 0
  // Table dtypes (M5K_BF16 / M5K_F16 / M5K_F32), read by the Tables<M5K_PMIX> kernels.
  int dt_gamma, dt_scale, dt_shift, dt_gate;
};

// sum / K for the row statistics: the IEEE quotient, or the same value as a multiply by the
// exact reciprocal when K is a power of two.
__device__ __forceinline__ float div_k(float x, const PrepParams& p) {
  if (p.inv_k != 0.0f) return x * p.inv_k;
  return x / static_cast<float>(p.k);
}

// Round 8 values through dtype DT in place (the O(...) / R(...) cast) and return their
// storage words; BF16 pairs take one v_cvt_pk_bf16_f32 each.
template <int DT>
__device__ __forceinline__ void round8(float (&v)[8], uint32_t (&w)[8 * dtype_bytes<DT>() / 4]) {
  if constexpr (DT == M5K_F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __float_as_uint(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == M5K_BF16) {
        w[i] = f32x2_to_bf16x2(v[2 * i], v[2 * i + 1]);
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      } else {
        const uint32_t lo = f32_to_f16_bits(v[2 * i]), hi = f32_to_f16_bits(v[2 * i + 1]);
        w[i] = lo | (hi << 16);
        v[2 * i] = f16_bits_to_f32(lo);
        v[2 * i + 1] = f16_bits_to_f32(hi);
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ void store_words8(void* base, int64_t e, const uint32_t (&w)[8 * dtype_bytes<DT>() / 4]) {
  uint4* p = reinterpret_cast<uint4*>(static_cast<uint8_t*>(base) + e * dtype_bytes<DT>());
  p[0] = make_uint4(w[0], w[1], w[2], w[3]);
  if constexpr (DT == M5K_F32) p[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// Which lanes own a row and how they reduce.  Chunk c of a row lives on lane c % kLanes.
struct GroupRow {  // one workgroup of 4 wave64 per row
  static constexpr int kLanes = kThreads;
  static constexpr int kRowsPerGroup = 1;
  __device__ static int64_t row() { return blockIdx.x; }
  __device__ static int lane() { return threadIdx.x; }
  __device__ static float sum(float v, float* red) { return block_sum<kWaves>(v, red); }
};

// Row input for 8 elements at column j: X, or the gated residual update rounded to the
// residual dtype and written to R_next (FP32 product, then add, then one cast).
template <int XDT, int PDT, bool GATED, int BDT = XDT>
__device__ __forceinline__ void load_input8(const PrepParams& p, int64_t row, int64_t goff, int64_t j,
                                            float (&v)[8]) {
  const int64_t e = row * p.k + j;
  load8<XDT>(p.x, e, v);
  if constexpr (GATED) {
    float b[8], g[8];
    load8<BDT>(p.branch, e, b);
    Tables<PDT>::load(p.gate, goff + j, p.dt_gate, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] + b[i] * g[i];
    uint32_t w[8 * dtype_bytes<XDT>() / 4];
    round8<XDT>(v, w);
    store_words8<XDT>(p.r_next, e, w);
  }
}

// Row statistics over the register-resident row.  LayerNorm centres v in place (v - mean,
// the reference's first modulation term, computed once); RMS leaves v as is.  Returns
// inv = 1 / sqrt(var + eps).  Reduction tree: lane partials in chunk order, then the
// layout's reduction (wave xor-butterfly; for GroupRow the 4 wave sums in order).  Chunks
// past the row hold zeros and are re-zeroed after centring.
template <class L, int NV, bool VAR_ONLY = false>
__device__ __forceinline__ float row_stats(float (&v)[NV], const bool (&live)[NV / 8], bool full,
                                           const PrepParams& p, float* red) {
  const int layer = p.layer;
  float first = 0.0f;
  if (layer) {
#pragma unroll
    for (int i = 0; i < NV; ++i) first += v[i];
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i) first = __builtin_fmaf(v[i], v[i], first);
  }
  first = div_k(L::sum(first, red), p);  // slot 0
  float var = first;
  if (layer) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] -= first;
    if (!full) {  // uniform: only rows with lanes past the last chunk
#pragma unroll
      for (int c = 0; c < NV / 8; ++c) {
        if (!live[c]) {
#pragma unroll
          for (int r = 0; r < 8; ++r) v[8 * c + r] = 0.0f;
        }
      }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) acc = __builtin_fmaf(v[i], v[i], acc);
    var = div_k(L::sum(acc, red + kWaves), p);  // slot 1
  }
  if constexpr (VAR_ONLY) return var;
  return 1.0f / sqrtf(var + p.eps);
}

// R_next's 8 values at column col, written with streaming stores (the row is not read back).
template <int DT>
__device__ __forceinline__ void store_words8_at(uint8_t* row_base, uint32_t col,
                                                const uint32_t (&w)[8 * dtype_bytes<DT>() / 4]) {
  uint8_t* q = row_base + col * static_cast<uint32_t>(dtype_bytes<DT>());
  store_stream16(q, make_uint4(w[0], w[1], w[2], w[3]));
  if constexpr (DT == M5K_F32) store_stream16(q + 16, make_uint4(w[4], w[5], w[6], w[7]));
}

// Fused kernel: one row per workgroup of 4 wave64, NCH chunks of EPC elements per lane
// (chunk c = tid + 256 i); FULL when every chunk of every lane lies in the row.  Every global load of the row (X, branch, gate, gamma, scale, shift,
// signs) is issued up front, so a row waits for memory once.  BDT is the branch dtype (any of
// BF16, FP16, FP32, read as is); PDT the parameter tables' (Tables).
//
// The signs fold into gamma and shift as sign-bit flips of their words:
// fma((c * inv) * (g * s), 1 + sc, sh * s) = s * fma((c * inv) * g, 1 + sc, sh) for s = +-1,
// since negation commutes with every rounding (and with the O cast); only the sign of a zero
// result can differ, and no code or scale depends on it (the butterflies, the row peak and the
// encode treat +0 and -0 alike).  Signs are +-1 and enter as their sign bits.  The 1/sqrt(B)
// multiply moves into the encode (FoldedI8).
template <int XDT, int PDT, int B, int NCH, bool GATED, int BDT, bool FULL>
__global__ __launch_bounds__(kThreads) void fused_prep_kernel(PrepParams p, int64_t rows) {
  __shared__ float red[3 * kWaves];  // one slot per block reduction
  __shared__ float row_consts[4];    // inverse, then scale and bracket multipliers (wave 0's)
  __shared__ int row_exact;
  constexpr int EPC = Shape<B>::EPC;
  constexpr int NV = NCH * EPC;
  constexpr int N8 = NV / 8;  // 8-element groups per lane
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t nchunks = p.k / EPC;
  const bool full = FULL || nchunks == static_cast<int64_t>(NCH) * kThreads;
  const int64_t toff = p.row_map ? static_cast<int64_t>(p.row_map[row]) * p.k : 0;
  const int64_t goff = GATED && p.gate_map ? static_cast<int64_t>(p.gate_map[row]) * p.k : 0;
  uint32_t col[N8];  // first column of each 8-element group
  bool live[N8];
#pragma unroll
  for (int g = 0; g < N8; ++g) {
    const int64_t c = lane + static_cast<int64_t>(g / (EPC / 8)) * kThreads;
    col[g] = static_cast<uint32_t>(c * EPC + 8 * (g % (EPC / 8)));
    live[g] = FULL || c < nchunks;
  }
  const uint8_t* xrow = static_cast<const uint8_t*>(p.x) + row * p.k * dtype_bytes<XDT>();
  Raw8<XDT> xr[N8];
  Raw8<BDT> br[GATED ? N8 : 1];
  using T = Tables<PDT>;
  typename T::raw gr[GATED ? N8 : 1], gam[N8], scl[N8], shf[N8];
  uint2 sgn[N8];
#pragma unroll
  for (int g = 0; g < N8; ++g) {
    if (live[g]) {
      xr[g] = fetch8_at<XDT>(xrow, col[g]);
      if constexpr (GATED) {
        br[g] = fetch8_at<BDT>(static_cast<const uint8_t*>(p.branch) + row * p.k * dtype_bytes<BDT>(), col[g]);
        gr[g] = T::fetch(p.gate, goff + col[g], p.dt_gate);
      }
      gam[g] = T::fetch(p.gamma, col[g], p.dt_gamma);
      scl[g] = T::fetch(p.scale, toff + col[g], p.dt_scale);
      shf[g] = T::fetch(p.shift, toff + col[g], p.dt_shift);
      sgn[g] = *reinterpret_cast<const uint2*>(p.signs + col[g]);
    }
  }
  // Row values: X, or the gated residual update (FP32 product, then add, one cast to the
  // residual dtype, written once as R_next).
  float v[NV];
#pragma unroll
  for (int g = 0; g < N8; ++g) {
    float t[8];
    if (live[g]) {
      decode8<XDT>(xr[g], t);
      if constexpr (GATED) {
        float b[8], gt[8];
        decode8<BDT>(br[g], b);
        T::decode(gr[g], p.dt_gate, gt);
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = t[i] + b[i] * gt[i];
        uint32_t w[8 * dtype_bytes<XDT>() / 4];
        round8<XDT>(t, w);
        store_words8_at<XDT>(static_cast<uint8_t*>(p.r_next) + row * p.k * dtype_bytes<XDT>(), col[g], w);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[8 * g + i] = t[i];
  }
  // The row's scalar chains (the square root and division of the inverse, later the scale and
  // bracket of the encoder) run on wave 0 alone and reach the other waves through the LDS.
  const float var = row_stats<GroupRow, NV, true>(v, live, full, p, red);
  if (wave == 0) {
    const float iv = 1.0f / sqrtf(var + p.eps);
    if (lane == 0) row_consts[0] = iv;
  }
  __syncthreads();
  const float inv = row_consts[0];
  // Modulation with the signs folded in, then the unscaled butterflies and the row peak:
  // t = O(fma((c * inv) * gs, 1 + sc, hs)), gs and hs the sign-flipped gamma and shift.
  float peak = 0.0f;
#pragma unroll
  for (int ci = 0; ci < NCH; ++ci) {
    float z[EPC];
#pragma unroll
    for (int h = 0; h < EPC / 8; ++h) {
      const int g = ci * (EPC / 8) + h;
      float t[8];
      if (live[g]) {
        float gs[8], sc[8], hs[8];
        T::decode(T::sign(gam[g], sgn[g], p.dt_gamma), p.dt_gamma, gs);
        T::decode(scl[g], p.dt_scale, sc);
        T::decode(T::sign(shf[g], sgn[g], p.dt_shift), p.dt_shift, hs);
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = __builtin_fmaf(v[8 * g + i] * inv * gs[i], 1.0f + sc[i], hs[i]);
        if (p.round_input) {
          uint32_t w[8 * dtype_bytes<XDT>() / 4];
          round8<XDT>(t, w);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) z[8 * h + i] = t[i];
    }
    hadamard::butterflies<B, false>(z);
#pragma unroll
    for (int r = 0; r < EPC; ++r) {
      v[ci * EPC + r] = z[r];
      peak = fmaxf(peak, fabsf(z[r]));
    }
  }
  {
    const float wmax = wave_max(peak);
    if ((lane & 63) == 0) red[2 * kWaves + wave] = wmax;  // slot 2
  }
  __syncthreads();
  if (wave == 0) {
    float r = red[2 * kWaves];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = fmaxf(r, red[2 * kWaves + w]);
    const hadamard::FoldedI8<B> e(r);
    if (lane == 0) {
      row_consts[1] = e.scale;
      row_consts[2] = e.bracket.lo;
      row_consts[3] = e.bracket.hi;
      row_exact = e.bracket.exact ? 1 : 0;
      p.scales[row] = e.scale;
    }
  }
  __syncthreads();
  const hadamard::FoldedI8<B> enc(row_consts[1], I8Bracket{row_consts[2], row_consts[3], row_exact != 0});
  int8_t* qrow = p.q + row * p.k;
#pragma unroll
  for (int g = 0; g < N8; ++g) {
    if (live[g]) {
      float t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = v[8 * g + i];
      uint32_t w[2];
      enc.template encode<8>(t, w);
      *reinterpret_cast<uint2*>(qrow + col[g]) = make_uint2(w[0], w[1]);
    }
  }
}

// Modulation of 8 centred values at column j, as in fused_prep_kernel:
// fma((c * inv) * gamma, 1 + scale, shift).
template <int PDT>
__device__ __forceinline__ void modulate8(const PrepParams& p, int64_t toff, int64_t j, float inv, float (&v)[8]) {
  float g[8], sc[8], sh[8];
  Tables<PDT>::load(p.gamma, j, p.dt_gamma, g);
  Tables<PDT>::load(p.scale, toff + j, p.dt_scale, sc);
  Tables<PDT>::load(p.shift, toff + j, p.dt_shift, sh);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(v[i] * inv * g[i], 1.0f + sc[i], sh[i]);
}

// Staged norm + modulation (norm_modulate.metal): the fused kernel's chunking (EPC = 8),
// layout and reduction tree, output in the round dtype.
template <class L, int XDT, int PDT, int NCH>
__global__ __launch_bounds__(kThreads) void norm_modulate_kernel(PrepParams p, int64_t rows) {
  __shared__ float red[2 * kWaves];  // one slot per block reduction
  constexpr int NV = NCH * 8;
  const int64_t row = L::row();
  const int lane = L::lane();
  const int64_t nchunks = p.k / 8;
  const int64_t toff = p.row_map ? static_cast<int64_t>(p.row_map[row]) * p.k : 0;
  float v[NV];
  bool live[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = lane + static_cast<int64_t>(i) * L::kLanes;
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
  const float inv = row_stats<L, NV>(v, live, nchunks == static_cast<int64_t>(NCH) * L::kLanes, p, red);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = lane + static_cast<int64_t>(i) * L::kLanes;
    if (c < nchunks) {
      float t[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) t[r] = v[8 * i + r];
      modulate8<PDT>(p, toff, c * 8, inv, t);
      if (p.round_input) {
        uint32_t w[8 * dtype_bytes<XDT>() / 4];
        round8<XDT>(t, w);
        store_words8<XDT>(p.y, row * p.k + c * 8, w);
      } else {
        uint32_t w[8];
        round8<M5K_F32>(t, w);
        store_words8<M5K_F32>(p.y, row * p.k + c * 8, w);
      }
    }
  }
}

// Staged gated residual add (gated_residual.metal): 8 elements per thread, branch dtype BDT.
template <int XDT, int PDT, int BDT>
__global__ __launch_bounds__(kThreads) void gated_residual_kernel(PrepParams p, int64_t total_chunks) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= total_chunks) return;
  const int64_t e = c * 8;
  const int64_t row = e / p.k, j = e - row * p.k;
  const int64_t goff = p.gate_map ? static_cast<int64_t>(p.gate_map[row]) * p.k : 0;
  float v[8];
  load_input8<XDT, PDT, true, BDT>(p, row, goff, j, v);  // writes R_next
}

template <int XDT, int PDT, int B, int NCH, bool GATED, int BDT>
int launch_prep(const PrepParams& p, int64_t rows, hipStream_t st) {
  // Rows that fill every lane's chunks (K = NCH * 256 * EPC, e.g. K 4096 at B <= 512) take the
  // FULL variant, whose lanes carry no liveness tests or zeroed stand-ins: 3-4% faster at
  // M 4096 / 9914, K 4096 (identical outputs).  FP32 residuals, and branches of another dtype
  // than the residual, keep the general kernel only.
  const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
  if constexpr (XDT != M5K_F32 && BDT == XDT) {
    if (p.k == static_cast<int64_t>(NCH) * kThreads * Shape<B>::EPC) {
      fused_prep_kernel<XDT, PDT, B, NCH, GATED, BDT, true><<<grid, block, 0, st>>>(p, rows);
      return launch_status("m5k_norm_hadamard_quantize");
    }
  }
  fused_prep_kernel<XDT, PDT, B, NCH, GATED, BDT, false><<<grid, block, 0, st>>>(p, rows);
  return launch_status("m5k_norm_hadamard_quantize");
}

template <int XDT, int PDT, int B, bool GATED, int BDT>
int launch_fused(const PrepParams& p, int64_t rows, hipStream_t st) {
  constexpr int EPC = Shape<B>::EPC;
  const int64_t per_thread = (p.k / EPC + kThreads - 1) / kThreads;
  if (per_thread <= 1) return launch_prep<XDT, PDT, B, 1, GATED, BDT>(p, rows, st);
  if (per_thread <= 2) return launch_prep<XDT, PDT, B, 2, GATED, BDT>(p, rows, st);
  if (per_thread <= 3) return launch_prep<XDT, PDT, B, 3, GATED, BDT>(p, rows, st);
  if (per_thread <= 4) return launch_prep<XDT, PDT, B, 4, GATED, BDT>(p, rows, st);
  if (per_thread <= 8) return launch_prep<XDT, PDT, B, 8, GATED, BDT>(p, rows, st);
  set_error("m5k_norm_hadamard_quantize: K=%lld exceeds the register-resident row limit %d", (long long)p.k,
            8 * kThreads * EPC);
  return M5K_EINVAL;
}

template <int XDT, int PDT, bool GATED, int BDT = XDT>
int fused_by_block(int block, const PrepParams& p, int64_t rows, hipStream_t st) {
  switch (block) {
    case 32: return launch_fused<XDT, PDT, 32, GATED, BDT>(p, rows, st);
    case 64: return launch_fused<XDT, PDT, 64, GATED, BDT>(p, rows, st);
    case 128: return launch_fused<XDT, PDT, 128, GATED, BDT>(p, rows, st);
    case 256: return launch_fused<XDT, PDT, 256, GATED, BDT>(p, rows, st);
    case 512: return launch_fused<XDT, PDT, 512, GATED, BDT>(p, rows, st);
    case 1024: return launch_fused<XDT, PDT, 1024, GATED, BDT>(p, rows, st);
    default: set_error("m5k_norm_hadamard_quantize: unsupported block %d", block); return M5K_EINVAL;
  }
}

// branch_dtype is BF16, FP16 or FP32 (checked by the entry point), read as is.
template <int XDT, int PDT>
int fused_dispatch(int block, int branch_dtype, const PrepParams& p, int64_t rows, hipStream_t st) {
  if (!p.branch) return fused_by_block<XDT, PDT, false>(block, p, rows, st);
  if (branch_dtype == XDT) return fused_by_block<XDT, PDT, true>(block, p, rows, st);
  switch (branch_dtype) {
    case M5K_BF16: return fused_by_block<XDT, PDT, true, M5K_BF16>(block, p, rows, st);
    case M5K_F16: return fused_by_block<XDT, PDT, true, M5K_F16>(block, p, rows, st);
    default: return fused_by_block<XDT, PDT, true, M5K_F32>(block, p, rows, st);
  }
}

// Every table BF16: the compile-time BF16 kernels; otherwise each table in its own dtype.
template <int XDT>
int fused_by_param(bool all_bf16, int block, int branch_dtype, const PrepParams& p, int64_t rows, hipStream_t st) {
  return all_bf16 ? fused_dispatch<XDT, M5K_BF16>(block, branch_dtype, p, rows, st)
                  : fused_dispatch<XDT, M5K_PMIX>(block, branch_dtype, p, rows, st);
}

template <int XDT, int PDT>
int launch_norm(const PrepParams& p, int64_t rows, hipStream_t st) {
  const dim3 block(kThreads);
  const int64_t per_thread = (p.k / 8 + kThreads - 1) / kThreads;
  const dim3 grid(static_cast<unsigned>(rows));
  if (per_thread <= 1) norm_modulate_kernel<GroupRow, XDT, PDT, 1><<<grid, block, 0, st>>>(p, rows);
  else if (per_thread <= 2) norm_modulate_kernel<GroupRow, XDT, PDT, 2><<<grid, block, 0, st>>>(p, rows);
  else if (per_thread <= 3) norm_modulate_kernel<GroupRow, XDT, PDT, 3><<<grid, block, 0, st>>>(p, rows);
  else if (per_thread <= 4) norm_modulate_kernel<GroupRow, XDT, PDT, 4><<<grid, block, 0, st>>>(p, rows);
  else if (per_thread <= 8) norm_modulate_kernel<GroupRow, XDT, PDT, 8><<<grid, block, 0, st>>>(p, rows);
  else {
    set_error("m5k_norm_modulate: K=%lld exceeds the register-resident row limit %d", (long long)p.k, 8 * kThreads * 8);
    return M5K_EINVAL;
  }
  return launch_status("m5k_norm_modulate");
}

template <int XDT>
int norm_by_param(bool all_bf16, const PrepParams& p, int64_t rows, hipStream_t st) {
  return all_bf16 ? launch_norm<XDT, M5K_BF16>(p, rows, st) : launch_norm<XDT, M5K_PMIX>(p, rows, st);
}

template <int XDT, int PDT, int BDT>
int launch_gate(const PrepParams& p, int64_t rows, hipStream_t st) {
  const int64_t chunks = rows * p.k / 8;
  const int64_t blocks = (chunks + kThreads - 1) / kThreads;
  M5K_REQUIRE(blocks <= 0x7FFFFFFF, "m5k_gated_residual_add: input too large");
  gated_residual_kernel<XDT, PDT, BDT><<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st>>>(p, chunks);
  return launch_status("m5k_gated_residual_add");
}

template <int XDT, int BDT>
int gate_by_param(bool bf16_gate, const PrepParams& p, int64_t rows, hipStream_t st) {
  return bf16_gate ? launch_gate<XDT, M5K_BF16, BDT>(p, rows, st) : launch_gate<XDT, M5K_PMIX, BDT>(p, rows, st);
}

// branch_dtype is BF16, FP16 or FP32 (checked by the entry point), read as is.
template <int XDT>
int gate_by_branch(bool bf16_gate, int branch_dtype, const PrepParams& p, int64_t rows, hipStream_t st) {
  switch (branch_dtype) {
    case M5K_BF16: return gate_by_param<XDT, M5K_BF16>(bf16_gate, p, rows, st);
    case M5K_F16: return gate_by_param<XDT, M5K_F16>(bf16_gate, p, rows, st);
    default: return gate_by_param<XDT, M5K_F32>(bf16_gate, p, rows, st);
  }
}

bool a16(const void* ptr) { return ptr == nullptr || aligned16(ptr); }

// 1/K for a power-of-two K (exactly representable), else 0.
float exact_inv_k(int64_t k) {
  return (k & (k - 1)) == 0 ? std::ldexp(1.0f, -__builtin_ctzll(static_cast<unsigned long long>(k))) : 0.0f;
}

bool float_code(int dt) { return dt == M5K_BF16 || dt == M5K_F16 || dt == M5K_F32; }

// The tables' dtypes from a param_dtype argument: one float code for every table, or
// M5K_PARAM_TABLES(gamma, scale, shift, gate).  all_bf16 selects the compile-time BF16 kernels.
int unpack_param_dtypes(int param_dtype, PrepParams& p, bool& all_bf16, const char* name) {
  if (float_code(param_dtype)) {
    p.dt_gamma = p.dt_scale = p.dt_shift = p.dt_gate = param_dtype;
  } else {
    M5K_REQUIRE((param_dtype & ~0x1FF) == 0 && (param_dtype & M5K_PARAM_PER_TABLE) != 0,
                "%s: parameter dtype %d is neither a float dtype code nor M5K_PARAM_TABLES(...)", name, param_dtype);
    p.dt_gamma = param_dtype & 3;
    p.dt_scale = (param_dtype >> 2) & 3;
    p.dt_shift = (param_dtype >> 4) & 3;
    p.dt_gate = (param_dtype >> 6) & 3;
    M5K_REQUIRE(float_code(p.dt_gamma) && float_code(p.dt_scale) && float_code(p.dt_shift) && float_code(p.dt_gate),
                "%s: M5K_PARAM_TABLES fields must be float dtype codes (got 0x%x)", name, param_dtype);
  }
  all_bf16 = p.dt_gamma == M5K_BF16 && p.dt_scale == M5K_BF16 && p.dt_shift == M5K_BF16 && p.dt_gate == M5K_BF16;
  return M5K_OK;
}

int check_common(const void* x, int x_dtype, int64_t rows, int64_t k, const char* name) {
  M5K_REQUIRE(x, "%s: null input", name);
  M5K_REQUIRE(rows > 0 && k > 0 && rows <= 0x7FFFFFFF, "%s: bad shape [%lld,%lld]", name, (long long)rows,
              (long long)k);
  M5K_REQUIRE(k % 8 == 0, "%s: K=%lld must be a multiple of 8", name, (long long)k);
  M5K_REQUIRE(x_dtype == M5K_BF16 || x_dtype == M5K_F16 || x_dtype == M5K_F32, "%s: unsupported input dtype %d",
              name, x_dtype);
  return M5K_OK;
}

}  // namespace
}  // namespace prep
}  // namespace m5k

using namespace m5k;
using namespace m5k::prep;

extern "C" int m5k_norm_hadamard_quantize(const void* x, int x_dtype, int64_t rows, int64_t k, const void* branch,
                                          int branch_dtype, const void* gate, const int32_t* gate_row_map,
                                          const void* gamma,
                                          const void* scale, const void* shift, int param_dtype,
                                          const int32_t* row_map, const int8_t* signs, int block, int norm,
                                          float epsilon, int round_to_input, int8_t* q, float* scales,
                                          void* residual_out, void* stream) {
  clear_error();
  const char* name = "m5k_norm_hadamard_quantize";
  if (int rc = check_common(x, x_dtype, rows, k, name)) return rc;
  M5K_REQUIRE(gamma && scale && shift && signs && q && scales, "%s: null pointer", name);
  M5K_REQUIRE(block >= 32 && block <= 1024 && (block & (block - 1)) == 0 && k % block == 0,
              "%s: block %d must be a power of two in [32,1024] dividing K", name, block);
  M5K_REQUIRE(!branch || (gate && residual_out), "%s: gated prep needs gate and residual_out", name);
  M5K_REQUIRE(!branch || float_code(branch_dtype), "%s: branch dtype %d must be BF16, F16 or F32", name,
              branch_dtype);
  M5K_REQUIRE(epsilon > 0.0f, "%s: epsilon must be positive", name);
  M5K_REQUIRE(a16(x) && a16(branch) && a16(gate) && a16(gamma) && a16(scale) && a16(shift) && a16(residual_out) &&
                  (reinterpret_cast<uintptr_t>(signs) & 7u) == 0 && (reinterpret_cast<uintptr_t>(q) & 7u) == 0,
              "%s: misaligned buffers", name);
  PrepParams p{x,     branch, gate, gate_row_map, gamma,  scale, shift, row_map, signs, q, scales, residual_out,
               nullptr, k, epsilon, norm == M5K_NORM_LAYER ? 1 : 0, round_to_input ? 1 : 0, exact_inv_k(k)};
  bool all_bf16 = false;
  if (int rc = unpack_param_dtypes(param_dtype, p, all_bf16, name)) return rc;
  if (!branch) all_bf16 = p.dt_gamma == M5K_BF16 && p.dt_scale == M5K_BF16 && p.dt_shift == M5K_BF16;
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return fused_by_param<M5K_BF16>(all_bf16, block, branch_dtype, p, rows, st);
    case M5K_F16: return fused_by_param<M5K_F16>(all_bf16, block, branch_dtype, p, rows, st);
    default: return fused_by_param<M5K_F32>(all_bf16, block, branch_dtype, p, rows, st);
  }
}

extern "C" int m5k_norm_modulate(const void* x, int x_dtype, int64_t rows, int64_t k, const void* gamma,
                                 const void* scale, const void* shift, int param_dtype, const int32_t* row_map,
                                 int norm, float epsilon, int round_to_input, void* y, void* stream) {
  clear_error();
  const char* name = "m5k_norm_modulate";
  if (int rc = check_common(x, x_dtype, rows, k, name)) return rc;
  M5K_REQUIRE(gamma && scale && shift && y, "%s: null pointer", name);
  M5K_REQUIRE(epsilon > 0.0f, "%s: epsilon must be positive", name);
  M5K_REQUIRE(a16(x) && a16(gamma) && a16(scale) && a16(shift) && a16(y), "%s: misaligned buffers", name);
  PrepParams p{x, nullptr, nullptr, nullptr, gamma,   scale, shift, row_map, nullptr, nullptr, nullptr, nullptr,
               y, k,       epsilon, norm == M5K_NORM_LAYER ? 1 : 0, round_to_input ? 1 : 0, exact_inv_k(k)};
  bool all_bf16 = false;
  if (int rc = unpack_param_dtypes(param_dtype, p, all_bf16, name)) return rc;
  all_bf16 = p.dt_gamma == M5K_BF16 && p.dt_scale == M5K_BF16 && p.dt_shift == M5K_BF16;  // no gate here
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case M5K_BF16: return norm_by_param<M5K_BF16>(all_bf16, p, rows, st);
    case M5K_F16: return norm_by_param<M5K_F16>(all_bf16, p, rows, st);
    default: return norm_by_param<M5K_F32>(all_bf16, p, rows, st);
  }
}

extern "C" int m5k_gated_residual_add(const void* residual, int dtype, int64_t rows, int64_t k, const void* branch,
                                      int branch_dtype, const void* gate, int gate_dtype,
                                      const int32_t* gate_row_map, void* out, void* stream) {
  clear_error();
  const char* name = "m5k_gated_residual_add";
  if (int rc = check_common(residual, dtype, rows, k, name)) return rc;
  M5K_REQUIRE(branch && gate && out, "%s: null pointer", name);
  M5K_REQUIRE(float_code(branch_dtype), "%s: branch dtype %d must be BF16, F16 or F32", name, branch_dtype);
  M5K_REQUIRE(float_code(gate_dtype), "%s: gate dtype %d must be BF16, F16 or F32", name, gate_dtype);
  M5K_REQUIRE(a16(residual) && a16(branch) && a16(gate) && a16(out), "%s: misaligned buffers", name);
  PrepParams p{residual, branch, gate, gate_row_map, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
               out,      nullptr, k,   1.0f,         0,       0};
  p.dt_gamma = p.dt_scale = p.dt_shift = p.dt_gate = gate_dtype;
  hipStream_t st = as_stream(stream);
  const bool bf16_gate = gate_dtype == M5K_BF16;
  switch (dtype) {
    case M5K_BF16: return gate_by_branch<M5K_BF16>(bf16_gate, branch_dtype, p, rows, st);
    case M5K_F16: return gate_by_branch<M5K_F16>(bf16_gate, branch_dtype, p, rows, st);
    default: return gate_by_branch<M5K_F32>(bf16_gate, branch_dtype, p, rows, st);
  }
}
