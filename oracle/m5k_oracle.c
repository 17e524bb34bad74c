/*
 * m5k_oracle.c -- CPU restatement of the reference's quantized-projection arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load liboracle.so.  The
 * product path (libm5k.so through m5kernels_amd) never calls it and has no CPU fallback.
 *
 * Built with -ffp-contract=off: every FP32 expression below rounds exactly as written.
 * Each function cites the reference definition it restates (paths relative to the
 * reference repository).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------------------
 * BF16 / FP16 boundaries
 * ------------------------------------------------------------------------------------- */

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* FP32 -> BF16 nearest-even on the FP32 producer: qk_rope_reference.py:37-42
 * (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000. */
EXPORT uint16_t oracle_bf16_bits(float f) {
  uint32_t u = f32_bits(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }
static inline float bf16_round(float f) { return bf16_to_f32(oracle_bf16_bits(f)); }

EXPORT void oracle_bf16_round_array(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_bits(x[i]);
}

/* ---------------------------------------------------------------------------------------
 * FP8 E4M3 (OCP "fn"): numerics.py:6-26
 * ------------------------------------------------------------------------------------- */

/* numerics.fp8_decode (numerics.py:6-14). */
EXPORT float oracle_fp8_decode(uint8_t q) {
  const float sign = (q & 128) ? -1.0f : 1.0f;
  const int e = (q >> 3) & 15, m = q & 7;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) return sign * (float)m * 0x1p-9f;
  return sign * (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
}

static float g_fp8_table[127];
static int g_fp8_ready = 0;

static void fp8_table_init(void) {
  if (g_fp8_ready) return;
  for (int c = 0; c < 127; ++c) g_fp8_table[c] = oracle_fp8_decode((uint8_t)c);
  g_fp8_ready = 1;
}

/* numerics.fp8_encode (numerics.py:17-26): nearest over the 127 positive finite codes,
 * ties to the even code index, |x| saturated to 448, sign bit from signbit(x). */
EXPORT uint8_t oracle_fp8_encode(float x) {
  fp8_table_init();
  float a = fabsf(x);
  if (a > 448.0f) a = 448.0f;
  /* searchsorted(table, a, side='left'): first index with table[i] >= a */
  int lo_i = 0, hi_i = 127;
  while (lo_i < hi_i) {
    const int mid = (lo_i + hi_i) / 2;
    if (g_fp8_table[mid] < a) lo_i = mid + 1;
    else hi_i = mid;
  }
  int hi = lo_i < 126 ? lo_i : 126;
  int lo = hi - 1 > 0 ? hi - 1 : 0;
  const float dl = a - g_fp8_table[lo];
  const float dh = g_fp8_table[hi] - a;
  const int chosen = (dl < dh || (dl == dh && (lo % 2) == 0)) ? lo : hi;
  return (uint8_t)(chosen | (signbit(x) ? 128 : 0));
}

/* ---------------------------------------------------------------------------------------
 * Per-row quantizer: numerics.quantize_reference (numerics.py:29-46), FP32 semantics.
 * peak = max|x| (float32); scale = peak == 0 ? 1 : peak / 127 (or 448); z = x / scale;
 * int8 q = clip(rint(z), -127, 127) (round half to even); fp8 q = fp8_encode(z).
 * ------------------------------------------------------------------------------------- */
EXPORT void oracle_quantize_rows(const float* x, int64_t rows, int64_t k, int mode, uint8_t* q, float* scales) {
  fp8_table_init(); /* before the threads start */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * k;
    float peak = 0.0f;
    for (int64_t j = 0; j < k; ++j) {
      const float a = fabsf(xr[j]);
      if (a > peak) peak = a;
    }
    const float scale = peak == 0.0f ? 1.0f : peak / (mode == 1 ? 448.0f : 127.0f);
    scales[r] = scale;
    for (int64_t j = 0; j < k; ++j) {
      const float z = xr[j] / scale;
      if (mode == 1) {
        q[r * k + j] = oracle_fp8_encode(z);
      } else {
        float c = nearbyintf(z); /* default rounding mode: nearest, ties to even */
        if (c > 127.0f) c = 127.0f;
        if (c < -127.0f) c = -127.0f;
        q[r * k + j] = (uint8_t)(int8_t)c;
      }
    }
  }
}

/* Same quantizer on BF16 storage (decoded exactly to FP32 first). */
EXPORT void oracle_quantize_rows_bf16(const uint16_t* x, int64_t rows, int64_t k, int mode, uint8_t* q,
                                      float* scales) {
  fp8_table_init();
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * k;
    float peak = 0.0f;
    for (int64_t j = 0; j < k; ++j) {
      const float a = fabsf(bf16_to_f32(xr[j]));
      if (a > peak) peak = a;
    }
    const float scale = peak == 0.0f ? 1.0f : peak / (mode == 1 ? 448.0f : 127.0f);
    scales[r] = scale;
    for (int64_t j = 0; j < k; ++j) {
      const float z = bf16_to_f32(xr[j]) / scale;
      if (mode == 1) {
        q[r * k + j] = oracle_fp8_encode(z);
      } else {
        float c = nearbyintf(z);
        if (c > 127.0f) c = 127.0f;
        if (c < -127.0f) c = -127.0f;
        q[r * k + j] = (uint8_t)(int8_t)c;
      }
    }
  }
}

/* ---------------------------------------------------------------------------------------
 * W8A8 GEMM: exact integer dot (engine.py:173-175 decoded reference is its float64
 * image), and the FP32 epilogue of metal.py:88-128.
 * ------------------------------------------------------------------------------------- */

/* acc[m,n] = sum_k a[m,k] * b[n,k], exact in int64, stored as int32 (|acc| <= 127^2 K). */
EXPORT void oracle_gemm_i8_acc(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k, int32_t* acc) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t i = 0; i < m; ++i) {
    const int8_t* ar = a + i * k;
    for (int64_t j = 0; j < n; ++j) {
      const int8_t* br = b + j * k;
      int64_t s = 0;
      for (int64_t t = 0; t < k; ++t) s += (int32_t)ar[t] * (int32_t)br[t];
      acc[i * n + j] = (int32_t)s;
    }
  }
}

/* Epilogue value before the output cast: (float(acc) * sa[m]) * sb[n] [+ bias].
 * metal.py:96 (left-to-right FP32 products) and :108-113 (bias before the cast). */
static inline float i8_epilogue_value(int32_t acc, float sa, float sb, const float* bias, const int32_t* bias_map,
                                      int64_t i, int64_t j, int64_t n) {
  float v = ((float)acc * sa) * sb;
  if (bias) v = v + bias[(bias_map ? (int64_t)bias_map[i] * n : 0) + j];
  return v;
}

/* out_kind: 0 = FP32 values, 2 = BF16 bits (uint16).  Optional gated residual
 * (metal.py:114-128): branch = bf16(value); out = bf16(float(res) + branch * gate). */
EXPORT void oracle_i8_epilogue(const int32_t* acc, const float* sa, const float* sb, int64_t m, int64_t n,
                               const float* bias, const int32_t* bias_map, const uint16_t* residual,
                               const uint16_t* gate, const int32_t* gate_map, int out_kind, void* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      float v = i8_epilogue_value(acc[i * n + j], sa[i], sb[j], bias, bias_map, i, j, n);
      if (residual) {
        const float branch = bf16_round(v);
        const float g = bf16_to_f32(gate[(gate_map ? (int64_t)gate_map[i] * n : 0) + j]);
        v = bf16_to_f32(residual[i * n + j]) + branch * g;
      }
      if (out_kind == 2) ((uint16_t*)out)[i * n + j] = oracle_bf16_bits(v);
      else ((float*)out)[i * n + j] = v;
    }
  }
}

/* The whole W8A8 online linear on the CPU (the timed CPU baseline):
 * quantize bf16 A per row -> exact int GEMM against prequantized W -> FP32 epilogue -> BF16. */
EXPORT void oracle_w8a8_linear_bf16(const uint16_t* a_bf16, const int8_t* wq, const float* wscale, int64_t m,
                                    int64_t n, int64_t k, int8_t* aq_scratch, float* ascale_scratch,
                                    uint16_t* out) {
  oracle_quantize_rows_bf16(a_bf16, m, k, 0, (uint8_t*)aq_scratch, ascale_scratch);
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t i = 0; i < m; ++i) {
    const int8_t* ar = aq_scratch + i * k;
    for (int64_t j = 0; j < n; ++j) {
      const int8_t* br = wq + j * k;
      int32_t s = 0; /* |s| <= 127*127*K fits int32 for K <= 133144 */
      for (int64_t t = 0; t < k; ++t) s += (int32_t)ar[t] * (int32_t)br[t];
      out[i * n + j] = oracle_bf16_bits(((float)s * ascale_scratch[i]) * wscale[j]);
    }
  }
}

/* ---------------------------------------------------------------------------------------
 * Block Hadamard in FP32 (hadamard.metal:6-26 stage order; hadamard_reference.py:26-68
 * defines the transform): v = x * sign; natural-order Sylvester stages s = 1, 2, .., B/2
 * with (a, b) -> (a + b, a - b); then one multiply by (float)(1 / sqrt(B)).
 * ------------------------------------------------------------------------------------- */
EXPORT float oracle_inv_sqrt_block(int block) { return (float)(1.0 / sqrt((double)block)); }

EXPORT void oracle_hadamard_f32(const float* x, int64_t rows, int64_t k, int block, const int8_t* signs, float* y) {
  const float inv = oracle_inv_sqrt_block(block);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float* yr = y + r * k;
    for (int64_t j = 0; j < k; ++j) yr[j] = x[r * k + j] * (float)signs[j];
    for (int64_t b0 = 0; b0 < k; b0 += block) {
      float* v = yr + b0;
      for (int s = 1; s < block; s <<= 1)
        for (int base = 0; base < block; base += 2 * s)
          for (int t = 0; t < s; ++t) {
            const float p = v[base + t], q = v[base + t + s];
            v[base + t] = p + q;
            v[base + t + s] = p - q;
          }
      for (int t = 0; t < block; ++t) v[t] = v[t] * inv;
    }
  }
}

/* Array forms used by the Python side. */
EXPORT void oracle_fp8_encode_array(const float* x, int64_t n, uint8_t* out) {
  fp8_table_init();
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_encode(x[i]);
}

EXPORT void oracle_fp8_decode_array(const uint8_t* q, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_decode(q[i]);
}

/* ---------------------------------------------------------------------------------------
 * Fixed-order FP32 restatements of the fused prep and the Q/K epilogue.
 *
 * The reference fixes these stages by formula (norm_hadamard_reference.py:24-94,
 * gated_residual_reference.py:21-60, qk_rope_reference.py:45-134, float64) and its GPU tests
 * hold the Metal kernels to +-1 code (tests/test_norm_hadamard_metal.py:33-82).  The functions
 * below state one FP32 evaluation of the same formulas completely -- every product, sum,
 * fused multiply-add, reduction tree and rounding boundary -- so that a GPU kernel that
 * evaluates the formulas in exactly this order can be compared bit for bit.  The order:
 *
 *   row sums over K   256 lanes; lane t owns chunks c = t, t + 256, ... of `epc` consecutive
 *                     elements and accumulates its elements in order (x^2 terms as fmaf);
 *                     each 64-lane wave then reduces by the DPP tree of wave_tree_sum and the
 *                     four wave sums add in wave order.
 *   statistics        RMS: var = S(x^2) / K.  LayerNorm: mean = S(x) / K, c = x - mean,
 *                     var = S(c^2) / K.  inv = 1 / sqrtf(var + eps) (IEEE sqrt and division).
 *   modulation        y = fmaf((c * inv) * gamma, 1 + scale, shift), then the O cast.
 *   gated update      r = R(x + branch * gate): FP32 product, FP32 sum, one cast.
 *   rotation, codes   oracle_hadamard_f32 and the INT8 row quantizer above.
 * ------------------------------------------------------------------------------------- */

/* FP32 -> FP16 -> FP32, round to nearest even (binary16: 10 fraction bits, normals from 2^-14,
 * subnormal quantum 2^-24, overflow to infinity from 65520). */
EXPORT float oracle_f16_round(float f) {
  if (isnan(f) || isinf(f)) return f;
  const double a = fabs((double)f);
  if (a >= 65520.0) return signbit(f) ? -INFINITY : INFINITY;
  double quantum;
  if (a < 0x1p-14) {
    quantum = 0x1p-24;
  } else {
    int e;
    frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    quantum = ldexp(1.0, e - 11);
  }
  const double r = nearbyint(a / quantum) * quantum; /* a / quantum is exact: a power-of-two scale */
  return (float)(signbit(f) ? -r : r);
}

EXPORT void oracle_f16_round_array(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_round(x[i]);
}

/* dtype codes of the library: 0 F32, 1 F16, 2 BF16. */
static inline float round_dtype(float v, int dt) {
  return dt == 2 ? bf16_round(v) : dt == 1 ? oracle_f16_round(v) : v;
}

/* The 64-lane DPP sum of the library's wave reduction: xor 1, xor 2 (quad_perm), lane i <- 7 - i
 * within each half row, lane i <- 15 - i within each row, then row 1 += lane 15 and row 3 +=
 * lane 47 (row_bcast15, rows 0 and 2 add 0), rows 2 and 3 += lane 31 (row_bcast31, rows 0 and 1
 * add 0); the result is lane 63.  Every step reads the lanes' values before the step. */
static float wave_tree_sum(const float* lanes) {
  float v[64], t[64];
  memcpy(v, lanes, sizeof(v));
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ 1];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ 2];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[(l & ~7) | (7 - (l & 7))];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[(l & ~15) | (15 - (l & 15))];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 64; ++l) {
    const int row = l >> 4;
    t[l] = v[l] + ((row & 1) ? v[(row - 1) * 16 + 15] : 0.0f);
  }
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 64; ++l) t[l] = v[l] + ((l >> 4) >= 2 ? v[31] : 0.0f);
  return t[63];
}

/* Sum of the 256 lane partials of a row: four wave trees, added in wave order. */
static float row_tree_sum(const float* partial) {
  float r = wave_tree_sum(partial);
  for (int w = 1; w < 4; ++w) r += wave_tree_sum(partial + 64 * w);
  return r;
}

/* Lane partials of one row in the lane/chunk order stated above: squares as fmaf when
 * `square`, plain sums otherwise. */
static void lane_partials(const float* v, int64_t k, int epc, int square, float* partial) {
  const int64_t chunks = k / epc;
  for (int t = 0; t < 256; ++t) {
    float acc = 0.0f;
    for (int64_t c = t; c < chunks; c += 256)
      for (int e = 0; e < epc; ++e) {
        const float x = v[c * epc + e];
        acc = square ? fmaf(x, x, acc) : acc + x;
      }
    partial[t] = acc;
  }
}

/* Fused row preparation (norm_hadamard.py:122-265 restated in the fixed FP32 order above).
 *   x [rows,k] values of dtype xdt (decoded to FP32); branch [rows,k] (FP32 values) or NULL;
 *   gate [k] or [P,k] selected by gate_map; gamma [k]; scale/shift [k] or [P,k] selected by
 *   row_map; signs [k]; epc: elements per lane chunk (the kernel's max(8, block / 64)).
 *   Outputs: codes q, scales s, r_next [rows,k] (FP32 values of the R cast) when gated, and
 *   optionally `modulated` [rows,k], the FP32 modulation before the O cast. */
EXPORT void oracle_prep_rows(const float* x, int xdt, const float* branch, const float* gate,
                             const int32_t* gate_map, const float* gamma, const float* scale, const float* shift,
                             const int32_t* row_map, const int8_t* signs, int64_t rows, int64_t k, int block,
                             int epc, int layer, float eps, int round_input, int8_t* q, float* s, float* r_next,
                             float* modulated) {
  const float kf = (float)k;
#pragma omp parallel
  {
    float* v = (float*)malloc((size_t)k * sizeof(float));
    float* y = (float*)malloc((size_t)k * sizeof(float));
    float partial[256];
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const float* xr = x + r * k;
      if (branch) {
        const float* gr = gate + (gate_map ? (int64_t)gate_map[r] * k : 0);
        for (int64_t j = 0; j < k; ++j) {
          const float prod = branch[r * k + j] * gr[j];
          v[j] = round_dtype(xr[j] + prod, xdt);
          r_next[r * k + j] = v[j];
        }
      } else {
        memcpy(v, xr, (size_t)k * sizeof(float));
      }
      float var;
      if (layer) {
        lane_partials(v, k, epc, 0, partial);
        const float mean = row_tree_sum(partial) / kf;
        for (int64_t j = 0; j < k; ++j) v[j] = v[j] - mean;
        lane_partials(v, k, epc, 1, partial);
        var = row_tree_sum(partial) / kf;
      } else {
        lane_partials(v, k, epc, 1, partial);
        var = row_tree_sum(partial) / kf;
      }
      const float inv = 1.0f / sqrtf(var + eps);
      const int64_t toff = row_map ? (int64_t)row_map[r] * k : 0;
      for (int64_t j = 0; j < k; ++j) {
        float t = fmaf((v[j] * inv) * gamma[j], 1.0f + scale[toff + j], shift[toff + j]);
        if (modulated) modulated[r * k + j] = t;
        if (round_input) t = round_dtype(t, xdt);
        y[j] = t;
      }
      oracle_hadamard_f32(y, 1, k, block, signs, v);
      oracle_quantize_rows(v, 1, k, 0, (uint8_t*)(q + r * k), s + r);
    }
    free(v);
    free(y);
  }
}

/* The 16-lane row sum of the Q/K epilogue: xor 1, xor 2, lane i <- 7 - i, lane i <- 15 - i. */
static float group16_tree_sum(const float* lanes) {
  float v[16], t[16];
  memcpy(v, lanes, sizeof(v));
  for (int l = 0; l < 16; ++l) t[l] = v[l] + v[l ^ 1];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 16; ++l) t[l] = v[l] + v[l ^ 2];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 16; ++l) t[l] = v[l] + v[(l & ~7) | (7 - (l & 7))];
  memcpy(v, t, sizeof(v));
  for (int l = 0; l < 16; ++l) t[l] = v[l] + v[15 - l];
  return t[0];
}

/* RMSNorm + split-half RoPE of one head of 128 BF16 projection values (qk_rope_reference.py:
 * 45-134 in the fixed FP32 order): lane g of 16 sums z^2 over channels 8g..8g+7 in order,
 * group16_tree_sum; inv = 1 / sqrtf(S / 128 + eps); u = (z * inv) * gamma;
 * d < R: u[d] c[d] - u[d+R] s[d]; R <= d < 2R: u[d] c[d-R] + u[d-R] s[d-R]; else u[d]; BF16. */
static void qk_head(const uint16_t* z, const uint16_t* gamma, const uint16_t* c, const uint16_t* s, int R, float eps,
                    uint16_t* y) {
  float zf[128], u[128], partial[16];
  for (int d = 0; d < 128; ++d) zf[d] = bf16_to_f32(z[d]);
  for (int g = 0; g < 16; ++g) {
    float acc = 0.0f;
    for (int t = 0; t < 8; ++t) acc = acc + zf[8 * g + t] * zf[8 * g + t];
    partial[g] = acc;
  }
  const float inv = 1.0f / sqrtf(group16_tree_sum(partial) / 128.0f + eps);
  for (int d = 0; d < 128; ++d) u[d] = (zf[d] * inv) * bf16_to_f32(gamma[d]);
  for (int d = 0; d < 128; ++d) {
    float out = u[d];
    if (d < R) out = (u[d] * bf16_to_f32(c[d])) - (u[d + R] * bf16_to_f32(s[d]));
    else if (d < 2 * R) out = (u[d] * bf16_to_f32(c[d - R])) + (u[d - R] * bf16_to_f32(s[d - R]));
    y[d] = oracle_bf16_bits(out);
  }
}

/* Q or K epilogue over a BF16 projection z [m, n] (n % 128 == 0): head-major y [n/128, m, 128]. */
EXPORT void oracle_qk_norm_rope(const uint16_t* z, int64_t m, int64_t n, const uint16_t* gamma, const uint16_t* cosv,
                                const uint16_t* sinv, int rope_half, float eps, uint16_t* y) {
  const int64_t heads = n / 128;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < m; ++r)
    for (int64_t h = 0; h < heads; ++h)
      qk_head(z + r * n + h * 128, gamma, cosv + r * rope_half, sinv + r * rope_half, rope_half, eps,
              y + (h * m + r) * 128);
}

/* Grouped Q/K/V (the H3 runtime's [head, stream, 128] weight rows, integrations/h3/
 * qkv_reference.h:15-35): block b of the projection z [m, heads * 384] is head b / 3, stream
 * b % 3; Q and K take their own gamma and the epilogue above, V is the BF16 projection. */
EXPORT void oracle_qkv_norm_rope(const uint16_t* z, int64_t m, int64_t heads, const uint16_t* q_gamma,
                                 const uint16_t* k_gamma, const uint16_t* cosv, const uint16_t* sinv, int rope_half,
                                 float eps, uint16_t* q_out, uint16_t* k_out, uint16_t* v_out) {
  const int64_t n = heads * 384;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < m; ++r)
    for (int64_t b = 0; b < 3 * heads; ++b) {
      const int64_t head = b / 3, stream = b % 3;
      const uint16_t* zb = z + r * n + b * 128;
      uint16_t* dst = (stream == 0 ? q_out : stream == 1 ? k_out : v_out) + (head * m + r) * 128;
      if (stream == 2) memcpy(dst, zb, 128 * sizeof(uint16_t));
      else qk_head(zb, stream == 0 ? q_gamma : k_gamma, cosv + r * rope_half, sinv + r * rope_half, rope_half, eps, dst);
    }
}
