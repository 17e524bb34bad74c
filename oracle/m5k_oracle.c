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
 * Block Hadamard in FP32 (hadamard.metal:6-26 stage order; hadamard_reference.py:103-145
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
