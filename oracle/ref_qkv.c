/*
 * ref_qkv.c -- exports the reference's own float64 grouped Q/K/V reference for tests.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile (target `ref`) into
 * oracle/_ref/libqkv_ref.so from the header where it lies in the reference checkout
 * (integrations/h3/qkv_reference.h, passed as QKV_REFERENCE); nothing of it is copied here.
 * Only tests/ load the library, to check the FP32 restatement in m5k_oracle.c.
 */
#include <stdint.h>

#include QKV_REFERENCE

#define EXPORT __attribute__((visibility("default")))

/* qvr_postprocess over `rows` head vectors: projection [rows,128] (float64), stream 0/1/2
 * (Q/K/V), gamma [128] BF16 bits, cosine/sine [rows,48] BF16 bits; output [rows,128]. */
EXPORT void ref_qkv_postprocess(const double* projection, int64_t rows, unsigned stream, const uint16_t* gamma,
                                const uint16_t* cosine, const uint16_t* sine, double epsilon, double* output) {
  for (int64_t r = 0; r < rows; ++r)
    qvr_postprocess(projection + r * 128, stream, gamma, cosine + r * 48, sine + r * 48, epsilon, output + r * 128);
}

/* qvr_h256 on a copy-in/copy-out row block of `width` floats (width % 256 == 0). */
EXPORT void ref_qkv_h256(float* values, unsigned width) { qvr_h256(values, width); }
