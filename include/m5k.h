/*
 * m5k.h -- C ABI of libm5k.so, the MI355X (gfx950) quantized-projection hot path.
 *
 * Every entry point takes device pointers to row-major, contiguous buffers,
 * 64-bit sizes and an opaque HIP stream (hipStream_t passed as void*; NULL is
 * the default stream). Launches are asynchronous on that stream. Inputs are
 * never written. The library never allocates device memory: the caller owns
 * every buffer, outputs included.
 *
 * Return value: 0 on success; a nonzero M5K_E* code otherwise, with a
 * human-readable message available from m5k_last_error() on the calling
 * thread. Argument checks here cover only what the kernels rely on for memory
 * safety and launch validity; the Python layer reproduces the reference's
 * ValueError / NotImplementedError contract before calling in.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   quantize                 src/m5kernels/metal.py:27-44 (int8, fp8, mxint8)
 *   gemm                     src/m5kernels/metal.py:158-269
 *   rotate                   src/m5kernels/hadamard.py:33-77
 *   fused_norm_hadamard_quantize
 *                            src/m5kernels/norm_hadamard.py:122-176
 *   fused_gated_residual_norm_hadamard_quantize
 *                            src/m5kernels/norm_hadamard.py:198-265
 *   gated_residual_add       src/m5kernels/norm_hadamard.py:280-300
 *   unfused_norm             src/m5kernels/norm_hadamard.py:321-348
 *   projection_qk_rope       src/m5kernels/qk_rope.py:120-182
 *   qk_norm_rope             src/m5kernels/qk_rope.py:185-203
 *   rms_quantize             src/m5kernels/rms_quant.py:41-117
 *   grouped QKV projection   integrations/h3/qkv_candidate.metal:1-20
 *   shift-split conditioning src/m5kernels/norm_hadamard_gemm.py:233-247,459-460
 */
#ifndef M5K_H
#define M5K_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
#define M5K_F32 0
#define M5K_F16 1
#define M5K_BF16 2
#define M5K_I8 3
#define M5K_U8 4
#define M5K_I32 5

/* Quantization modes. */
#define M5K_QUANT_INT8 0 /* symmetric [-127,127], scale = peak/127 */
#define M5K_QUANT_FP8 1  /* OCP E4M3 codes in uint8, scale = peak/448 */

/* Normalization kinds for the fused prep. */
/* Prep parameter-table dtypes (param_dtype of m5k_norm_hadamard_quantize and m5k_norm_modulate):
 * one float dtype code for every table, or one code per table packed by M5K_PARAM_TABLES (the
 * gate field is ignored by calls without a gate). */
#define M5K_PARAM_PER_TABLE 0x100
#define M5K_PARAM_TABLES(gamma, scale, shift, gate) \
  (M5K_PARAM_PER_TABLE | (gamma) | ((scale) << 2) | ((shift) << 4) | ((gate) << 6))

#define M5K_NORM_RMS 0
#define M5K_NORM_LAYER 1

/* Status codes. */
#define M5K_OK 0
#define M5K_EINVAL 1  /* argument outside what the kernels support */
#define M5K_ELAUNCH 2 /* HIP launch or runtime error */

/* Message for the last failure on this thread ("" if none). */
const char* m5k_last_error(void);

/* ABI version (major*100 + minor). */
int m5k_abi_version(void);

/*
 * Per-row symmetric quantizer.  Replaces metal.quantize(x, mode) for modes
 * "int8" and "fp8" (src/m5kernels/metal.py:27-44, shaders/quantize.metal:1-38).
 * x: [rows,k] of x_dtype (F32/F16/BF16).  q: [rows,k] int8 (INT8) or uint8
 * E4M3 codes (FP8).  scales: [rows] float32.
 * peak = max|x|; scale = peak==0 ? 1 : peak/127 (or /448), IEEE fp32 division;
 * INT8 code = clamp(rint_even(x/scale), -127, 127); FP8 code = nearest E4M3
 * (ties to even, saturating at 448, sign from the sign bit).
 */
int m5k_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int mode,
                      void* q, float* scales, void* stream);

/*
 * MXINT8 block quantizer.  Replaces metal.quantize(x, "mxint8") (src/m5kernels/metal.py:27-44,
 * block mode of shaders/quantize.metal:13-37; spec numerics.py:33-41).  x: [rows,k] F32/F16/BF16
 * with k % 32 == 0.  Per 32-element block: e = 0 for an all-zero block, else
 * clamp(floor(log2(peak)) - 6, -127, 127) with log2 rounded to FP32 before the floor;
 * q = clamp(rint(x / 2^e), -127, 127) int8 [rows,k]; exponents[rows, k/32] = e + 127 (uint8,
 * the E8M0 scale byte of the OCP S1.6 convention with the /64 folded in).
 */
int m5k_quantize_mxint8(const void* x, int x_dtype, int64_t rows, int64_t k, int8_t* q,
                        uint8_t* exponents, void* stream);

/*
 * MXINT8 codes to BF16 values q * 2^(exponent - 127), exact.  Operand expansion for the MXINT8
 * linear (metal.gemm(..., "mxint8", ...), src/m5kernels/metal.py:81-86, plane scales of
 * 32 x 1 blocks): y[rows,k] BF16, 16-byte aligned; q 8-byte aligned; k % 32 == 0.
 */
int m5k_mxint8_to_bf16(const int8_t* q, const uint8_t* exponents, int64_t rows, int64_t k, void* y,
                       void* stream);

/*
 * W8A8 linear.  Replaces metal.gemm(a, b, "int8", ...) (src/m5kernels/metal.py:158-269,
 * epilogues :88-128).  a: [m,k] int8, b: [n,k] int8 (weights, K-contiguous).
 * c[m,n] = O(float(sum_k a*b) * a_scales[m] * b_scales[n] [+ bias]) with int32
 * accumulation and the FP32 products evaluated left to right; O = c_dtype
 * (F32/F16/BF16, round to nearest even).
 * bias (optional, may be NULL): float32 [n], or [P,n] selected by
 *   bias_row_map[m] (int32) when bias_row_map is non-NULL.
 * residual/gate (optional, both or neither; excludes bias; c_dtype must be BF16):
 *   residual bf16 [m,n], gate bf16 [n] or [P,n] with gate_row_map[m];
 *   c = bf16(float(residual) + float(bf16(branch)) * float(gate)).
 */
int m5k_gemm_i8(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                const float* a_scales, const float* b_scales, void* c, int c_dtype,
                const float* bias, const int32_t* bias_row_map,
                const void* residual, const void* gate, const int32_t* gate_row_map,
                void* stream);

/*
 * The same W8A8 linear as m5k_gemm_i8 for short M: each output tile (256 x 256, or 256 x 64
 * (k <= 8192) or 256 x 128 when the tiles x splits fit in one round) is split over `splits`
 * contiguous ranges of K (1..64), the raw INT32 partial tiles go to workspace[splits][m][n]
 * (int32, caller-owned, at least splits*m*n elements), and a second kernel sums them in
 * split order and applies the identical epilogue.  INT32 sums are exact, so c is bit-identical
 * to m5k_gemm_i8's.  Needs k % 16 == 0 and 16-byte aligned a/b (any operand size).  Same
 * contract as metal.gemm(a, b, "int8", ...) (src/m5kernels/metal.py:158-269); the split is
 * this library's schedule for few-tile shapes (one or two 256-row tile rows).
 */
int m5k_gemm_i8_splitk(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                       const float* a_scales, const float* b_scales, void* c, int c_dtype,
                       const float* bias, const int32_t* bias_row_map, const void* residual,
                       const void* gate, const int32_t* gate_row_map, int splits, int32_t* workspace,
                       int64_t workspace_elems, void* stream);

/*
 * m5k_gemm_i8_splitk without the caller's workspace: the INT32 partials go to a scratch array
 * of the library (M5K_SCRATCH_ELEMS int32 = 64 MiB per GPU, a static device array held until
 * the process ends), so the call allocates nothing -- no hipMalloc, no hipFree, no allocating
 * library routine.  No counterpart in the reference: it is for callers that cannot allocate
 * (HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * splits * m * n must not exceed M5K_SCRATCH_ELEMS (M5K_EINVAL otherwise).  The array used is
 * the one on the device of `stream` (the current device for the null stream); its address is
 * looked up once per device, the first call on that device.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, other host threads) race.  Results
 * are bit-identical to m5k_gemm_i8_splitk and m5k_gemm_i8.
 */
#define M5K_SCRATCH_ELEMS (16 * 1024 * 1024)
int m5k_gemm_i8_splitk_noalloc(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                               const float* a_scales, const float* b_scales, void* c, int c_dtype,
                               const float* bias, const int32_t* bias_row_map, const void* residual,
                               const void* gate, const int32_t* gate_row_map, int splits, void* stream);

/*
 * Launch plan of the MFMA GEMMs (host only, launches nothing).  No counterpart in the
 * reference; it lets a host scheduler compose with the library's own choice.  For an
 * [m,n] output with operands of ab_dtype (M5K_I8, M5K_U8 for FP8 codes, M5K_BF16, M5K_F16,
 * M5K_F32) on a device of `cus` compute units, *schedule receives
 *   0  plain: 256 x 256 tiles;
 *   1  mixed: the leading *full_tiles 256 x 256 tiles (whole rounds), every other tile as
 *      two 256 x 128 halves in the same launch;
 *   2  narrow: 256 x 224 tiles (I8 / BF16 / F16 only);
 *   3  quad: 256 x 256 tiles on four waves of 128 x 128 (I8 only; only when forced, below);
 * and *full_tiles is -1 unless the schedule is 1.  Every m5k_gemm_* entry point makes this
 * choice with the device's CU count for operands on the direct-to-LDS path (row bytes a
 * multiple of 16, 16-byte aligned bases); the others run the plain schedule.  Results are
 * bit-identical under every schedule.  M5K_GEMM_MIXED_TILES=0 / M5K_GEMM_NARROW_TILES=0 in
 * the environment switch schedule 1 / 2 off.
 */
int m5k_gemm_launch_plan(int ab_dtype, int64_t m, int64_t n, int cus, int* schedule, int64_t* full_tiles);

/*
 * Force the schedule of the MFMA GEMM launches made by the calling host thread: -1 restores the
 * library's own plan (m5k_gemm_launch_plan), 0 plain, 1 mixed, 2 narrow (plain for FP8/FP32),
 * 3 quad (plain for all but I8; never the library's own choice, as it measured slower).
 * *previous (may be NULL) receives the thread's earlier setting.  No counterpart in the
 * reference, whose tuner searches Metal threadgroup tiles through gemm's `tile` argument
 * (src/m5kernels/cli.py:66-151); this is the gfx950 knob the harness tuner searches instead.
 * The setting is thread-local, so other host threads keep their own plan; for tools outside the
 * process, M5K_GEMM_SCHEDULE=plain|mixed|narrow|quad in the environment does the same when no thread
 * setting is made.  Results are bit-identical under every schedule.
 */
int m5k_gemm_set_schedule(int schedule, int* previous);

/*
 * Raw INT32 accumulators of the W8A8 GEMM (test hook for bit-exact parity):
 * acc[m,n] = sum_k a[m,k]*b[n,k].  Same kernel main loop as m5k_gemm_i8.
 */
int m5k_gemm_i8_acc(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k,
                    int32_t* acc, void* stream);

/*
 * FP8 E4M3 linear with FP32 accumulation.  Replaces metal.gemm(a, b, "fp8", ...)
 * (src/m5kernels/metal.py:75-80,191-194).  a: [m,k], b: [n,k] uint8 E4M3 codes;
 * k % 128 == 0.  c = O(acc * a_scales[m] * b_scales[n]).
 */
int m5k_gemm_f8(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                const float* a_scales, const float* b_scales, void* c, int c_dtype,
                void* stream);

/*
 * Split-K FP8 linear for short M: the same contract as m5k_gemm_f8 (metal.gemm(a, b, "fp8", ...),
 * src/m5kernels/metal.py:75-80,191-194), computed as `splits` K ranges per output tile into
 * FP32 partials workspace[splits][m][n] (workspace_elems >= splits*m*n floats, caller-owned),
 * summed in split order before the scale epilogue.  Deterministic; its FP32 sums may differ
 * from m5k_gemm_f8's in the last bits (FP8 accumulation order is not pinned).  splits in
 * [1, 64]; operands 16-byte aligned.
 */
int m5k_gemm_f8_splitk(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                       const float* a_scales, const float* b_scales, void* c, int c_dtype, int splits,
                       float* workspace, int64_t workspace_elems, void* stream);

/*
 * Floating GEMM with FP32 accumulation.  Replaces metal.gemm(a, b, "bf16"|"fp16", ...)
 * (src/m5kernels/metal.py:59-74,101-107).  a: [m,k], b: [n,k] of ab_dtype (BF16/F16).
 * c = O(acc).  Optional gated residual epilogue as for m5k_gemm_i8 (BF16 only).
 */
int m5k_gemm_float(const void* a, const void* b, int ab_dtype, int64_t m, int64_t n, int64_t k,
                   void* c, int c_dtype, const void* residual, const void* gate,
                   const int32_t* gate_row_map, void* stream);

/*
 * Signed block-Hadamard rotation  Y = (X * signs) H_B, FP32 output.
 * Replaces hadamard.rotate (src/m5kernels/hadamard.py:33-77, shaders/hadamard.metal:1-26).
 * x: [rows,k] of x_dtype, signs: int8 [k] (+-1), block in {32,...,1024}, k % block == 0.
 * Natural-order Sylvester butterflies in FP32, then one multiply by the FP32
 * constant 1/sqrt(block).
 */
int m5k_hadamard_rotate(const void* x, int x_dtype, int64_t rows, int64_t k, int block,
                        const int8_t* signs, float* y, void* stream);

/*
 * Fused rotation + per-row INT8 quantization: the codes and scales of
 * quantize(rotate(x, block, signs), "int8") without materializing the FP32
 * rotation (the online composition of src/m5kernels/hadamard_gemm.py:27-69).
 */
int m5k_hadamard_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int block,
                               const int8_t* signs, int8_t* q, float* scales, void* stream);

/*
 * Fused row preparation (one dispatch): [gated residual update] -> RMS or LayerNorm ->
 * modulation -> O cast -> signs -> block Hadamard -> per-row INT8.
 * Replaces norm_hadamard.fused_norm_hadamard_quantize (branch == NULL) and
 * fused_gated_residual_norm_hadamard_quantize (src/m5kernels/norm_hadamard.py:122-265,
 * shaders/norm_hadamard.metal:1-121).
 *   x: [rows,k] of x_dtype (the residual when gated); k % block == 0.
 *   gated: branch [rows,k] of branch_dtype (BF16, F16 or F32, independent of x_dtype, read as
 *          is), gate [k] or [P,k] with gate_row_map[rows]; residual_out[rows,k] (x_dtype)
 *          receives R(x + branch*gate), written once.  branch_dtype is ignored when branch is
 *          NULL.
 *   gamma [k]; scale/shift [k], or [P,k] tables selected by row_map[rows]; param_dtype gives
 *   the tables' dtypes: one float code for all, or M5K_PARAM_TABLES(gamma, scale, shift,
 *   gate).  signs int8 [k].
 *   norm: M5K_NORM_RMS / M5K_NORM_LAYER; round_to_input: 1 rounds the modulated value to
 *   x_dtype before the signs (round_output="input"), 0 keeps FP32.
 *   Outputs: q int8 [rows,k], scales float32 [rows].
 */
int m5k_norm_hadamard_quantize(const void* x, int x_dtype, int64_t rows, int64_t k, const void* branch,
                               int branch_dtype, const void* gate, const int32_t* gate_row_map,
                               const void* gamma,
                               const void* scale, const void* shift, int param_dtype,
                               const int32_t* row_map, const int8_t* signs, int block, int norm,
                               float epsilon, int round_to_input, int8_t* q, float* scales,
                               void* residual_out, void* stream);

/*
 * Staged norm + modulation with the fused kernel's arithmetic and reduction tree.
 * Replaces norm_hadamard.unfused_norm (src/m5kernels/norm_hadamard.py:321-348,
 * shaders/norm_modulate.metal:1-37).  y: [rows,k] of x_dtype (round_to_input=1) or F32.
 */
int m5k_norm_modulate(const void* x, int x_dtype, int64_t rows, int64_t k, const void* gamma,
                      const void* scale, const void* shift, int param_dtype, const int32_t* row_map,
                      int norm, float epsilon, int round_to_input, void* y, void* stream);

/*
 * Staged gated residual update out = R(float(residual) + float(branch) * float(gate)).
 * Replaces norm_hadamard.gated_residual_add (src/m5kernels/norm_hadamard.py:280-300,
 * shaders/gated_residual.metal:1-9).  gate [k] or [P,k] of gate_dtype with gate_row_map[rows];
 * branch of branch_dtype; both BF16, F16 or F32, independent of the residual dtype.
 */
int m5k_gated_residual_add(const void* residual, int dtype, int64_t rows, int64_t k, const void* branch,
                           int branch_dtype, const void* gate, int gate_dtype, const int32_t* gate_row_map,
                           void* out, void* stream);

/*
 * Q or K projection + per-head RMSNorm + split-half RoPE, head-major BF16 output.
 * Replaces qk_rope.projection_qk_rope (src/m5kernels/qk_rope.py:120-182,
 * shaders/qk_rope_projection.metal:1-39, shaders/qk_rope_body.metal:1-20).
 *   a [m,k], b [n,k] of ab_dtype: M5K_I8 (with float32 a_scales[m], b_scales[n]; k <= 131071)
 *   or M5K_BF16 (scales NULL); n % 128 == 0.  gamma bf16 [128]; cos, sin bf16 [m, rope_half],
 *   0 <= rope_half <= 64.  y bf16 [n/128, m, 128].
 *   z = bf16(projection); inv = 1/sqrt(sum(z^2)/128 + eps); u = z*inv*gamma;
 *   y[d] = u[d]*c - u[d+R]*s (d < R), u[d]*c + u[d-R]*s (R <= d < 2R), u[d] otherwise.
 */
int m5k_projection_qk_rope(const void* a, const void* b, int ab_dtype, int64_t m, int64_t n, int64_t k,
                           const float* a_scales, const float* b_scales, const void* gamma, const void* cos,
                           const void* sin, int rope_half, float epsilon, void* y, void* stream);

/*
 * Staged postprocess of a BF16 [m,n] projection with the fused kernel's per-(row, head) code.
 * Replaces qk_rope.qk_norm_rope (src/m5kernels/qk_rope.py:185-203, shaders/qk_rope_norm.metal).
 */
int m5k_qk_norm_rope(const void* projected, int64_t m, int64_t n, const void* gamma, const void* cos,
                     const void* sin, int rope_half, float epsilon, void* y, void* stream);

/*
 * Grouped Q/K/V projection in the H3 runtime's native layout
 * (integrations/h3/qkv_candidate.metal:5-81, reference math qkv_reference.h:15-35).
 * b: [heads*3*128, k] weight rows ordered [head][stream Q,K,V][channel]; a: [m,k] (INT8
 * with a_scales/b_scales, or BF16).  Every 128-column block is rounded to BF16 as in
 * m5k_projection_qk_rope; Q blocks then take q_gamma and K blocks k_gamma through the same
 * per-head RMSNorm + split-half RoPE (cos/sin [m, rope_half]); V blocks are the rounded
 * projection.  q_out, k_out, v_out: BF16 [heads, m, 128], 16-byte aligned.
 */
int m5k_projection_qkv_rope(const void* a, const void* b, int ab_dtype, int64_t m, int64_t heads,
                            int64_t k, const float* a_scales, const float* b_scales,
                            const void* q_gamma, const void* k_gamma, const void* cos,
                            const void* sin, int rope_half, float epsilon, void* q_out,
                            void* k_out, void* v_out, void* stream);

/*
 * RMS dynamic INT8 quantization with the inverse RMS folded into the row scales.  Replaces
 * rms_quant.rms_quantize (src/m5kernels/rms_quant.py:41-117, shaders/rms_quant.metal:1-97).
 * x: [rows,k] F32/F16/BF16; gamma: FP32 [k]; signs: int8 +-1 [k]; block 1 (no transform, any
 * k) or a power of two in [32,1024] dividing k.  ss = sum x^2, inv = 1/sqrt(ss/k + eps);
 * v = fold ? (x*gamma)*s : ((x*inv)*gamma)*s; z = blockdiag(H_B) v; peak = max|z|;
 * scales[row] = peak == 0 ? 1 : (peak * (fold ? inv : 1)) / 127;
 * q = peak == 0 ? 0 : clamp(rint((z/peak)*127), -127, 127) int8 [rows,k].
 */
int m5k_rms_quantize(const void* x, int x_dtype, int64_t rows, int64_t k, const float* gamma,
                     const int8_t* signs, int block, int fold_scale, float epsilon, int8_t* q,
                     float* scales, void* stream);

/*
 * Conditioning tables of the shift-split projection.  Replaces condition_prepare and
 * bias_prepare of the norm-shift-split backend (src/m5kernels/norm_hadamard_gemm.py:233-247,
 * 459-460).  gamma: [k]; scale, shift: [p_rows,k] (param_dtype and operand_dtype
 * respectively; F32/F16/BF16); w: [n,k] original projection weights (operand_dtype).
 * combined[p,j] = float(gamma[j]) * (1 + float(scale[p,j]))  FP32 [p_rows,k];
 * bias[p,n] = sum_j float(shift[p,j]) * float(w[n,j])       FP32 [p_rows,n] (FP32
 * accumulation; p_rows <= 8 one pass over w, more rows on the MFMA GEMM of m5k_gemm_float).
 * The online projection is m5k_rms_quantize(x, combined[p], fold) followed by m5k_gemm_i8 with
 * bias[p].
 */
int m5k_shift_split_condition(const void* gamma, const void* scale, int param_dtype,
                              const void* shift, const void* w, int operand_dtype, int64_t p_rows,
                              int64_t k, int64_t n, float* combined, float* bias, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* M5K_H */
