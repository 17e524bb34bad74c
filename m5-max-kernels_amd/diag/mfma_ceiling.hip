// MFMA throughput ceiling on a GEMM's own operand codes (diagnostic library libm5k_diag.so; not
// part of the C ABI in include/m5k.h and not used by any op).
//
// The kernel issues the W8A8 GEMM main loop's matrix instructions with nothing else in the loop:
// every workgroup takes one 256 x 256 output tile of an [m, n] GEMM, 8 wave64 in the GEMM's 2 x 4
// grid (128 x 64 per wave, two waves per SIMD), reads its A and W fragments once from the real
// operand codes (two K slices, far apart in K) into registers, then runs `iters` x 2 x 8 x 4
// v_mfma_i32_16x16x64_i8 (or 2 x 2 x 4 x 2 x 2 v_mfma_i32_32x32x32_i8 of the same K bytes) back to
// back.  With iters = K / 128 it performs the GEMM's MFMA count on data with the GEMM's value
// distribution, so its duration bounds what the matrix cores deliver at the clock the chip holds
// on that data.  `constant` replaces every code with 1 (the low-power case).  The one-wave form
// (md = 4) runs the same MFMA stream as 4 waves, one per SIMD, each doing the work of two: it
// measures what a single wave's back-to-back 16 x 16 x 64 MFMAs can issue.  Both forms are
// compiled for two waves per SIMD (at most 256 VGPRs), so each loop holds its MFMAs and nothing
// else.  (Compiled for one wave per SIMD, the one-wave loop gained 192 accumulator moves per 64
// MFMAs.)  The one-wave form is launched with 96 KiB of dynamic LDS that it never touches, so that
// a CU (160 KiB) holds one of its workgroups.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <int MD, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void mfma_ceiling_kernel(const int8_t* __restrict__ A,
                                                              const int8_t* __restrict__ B, int tiles_n,
                                                              int64_t kb, int iters, int constant,
                                                              int32_t* __restrict__ out) {
  constexpr int WM = 128, WN = 64;
  constexpr int FM = WM / MD, FN = WN / MD;
  constexpr int KPER = MD == 16 ? 64 : 32;  // K bytes of one MFMA
  constexpr int SLICES = 128 / KPER;        // the K bytes of one 128-byte GEMM stage
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave % 8) / 4, wn = wave % 4;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int r_in = lane % MD, chunk = lane / MD;
  v4i a[SLICES][FM], b[SLICES][FN];
#pragma unroll
  for (int s = 0; s < SLICES; ++s) {
    // Slices spread over K (16-byte aligned, inside the row).
    const int64_t kofs = static_cast<int64_t>(s) * (kb / SLICES / KPER) * KPER + 16 * chunk;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int64_t row = static_cast<int64_t>(tm) * 256 + wm * WM + MD * i + r_in;
      a[s][i] = constant ? v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101}
                         : *reinterpret_cast<const v4i*>(A + row * kb + kofs);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t row = static_cast<int64_t>(tn) * 256 + wn * WN + MD * j + r_in;
      b[s][j] = constant ? v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101}
                         : *reinterpret_cast<const v4i*>(B + row * kb + kofs);
    }
  }
  using acc_t = typename std::conditional<MD == 16, v4i, v16i>::type;
  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{};
  for (int it = 0; it < iters * (8 / WAVES); ++it) {
#pragma unroll
    for (int s = 0; s < SLICES; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if constexpr (MD == 16)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[s][i], b[s][j], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][i], b[s][j], acc[i][j], 0, 0, 0);
        }
  }
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < (MD == 16 ? 4 : 16); ++e) sum += acc[i][j][e];
  out[static_cast<int64_t>(blockIdx.x) * 512 + threadIdx.x] = sum;
}

}  // namespace

// m, n multiples of 256; kb >= 128 a multiple of 16; out holds (m / 256) * (n / 256) * 512 int32.
// md: 16 (v_mfma_i32_16x16x64_i8), 32 (v_mfma_i32_32x32x32_i8) or 4 (16 x 16 x 64 on one wave per
// SIMD).  Returns 0 or a HIP error code (1 for invalid arguments).
extern "C" int m5k_diag_mfma_ceiling(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t kb, int iters,
                                     int constant, int md, int32_t* out, void* stream) {
  if (!a || !b || !out || m <= 0 || n <= 0 || m % 256 || n % 256 || kb < 128 || kb % 16 || iters < 0 ||
      (md != 16 && md != 32 && md != 4) || (m / 256) * (n / 256) > 0x7FFFFFFF)
    return 1;
  const int tiles_n = static_cast<int>(n / 256);
  const dim3 grid(static_cast<unsigned>((m / 256) * tiles_n)), block(512);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (md == 16) mfma_ceiling_kernel<16, 8><<<grid, block, 0, st>>>(a, b, tiles_n, kb, iters, constant, out);
  else if (md == 32) mfma_ceiling_kernel<32, 8><<<grid, block, 0, st>>>(a, b, tiles_n, kb, iters, constant, out);
  else mfma_ceiling_kernel<16, 4><<<grid, dim3(256), 96 * 1024, st>>>(a, b, tiles_n, kb, iters, constant, out);
  return static_cast<int>(hipGetLastError());
}
