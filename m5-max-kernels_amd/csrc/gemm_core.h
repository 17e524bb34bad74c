// MFMA GEMM main loop for gfx950: C[M,N] = A[M,K] . B[N,K]^T with both operands
// K-contiguous ("NT", the reference's weight layout [N,K], metal.py:72-73).
//
// Workgroup tile 256 x 256, 4 wave64 in a 2 x 2 grid, each wave owning a 128 x 128
// sub-tile as 4 x 4 blocks of 32 x 32 MFMA accumulators (256 accumulator registers,
// allocated by the compiler into AGPR/VGPR).  K advances 128 bytes per stage; a stage is
// A[256 x 128 B] + B[256 x 128 B] = 64 KiB of LDS, double-buffered (128 KiB of the
// 160 KiB per CU).  LDS rows are 128 B with the 16-byte chunk index XOR-swizzled by
// (row & 7), so the 32 lanes reading one MFMA fragment column hit distinct banks.
//
// MFMA operand layout (32 x 32 blocks): lane l supplies row (l & 31) and a 16-byte
// (32-byte for FP8) slice of K selected by (l >> 5).  A and B use the same K-slice
// mapping, so the products pair up correctly whatever order the hardware sums them in
// (exact for INT32 accumulation).  Accumulator register r of lane l holds
// C[(r >> 2) * 8 + (l >> 5) * 4 + (r & 3)][l & 31].
#pragma once

#include "m5k_common.h"

namespace m5k {
namespace gemm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

enum Mode { I8 = 0, F8 = 1, BF16 = 2, F16 = 3 };

constexpr int BM = 256;   // tile rows (A rows / C rows)
constexpr int BN = 256;   // tile cols (B rows / C cols)
constexpr int BKB = 128;  // K bytes per stage
constexpr int THREADS = 256;
constexpr int WM = 128, WN = 128;  // wave sub-tile
constexpr int FM = WM / 32, FN = WN / 32;
constexpr int STAGE_BYTES = BM * BKB;  // one operand, one stage
constexpr int GROUP_M = 4;             // tile-rows per raster band

template <int MODE>
struct Traits {
  using acc_t = v16f;
  static constexpr int elem_bytes = 2;
  static constexpr int sub_steps = BKB / 32;  // 32 K-bytes per MFMA
};
template <>
struct Traits<I8> {
  using acc_t = v16i;
  static constexpr int elem_bytes = 1;
  static constexpr int sub_steps = BKB / 32;
};
template <>
struct Traits<F8> {
  using acc_t = v16f;
  static constexpr int elem_bytes = 1;
  static constexpr int sub_steps = BKB / 64;  // 64 K-bytes per MFMA
};

// Operand fragment for one MFMA: 16 bytes (I8/BF16/F16) or 32 bytes (F8).
template <int MODE>
struct Frag {
  v4i lo;
  v4i hi;  // F8 only
};

template <int MODE>
__device__ __forceinline__ void mfma(typename Traits<MODE>::acc_t& acc, const Frag<MODE>& a,
                                     const Frag<MODE>& b) {
  if constexpr (MODE == I8) {
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.lo, b.lo, acc, 0, 0, 0);
  } else if constexpr (MODE == BF16) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a.lo),
                                                  __builtin_bit_cast(bf16x8, b.lo), acc, 0, 0, 0);
  } else if constexpr (MODE == F16) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a.lo),
                                                 __builtin_bit_cast(f16x8, b.lo), acc, 0, 0, 0);
  } else {
    const v8i av = {a.lo[0], a.lo[1], a.lo[2], a.lo[3], a.hi[0], a.hi[1], a.hi[2], a.hi[3]};
    const v8i bv = {b.lo[0], b.lo[1], b.lo[2], b.lo[3], b.hi[0], b.hi[1], b.hi[2], b.hi[3]};
    // Format codes 0/0 = FP8 E4M3 (OCP) for both operands; zero scales select the
    // unscaled instruction.
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, 0, 0, 0, 0, 0, 0);
  }
}

// Tile coordinates for workgroup `bid`.  Workgroups are dispatched round-robin over the
// 8 XCDs (bid % 8); renumber so that each XCD receives a contiguous run of logical tiles,
// then raster the logical order in bands of GROUP_M tile-rows (column-major inside a
// band), so an XCD's concurrent tiles share A rows and B rows in its own L2.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int logical = bid;
  if (total >= 16) {
    const int per = total >> 3, rem = total & 7;
    const int xcd = bid & 7, local = bid >> 3;
    logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
  }
  const int band_size = GROUP_M * tiles_n;
  const int band = logical / band_size;
  const int first = band * GROUP_M;
  const int h = min(GROUP_M, tiles_m - first);
  const int inner = logical - band * band_size;
  tm = first + inner % h;
  tn = inner / h;
}

// Main loop.  ALIGNED: rows are 16-byte multiples and bases 16-byte aligned, so every
// 16-byte chunk is either fully inside K or fully outside.  Otherwise bytes are loaded
// one at a time with exact K bounds (small/odd shapes only).
template <int MODE, bool ALIGNED>
__device__ __forceinline__ void mainloop(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                         int M, int N, int64_t Kb, int tile_m0, int tile_n0,
                                         uint8_t* smem, typename Traits<MODE>::acc_t (&acc)[FM][FN]) {
  using acc_t = typename Traits<MODE>::acc_t;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{};

  // Loader mapping: thread t moves chunk (t & 7) of rows (t >> 3) + 32 * i, i = 0..7.
  const int lc = tid & 7, lr = tid >> 3;
  const int sw_store = ((lr & 7) ^ lc) << 4;  // (row & 7) == (lr & 7) for every i
  const int64_t kt_count = (Kb + BKB - 1) / BKB;

  uint4 ra[8], rb[8];
  auto gload = [&](int64_t kt) {
    const int64_t kb = kt * BKB + lc * 16;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = lr + 32 * i;
      const int am = tile_m0 + r, bn = tile_n0 + r;
      if constexpr (ALIGNED) {
        ra[i] = (am < M && kb < Kb) ? *reinterpret_cast<const uint4*>(A + (int64_t)am * Kb + kb)
                                    : make_uint4(0, 0, 0, 0);
        rb[i] = (bn < N && kb < Kb) ? *reinterpret_cast<const uint4*>(B + (int64_t)bn * Kb + kb)
                                    : make_uint4(0, 0, 0, 0);
      } else {
        uint32_t wa[4] = {0, 0, 0, 0}, wb[4] = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const bool kin = kb + e < Kb;
          const uint32_t va = (am < M && kin) ? A[(int64_t)am * Kb + kb + e] : 0u;
          const uint32_t vb = (bn < N && kin) ? B[(int64_t)bn * Kb + kb + e] : 0u;
          wa[e >> 2] |= va << (8 * (e & 3));
          wb[e >> 2] |= vb << (8 * (e & 3));
        }
        ra[i] = make_uint4(wa[0], wa[1], wa[2], wa[3]);
        rb[i] = make_uint4(wb[0], wb[1], wb[2], wb[3]);
      }
    }
  };
  auto sstore = [&](int stage) {
    uint8_t* sa = smem + stage * 2 * STAGE_BYTES;
    uint8_t* sb = sa + STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int off = (lr + 32 * i) * BKB + sw_store;
      *reinterpret_cast<uint4*>(sa + off) = ra[i];
      *reinterpret_cast<uint4*>(sb + off) = rb[i];
    }
  };

  // Fragment addressing: row (lane & 31) of each 32-row block; swizzle uses row & 7 == lane & 7.
  const int frow = lane & 31, fhalf = lane >> 5, fsw = lane & 7;
  const int a_row0 = wm * WM + frow, b_row0 = wn * WN + frow;

  auto compute = [&](int stage) {
    const uint8_t* sa = smem + stage * 2 * STAGE_BYTES;
    const uint8_t* sb = sa + STAGE_BYTES;
#pragma unroll
    for (int s = 0; s < Traits<MODE>::sub_steps; ++s) {
      Frag<MODE> fa[FM], fb[FN];
      if constexpr (MODE == F8) {
        const int c0 = s * 4 + fhalf * 2;
        const int o0 = ((c0 ^ fsw) << 4), o1 = (((c0 + 1) ^ fsw) << 4);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const uint8_t* p = sa + (a_row0 + 32 * i) * BKB;
          fa[i].lo = *reinterpret_cast<const v4i*>(p + o0);
          fa[i].hi = *reinterpret_cast<const v4i*>(p + o1);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const uint8_t* p = sb + (b_row0 + 32 * j) * BKB;
          fb[j].lo = *reinterpret_cast<const v4i*>(p + o0);
          fb[j].hi = *reinterpret_cast<const v4i*>(p + o1);
        }
      } else {
        const int o = (((s * 2 + fhalf) ^ fsw) << 4);
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i].lo = *reinterpret_cast<const v4i*>(sa + (a_row0 + 32 * i) * BKB + o);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j].lo = *reinterpret_cast<const v4i*>(sb + (b_row0 + 32 * j) * BKB + o);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mfma<MODE>(acc[i][j], fa[i], fb[j]);
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int64_t kt = 0; kt < kt_count; ++kt) {
    const bool more = kt + 1 < kt_count;
    if (more) gload(kt + 1);
    compute(static_cast<int>(kt & 1));
    if (more) sstore(static_cast<int>((kt + 1) & 1));
    __syncthreads();
  }
}

// Visit every accumulator element with its global (row, col).
template <class AccT, class F>
__device__ __forceinline__ void for_each_acc(const AccT (&acc)[FM][FN], int tile_m0, int tile_n0, F&& f) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int col_in = lane & 31, row_half = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = tile_m0 + wm * WM + i * 32 + (r >> 2) * 8 + row_half + (r & 3);
        const int n = tile_n0 + wn * WN + j * 32 + col_in;
        f(m, n, acc[i][j][r]);
      }
}

}  // namespace gemm
}  // namespace m5k
