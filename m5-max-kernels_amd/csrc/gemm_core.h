// MFMA GEMM main loop for gfx950: C[M,N] = A[M,K] . B[N,K]^T with both operands
// K-contiguous ("NT", the reference's weight layout [N,K], metal.py:72-73).
//
// Workgroup tile 256 x 256 with 8 wave64 in a 2 x 4 grid; each wave owns a 128 x 64
// sub-tile.  K advances 128 bytes (one L2 line of every row) per stage; a stage is
// A[256 x 128 B] + B[256 x 128 B] = 64 KiB of LDS, double-buffered (128 KiB of the 160 KiB
// per CU) and filled by direct global->LDS buffer loads of whole rows issued one stage ahead.
// LDS rows are 128 B with the 16-byte chunk index XOR-swizzled by (row >> 1) & 7 (see swz()).
// Against 64-byte stages in a 4-deep ring (half-line requests, one barrier per 64 bytes) this
// measured 6-10% (INT8) and 12-14% (BF16) faster at K = 16384 and 1-5% faster elsewhere,
// with bit-identical results.
//
// MFMA blocks.  INT8, BF16 and FP16 use 16 x 16 blocks that take 64 bytes of K per
// instruction (v_mfma_i32_16x16x64_i8, v_mfma_f32_16x16x32_{bf16,f16}): 8 x 4 blocks per
// wave, 4 accumulator registers each.  FP8 uses 16 x 16 blocks that take the whole 128-byte
// stage per instruction (v_mfma_scale_f32_16x16x128_f8f6f4).  FP32 (v_mfma_f32_32x32x2_f32)
// uses 32 x 32 blocks: 4 x 2 per wave, 16 registers each.  The 16 x 16 form measured ~5%
// faster than 32 x 32 on the FFN-down and 4096^3 shapes with the same LDS traffic and MFMA
// cycles per slab (INT8); for FP8, 16 x 16 x 128 with its own stage schedule (see
// mainloop_dma) measured 5-7% faster than 32 x 32 x 64 on five shapes, with the same bits.
//
// Operand layout.  16 x 16: lane l supplies row (l & 15) and the 16-byte K chunk (l >> 4)
// of a 64-byte sub-step, or for FP8 the chunks (l >> 4) and 4 + (l >> 4) of the 128-byte
// stage (32 bytes).  32 x 32 (FP32): row (l & 31) and chunk 2s + (l >> 5) of 32-byte
// sub-step s, one K = 2 MFMA per float of the chunk.  A and B use the same K-slice mapping,
// so the products pair up correctly
// whatever order the hardware sums them in (exact for INT32 accumulation).  Accumulator
// register r of lane l holds C[(l >> 4) * 4 + r][l & 15] (16 x 16) or
// C[(r >> 2) * 8 + (l >> 5) * 4 + (r & 3)][l & 31] (32 x 32).
#pragma once

#include <type_traits>

#include "m5k_common.h"

namespace m5k {
namespace gemm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

enum Mode { I8 = 0, F8 = 1, BF16 = 2, F16 = 3, F32 = 4 };

constexpr int BM = 256;   // tile rows (A rows / C rows)
constexpr int BN = 256;   // tile cols (B rows / C cols)
constexpr int BKB = 128;  // K bytes per stage (LDS row length, one L2 line)
constexpr int NST = 2;    // LDS stage buffers
constexpr int STAGE_BYTES = BM * BKB;  // one operand, one stage
constexpr int GROUP_M = 4;             // tile-rows per raster band

// Wave grid of a 256 x 256 tile.  WAVES_M x WAVES_N wave64, each owning a (256/WAVES_M) x
// (256/WAVES_N) sub-tile of MFMA blocks.  2 x 2 = one wave per SIMD with 256 accumulator
// registers; 2 x 4 = two waves per SIMD with 128 each, so one wave's MFMAs keep the pipe busy
// while its sibling waits at a barrier.
// TN is the tile's column count: BN for the full tile, less for the narrower tiles that refill
// a partial last round or make the tile count a whole number of rounds.  B rows are moved in
// whole 16-row groups per wave; rows past TN load nothing (their LDS rows are never read).
template <int WAVES_M_, int WAVES_N_, int TN_ = BN>
struct Grid {
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int WAVES = WAVES_M * WAVES_N;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int TN = TN_;
  static constexpr int WM = BM / WAVES_M, WN = TN / WAVES_N;
  static constexpr int DMA_ROWS = BM / WAVES;       // A rows one wave DMAs per stage
  static constexpr int DMA_INSTR = DMA_ROWS / 8;    // 1 KiB (8 rows of 128 B) per instruction
  static constexpr int DMA_ROWS_B = (TN / WAVES + 15) / 16 * 16;  // B rows one wave DMAs per stage
  static constexpr int DMA_INSTR_B = DMA_ROWS_B / 8;
};
using Grid4 = Grid<2, 2>;
using Grid8 = Grid<2, 4>;
using Grid8Half = Grid<4, 2, BN / 2>;     // 256 x 128 tile, 8 waves of 64 x 64
using Grid8Narrow = Grid<4, 2, 7 * BN / 8>;  // 256 x 224 tile, 8 waves of 64 x 112 (16 x 16 modes)
using Grid8Skinny = Grid<8, 1, BN / 4>;      // 256 x 64 tile, 8 waves of 32 x 64 (split-K of short M)

typedef float v4f __attribute__((ext_vector_type(4)));
template <int MODE>
struct Traits {
  using acc_t = v4f;
  static constexpr int MD = 16;
  static constexpr int elem_bytes = 2;
  static constexpr int sub_steps = BKB / 64;  // 64 K-bytes per 16x16 MFMA
};
template <>
struct Traits<I8> {
  using acc_t = v4i;
  static constexpr int MD = 16;
  static constexpr int elem_bytes = 1;
  static constexpr int sub_steps = BKB / 64;
};
template <>
struct Traits<F32> {
  using acc_t = v16f;
  static constexpr int MD = 32;
  static constexpr int elem_bytes = 4;
  static constexpr int sub_steps = BKB / 32;  // 8 floats of K per sub-step, 4 MFMAs of K = 2
};
template <>
struct Traits<F8> {
  using acc_t = v4f;
  static constexpr int MD = 16;
  static constexpr int elem_bytes = 1;
  static constexpr int sub_steps = BKB / 128;  // 128 K-bytes per 16x16x128 MFMA: one per stage
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
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.lo, b.lo, acc, 0, 0, 0);
  } else if constexpr (MODE == BF16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.lo),
                                                  __builtin_bit_cast(bf16x8, b.lo), acc, 0, 0, 0);
  } else if constexpr (MODE == F16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a.lo),
                                                 __builtin_bit_cast(f16x8, b.lo), acc, 0, 0, 0);
  } else if constexpr (MODE == F32) {
    // A 16-byte fragment holds 4 consecutive floats of K; MFMA j takes float j of every lane,
    // so lanes l and l + 32 contribute K offsets j and 4 + j of the 8-float sub-step.
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__int_as_float(a.lo[j]), __int_as_float(b.lo[j]), acc, 0, 0, 0);
  } else {
    const v8i av = {a.lo[0], a.lo[1], a.lo[2], a.lo[3], a.hi[0], a.hi[1], a.hi[2], a.hi[3]};
    const v8i bv = {b.lo[0], b.lo[1], b.lo[2], b.lo[3], b.hi[0], b.hi[1], b.hi[2], b.hi[3]};
    // Format codes 0/0 = FP8 E4M3 (OCP) for both operands; zero scales select the
    // unscaled instruction.
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 0, 0, 0, 0, 0, 0);
  }
}

// Tile coordinates for workgroup `bid`.  Workgroups are dispatched round-robin over the
// 8 XCDs (bid % 8); renumber so that each XCD receives a contiguous run of logical tiles,
// then raster the logical order in bands of GROUP_M tile-rows (column-major inside a
// band), so an XCD's concurrent tiles share A rows and B rows in its own L2.
__device__ __forceinline__ int xcd_logical(int bid, int total) {
  if (total < 16) return bid;
  const int per = total >> 3, rem = total & 7;
  const int xcd = bid & 7, local = bid >> 3;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
}

__device__ __forceinline__ void band_coords(int logical, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int band_size = GROUP_M * tiles_n;
  const int band = logical / band_size;
  const int first = band * GROUP_M;
  const int h = min(GROUP_M, tiles_m - first);
  const int inner = logical - band * band_size;
  tm = first + inner % h;
  tn = inner / h;
}

__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  band_coords(xcd_logical(bid, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// LDS layout of one operand stage: 256 rows x 128 bytes (one L2 line per row); the 16-byte
// chunk c of row r sits at physical chunk c ^ ((r >> 1) & 7).  gfx950 serves ds_read_b128 16
// lanes at a time over 64 banks (256 B); a fragment read covers 16 consecutive rows with one
// logical chunk, which lands on 16 distinct (row parity, physical chunk) bank groups.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// Row stride (elements) of a 256 x 256 16-bit tile staged in LDS by an epilogue: 528 bytes, so
// the four rows a wave writes per accumulator register (rows 4 apart) land 16 banks apart
// instead of on the same 8 banks, and 16-byte row chunks stay aligned.
constexpr int TILE16_STRIDE = BN + 8;

// All LDS of a GEMM kernel: NST stages x (A, B) x 32 KiB = 128 KiB for the main loop, which uses
// it as the stage ring; epilogues may reuse it afterwards (a 256 x TILE16_STRIDE 16-bit tile,
// 132 KiB, then the tile's row and column scales, 2 KiB).  The DMA writes are inline asm with
// "memory" clobbers and every consumer sits behind an explicit wait and barrier, so one array
// serves all stages.
constexpr int EPI_SCALES_OFFSET = BM * TILE16_STRIDE * 2;
constexpr int EPI_BYTES = EPI_SCALES_OFFSET + (BM + BN) * 4;
constexpr int LDS_BYTES = NST * 2 * STAGE_BYTES > EPI_BYTES ? NST * 2 * STAGE_BYTES : EPI_BYTES;
__shared__ __attribute__((aligned(16))) uint8_t g_lds[LDS_BYTES];

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One 16-byte-per-lane buffer load straight into LDS: lane l's 16 bytes land at
// lds_base + 16 l (M0 holds the wave-uniform LDS base); an offset past num_records loads 0.
// Issued as inline asm so the compiler does not serialize it against LDS reads of other
// stage buffers; every consumer waits with an explicit vmcnt and a barrier instead.  The
// main loop issues no other vector-memory instruction, so those explicit counts are exact.
// lds_base and rsrc are wave-uniform by construction.  UNIFORM states it with readfirstlane, so
// that they stay in SGPRs (the asm's "s" operands) where the compiler cannot prove it (the
// four-wave grid, whose 256 accumulators leave it under register pressure).
template <bool UNIFORM = false>
__device__ __forceinline__ void dma16(uint32_t lds_base, uint32_t voffset, v4i rsrc) {
  if constexpr (UNIFORM) {
    rsrc = v4i{__builtin_amdgcn_readfirstlane(rsrc[0]), __builtin_amdgcn_readfirstlane(rsrc[1]),
               __builtin_amdgcn_readfirstlane(rsrc[2]), __builtin_amdgcn_readfirstlane(rsrc[3])};
    lds_base = __builtin_amdgcn_readfirstlane(lds_base);
  }
  __asm__ volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds_base), "v"(voffset), "s"(rsrc)
      : "memory", "m0");
}

__device__ __forceinline__ v4i buffer_rsrc(const void* base, uint32_t num_records) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  // word1: base[47:32], stride 0; word3: raw (untyped) 32-bit access, the gfx9 default.
  return v4i{static_cast<int>(addr & 0xFFFFFFFFu), static_cast<int>((addr >> 32) & 0xFFFFu),
             static_cast<int>(num_records), 0x00020000};
}

// Wave-uniform buffer window [base + ofs, base + records): the descriptor of one K stage of a
// tile's rows (scalar arithmetic only; ofs <= records).
__device__ __forceinline__ v4i window_rsrc(const uint8_t* base, uint32_t records, uint32_t ofs) {
  return buffer_rsrc(base + ofs, records - ofs);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(const_cast<void*>(p))));
}

// Wait until at most N of this wave's DMA instructions are outstanding (vmcnt counts them
// in issue order).
template <int N>
__device__ __forceinline__ void wait_stage() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the memory fence of __syncthreads(): the fence would wait for
// every outstanding load of this wave, including the DMA of stages still being prefetched.
// Callers wait explicitly (vmcnt for their own stage loads) before calling it.
__device__ __forceinline__ void stage_barrier() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

template <int ST>
__device__ __forceinline__ uint8_t* stage_a() {
  return g_lds + ST * 2 * STAGE_BYTES;
}
template <int ST>
__device__ __forceinline__ uint8_t* stage_b() {
  return g_lds + ST * 2 * STAGE_BYTES + STAGE_BYTES;
}

template <int MODE, class G>
struct Blk {
  static constexpr int MD = Traits<MODE>::MD, FM = G::WM / MD, FN = G::WN / MD;
};

// Fragments of one MFMA sub-step for a wave's FM x FN block grid.
template <int MODE, class G>
struct FragSet {
  Frag<MODE> a[Blk<MODE, G>::FM];
  Frag<MODE> b[Blk<MODE, G>::FN];
};

// Fragments of sub-step s.  16 x 16 blocks: lane l reads row (l & 15) of each block at
// logical chunk 4s + (l >> 4) (64-byte sub-steps).  FP8: row (l & 15), chunks (l >> 4) and
// 4 + (l >> 4) (one 128-byte sub-step, 32 bytes a lane).  FP32: row (l & 31), chunk
// 2s + (l >> 5) (32-byte sub-steps).  `fq` is the lane's chunk term (l >> 4 or l >> 5), `fsw`
// the swizzle of its row, which a block offset of 16 or 32 rows leaves alone.
template <int MODE, class G>
__device__ __forceinline__ void read_frags(const uint8_t* sa, const uint8_t* sb, int s, int a_row0, int b_row0,
                                           int fq, int fsw, FragSet<MODE, G>& f) {
  constexpr int MD = Blk<MODE, G>::MD;
  if constexpr (MODE == F8) {
    const int o0 = (fq ^ fsw) << 4, o1 = ((4 + fq) ^ fsw) << 4;
#pragma unroll
    for (int i = 0; i < Blk<MODE, G>::FM; ++i) {
      const uint8_t* p = sa + (a_row0 + MD * i) * BKB;
      f.a[i].lo = *reinterpret_cast<const v4i*>(p + o0);
      f.a[i].hi = *reinterpret_cast<const v4i*>(p + o1);
    }
#pragma unroll
    for (int j = 0; j < Blk<MODE, G>::FN; ++j) {
      const uint8_t* p = sb + (b_row0 + MD * j) * BKB;
      f.b[j].lo = *reinterpret_cast<const v4i*>(p + o0);
      f.b[j].hi = *reinterpret_cast<const v4i*>(p + o1);
    }
  } else {
    const int o = (((MODE == F32 ? 2 : 4) * s + fq) ^ fsw) << 4;
#pragma unroll
    for (int i = 0; i < Blk<MODE, G>::FM; ++i)
      f.a[i].lo = *reinterpret_cast<const v4i*>(sa + (a_row0 + MD * i) * BKB + o);
#pragma unroll
    for (int j = 0; j < Blk<MODE, G>::FN; ++j)
      f.b[j].lo = *reinterpret_cast<const v4i*>(sb + (b_row0 + MD * j) * BKB + o);
  }
}

template <int MODE, class G>
using AccTile = typename Traits<MODE>::acc_t[Blk<MODE, G>::FM][Blk<MODE, G>::FN];

// MFMAs of block rows [I0, I1) of one fragment set.
template <int MODE, class G, int I0, int I1>
__device__ __forceinline__ void mfma_rows(AccTile<MODE, G>& acc, const FragSet<MODE, G>& f) {
#pragma unroll
  for (int i = I0; i < I1; ++i)
#pragma unroll
    for (int j = 0; j < Blk<MODE, G>::FN; ++j) mfma<MODE>(acc[i][j], f.a[i], f.b[j]);
}

template <int MODE, class G>
__device__ __forceinline__ void zero_acc(AccTile<MODE, G>& acc) {
#pragma unroll
  for (int i = 0; i < Blk<MODE, G>::FM; ++i)
#pragma unroll
    for (int j = 0; j < Blk<MODE, G>::FN; ++j) acc[i][j] = typename Traits<MODE>::acc_t{};
}

// Lane constants of the fragment reads: (row in block, chunk term, row swizzle).
template <int MODE>
__device__ __forceinline__ void frag_lane(int lane, int& frow, int& fq, int& fsw) {
  if constexpr (Traits<MODE>::MD == 16) {
    frow = lane & 15;
    fq = lane >> 4;
  } else {
    frow = lane & 31;
    fq = lane >> 5;
  }
  fsw = swz(frow);
}

// One operand fragment of sub-step s (the per-mode chunk mapping of read_frags).
template <int MODE>
__device__ __forceinline__ void read_frag(const uint8_t* row, int s, int fq, int fsw, Frag<MODE>& f) {
  if constexpr (MODE == F8) {
    f.lo = *reinterpret_cast<const v4i*>(row + ((fq ^ fsw) << 4));
    f.hi = *reinterpret_cast<const v4i*>(row + (((4 + fq) ^ fsw) << 4));
  } else {
    f.lo = *reinterpret_cast<const v4i*>(row + ((((MODE == F32 ? 2 : 4) * s + fq) ^ fsw) << 4));
  }
}

// MFMAs of block rows [I0, I1) of fc, with the reads of fn (sub-step s of sa/sb; B fragments
// first, then A rows in order, as the next sub-step consumes them) spread evenly over those
// rows, and hook(k) called before row k's reads (the stage DMA uses it).  Scheduling fences keep
// each read ahead of the MFMA row it is placed before; left alone, the compiler sinks every read
// next to its first use, which exposes the LDS latency.  Measured on the 16 x 16 modes: INT8
// +1-4%, BF16 +2-4%.  (FP8, one sub-step per stage, has its own schedule in mainloop_dma.)
template <int MODE, class G, int I0, int I1, class H>
__device__ __forceinline__ void mfma_rows_reading(AccTile<MODE, G>& acc, const FragSet<MODE, G>& fc,
                                                  FragSet<MODE, G>& fn, const uint8_t* sa, const uint8_t* sb,
                                                  int s, int a_row0, int b_row0, int fq, int fsw, H&& hook) {
  constexpr int FM = Blk<MODE, G>::FM, FN = Blk<MODE, G>::FN, MD = Blk<MODE, G>::MD;
  constexpr int NR = FM + FN, ROWS = I1 - I0;
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    hook(k);
#pragma unroll
    for (int r = k * NR / ROWS; r < (k + 1) * NR / ROWS; ++r) {
      if (r < FN) read_frag<MODE>(sb + (b_row0 + MD * r) * BKB, s, fq, fsw, fn.b[r]);
      else read_frag<MODE>(sa + (a_row0 + MD * (r - FN)) * BKB, s, fq, fsw, fn.a[r - FN]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < FN; ++j) mfma<MODE>(acc[I0 + k][j], fc.a[I0 + k], fc.b[j]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Number of 128-byte K stages of a row of Kb bytes.
__host__ __device__ constexpr int64_t k_stages(int64_t Kb) { return (Kb + BKB - 1) / BKB; }

// Direct-to-LDS main loop (rows 16-byte multiples of at most 2^23 bytes, bases 16-byte aligned;
// operands of any size, each workgroup addressing only its own rows).
//
// DMA: per stage each wave moves DMA_ROWS rows of both operand tiles with DMA_INSTR + DMA_INSTR
// buffer loads of 1 KiB: lane l -> row 8i + l/8, physical chunk l & 7, i.e. whole 128-byte
// rows, so both halves of an L2 line are requested by one instruction.  Rows past M/N and
// chunks past K read as zero through out-of-range buffer offsets.
//
// Two stage buffers.  Per stage kt (buffer kt & 1, SUB sub-steps), 16 x 16 modes:
//   read sub-step s+1 fragments | MFMAs of sub-step s            (s < SUB - 1; the reads are
//                                                                 interleaved with the MFMA rows,
//                                                                 see mfma_rows_reading)
//   wait for own stage kt+1 loads and all LDS reads; barrier  (stage kt+1 visible, buffer free)
//   read stage kt+1 sub-step 0 fragments | MFMAs of the last sub-step, with the DMA of stage
//   kt+2 into buffer kt & 1 spread over all of its MFMA rows
// The barrier thus sits between sub-steps: the next stage's first fragments and the DMA have a
// whole sub-step of MFMAs to hide behind.  Against a barrier after half of the last sub-step's
// rows (its reads and DMA over the other half), this measured 1.4-1.6% faster at K = 16384 and
// at FFN-up (N = 16384, K = 4096), equal at 4096^3, same bits.  FP32 (32 x 32 blocks) keeps
// the barrier after half of the last sub-step, with the DMA in one burst.  FP8 (one sub-step
// per stage) has the schedule described at stage_f8 below.
// Stage kt+1's loads have one whole stage to land.  Each accumulator sees K in order, sub-step
// by sub-step.
//
// The loop covers the 128-byte K stages [kt_begin, kt_begin + kt_count); a split-K launch
// gives each workgroup one such range (stages past the range, like chunks past K, load zeros).
template <int MODE, class G, bool PIPELINED = Traits<MODE>::MD == 16>
__device__ __forceinline__ void mainloop_dma(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, int M,
                                             int N, int64_t Kb, int tile_m0, int tile_n0, AccTile<MODE, G>& acc,
                                             int64_t kt_begin, int64_t kt_count) {
  constexpr int SUB = Traits<MODE>::sub_steps;
  static_assert(MODE == F8 || SUB % 2 == 0, "the last sub-step of a stage uses the second fragment set");
  static_assert(!PIPELINED || Traits<MODE>::MD == 16, "interleaved reads are measured for 16 x 16 modes");
  constexpr int FM = Blk<MODE, G>::FM;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  zero_acc<MODE, G>(acc);

  // Each workgroup addresses only its own rows: the windows [A + tile_m0 * Kb, + rows_a * Kb)
  // and [B + tile_n0 * Kb, + rows_b * Kb) are at most 256 rows of Kb < 2^23 bytes, so 32-bit
  // buffer offsets cover operands of any size.
  constexpr uint32_t kOob = 0x80000000u;  // beyond num_records: the load returns zeros
  const int uwave = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform copy for LDS bases
  const int rows_a = min(M - tile_m0, BM), rows_b = min(N - tile_n0, G::TN);
  const uint8_t* a_win = A + static_cast<int64_t>(tile_m0) * Kb;
  const uint8_t* b_win = B + static_cast<int64_t>(tile_n0) * Kb;
  const uint32_t rec_a = static_cast<uint32_t>(rows_a * Kb), rec_b = static_cast<uint32_t>(rows_b * Kb);

  // Per-lane window offsets of each DMA instruction (kOob for rows past the window) and the
  // byte offset of the logical chunk the lane moves.  Instruction i covers rows
  // wave * DMA_ROWS + 8i + [0, 8) (DMA_ROWS a multiple of 16), whose swizzle is
  // 4 (i & 1) + (l >> 4): the chunk offset depends on the parity of i only.
  static_assert(G::DMA_ROWS % 16 == 0 && G::DMA_ROWS_B % 16 == 0, "DMA row groups start at even row pairs");
  const uint32_t lchunk[2] = {static_cast<uint32_t>(((lane & 7) ^ (lane >> 4)) << 4),
                              static_cast<uint32_t>(((lane & 7) ^ (4 + (lane >> 4))) << 4)};
  uint32_t a_base[G::DMA_INSTR], b_base[G::DMA_INSTR_B];
#pragma unroll
  for (int i = 0; i < G::DMA_INSTR; ++i) {
    const int r = wave * G::DMA_ROWS + 8 * i + (lane >> 3);
    a_base[i] = r < rows_a ? static_cast<uint32_t>(r * Kb) + lchunk[i & 1] : kOob;
  }
#pragma unroll
  for (int i = 0; i < G::DMA_INSTR_B; ++i) {
    const int r = wave * G::DMA_ROWS_B + 8 * i + (lane >> 3);
    b_base[i] = r < rows_b ? static_cast<uint32_t>(r * Kb) + lchunk[i & 1] : kOob;
  }
  const uint32_t lds_row0 = static_cast<uint32_t>(uwave * G::DMA_ROWS * BKB);
  const uint32_t lds_row0_b = static_cast<uint32_t>(uwave * G::DMA_ROWS_B * BKB);
  // Stage kr (relative to kt_begin) moves the window start by the stage offset (scalar) and
  // keeps the lane offsets: row r's chunk then ends before row r + 1 starts, and rows past the
  // window stay out of range.  In the last partial stage of a ragged K (Kb % 128 != 0) the lanes
  // whose chunk starts at or past K set the offset's top bit (out of range: zeros); stages past
  // the range use an empty window.  One VALU op per DMA instruction.
  //
  // A stage is NQ instructions, A_0 B_0 A_1 B_1 ... (then the rest of the longer list);
  // dma_range issues instructions [q0, q1) of stage kr.
  constexpr int NQ = G::DMA_INSTR + G::DMA_INSTR_B;
  constexpr int NPAIR = G::DMA_INSTR < G::DMA_INSTR_B ? G::DMA_INSTR : G::DMA_INSTR_B;
  auto dma_range = [&](uint8_t* sa, uint8_t* sb, int64_t kr, int q0, int q1) {
    const uint32_t kofs = static_cast<uint32_t>((kt_begin + kr) * BKB);
    const uint32_t la = lds_addr(sa) + lds_row0, lb = lds_addr(sb) + lds_row0_b;
    const bool live = kr < kt_count;
    const int64_t rem = Kb - static_cast<int64_t>(kofs);  // bytes of K left at this stage
    const uint32_t kill[2] = {static_cast<int64_t>(lchunk[0]) < rem ? 0u : kOob,
                              static_cast<int64_t>(lchunk[1]) < rem ? 0u : kOob};
    const uint32_t ofs = live ? kofs : 0;
    const v4i ra = window_rsrc(a_win, live ? rec_a : 0, ofs), rb = window_rsrc(b_win, live ? rec_b : 0, ofs);
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      const bool is_b = q < 2 * NPAIR ? (q & 1) != 0 : G::DMA_INSTR_B > G::DMA_INSTR;
      const int i = q < 2 * NPAIR ? q >> 1 : q - NPAIR;
      if (!is_b) dma16<G::WAVES == 4>(la + 8 * i * BKB, a_base[i] | kill[i & 1], ra);
      else dma16<G::WAVES == 4>(lb + 8 * i * BKB, b_base[i] | kill[i & 1], rb);
    }
  };
  auto dma = [&](uint8_t* sa, uint8_t* sb, int64_t kr) { dma_range(sa, sb, kr, 0, NQ); };
  // The DMA of stage kr spread over the ROWS MFMA rows that follow the stage barrier: row k issues
  // instructions [k NQ / ROWS, (k + 1) NQ / ROWS).  Issued in one burst right after the barrier,
  // the eight waves' DMA queued behind each other while both waves of every SIMD stalled; spread
  // over the rows the FFN-down main loop measured 7-10% faster (same bits).
  auto dma_spread = [&](uint8_t* sa, uint8_t* sb, int64_t kr, auto rows_tag) {
    constexpr int ROWS = decltype(rows_tag)::value;
    return [&, sa, sb, kr](int k) {
#pragma unroll
      for (int kk = 0; kk < ROWS; ++kk)
        if (kk == k) dma_range(sa, sb, kr, kk * NQ / ROWS, (kk + 1) * NQ / ROWS);
    };
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  const int64_t kt_padded = (kt_count + 1) / 2 * 2;

  // A wave whose block rows all lie past the matrix (short M: rows [M, 256) of the tile) has
  // nothing to multiply.  It still moves its share of every stage and meets every barrier of the
  // loop below (prologue, one per stage, drain), at the same points, and leaves its
  // accumulators at zero, as the zero rows it would load give; the epilogue stores no row past
  // M.  At M = 128 this halves the tile's MFMAs and fragment reads (one of each SIMD's two waves
  // idles); the outputs are unchanged.  Eight-wave grids only: the four-wave grid, at 256
  // accumulators, spills with the second loop beside its main one.
  if (G::WAVES == 8 && (uwave / G::WAVES_N) * G::WM >= rows_a) {
    auto idle_stage = [&](auto cur_tag, int64_t kt) {
      constexpr int CUR = decltype(cur_tag)::value;
      wait_stage<0>();
      stage_barrier();
      dma(stage_a<CUR>(), stage_b<CUR>(), kt + 2);
    };
    dma(stage_a<0>(), stage_b<0>(), 0);
    dma(stage_a<1>(), stage_b<1>(), 1);
    wait_stage<NQ>();
    stage_barrier();
    for (int64_t kt = 0; kt < kt_padded; kt += 2) {
      idle_stage(I0{}, kt);
      idle_stage(I1{}, kt + 1);
    }
    wait_stage<0>();
    stage_barrier();
    return;
  }

  int frow, fq, fsw;
  frag_lane<MODE>(lane, frow, fq, fsw);
  const int a_row0 = wm * G::WM + frow, b_row0 = wn * G::WN + frow;

  FragSet<MODE, G> f0, f1;

  auto no_hook = [](int) {};
  auto stage = [&](auto cur_tag, int64_t kt) {
    constexpr int CUR = decltype(cur_tag)::value, NXT = CUR ^ 1;
#pragma unroll
    for (int s = 0; s + 1 < SUB; ++s) {
      if constexpr (PIPELINED) {
        mfma_rows_reading<MODE, G, 0, FM>(acc, (s & 1) ? f1 : f0, (s & 1) ? f0 : f1, stage_a<CUR>(),
                                          stage_b<CUR>(), s + 1, a_row0, b_row0, fq, fsw, no_hook);
      } else {
        read_frags<MODE, G>(stage_a<CUR>(), stage_b<CUR>(), s + 1, a_row0, b_row0, fq, fsw, (s & 1) ? f0 : f1);
        mfma_rows<MODE, G, 0, FM>(acc, (s & 1) ? f1 : f0);
      }
    }
    if constexpr (PIPELINED) {
      wait_stage<0>();
      // The DMA below overwrites this buffer: every wave's reads of it must have returned.
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      stage_barrier();
      auto hook = dma_spread(stage_a<CUR>(), stage_b<CUR>(), kt + 2, std::integral_constant<int, FM>{});
      mfma_rows_reading<MODE, G, 0, FM>(acc, f1, f0, stage_a<NXT>(), stage_b<NXT>(), 0, a_row0, b_row0, fq, fsw,
                                        hook);
    } else {
      // FP32 (32 x 32 blocks, two rows per half): half of the last sub-step's rows before the
      // barrier, and the DMA in one burst.
      mfma_rows<MODE, G, 0, FM / 2>(acc, f1);
      wait_stage<0>();
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      stage_barrier();
      dma(stage_a<CUR>(), stage_b<CUR>(), kt + 2);
      read_frags<MODE, G>(stage_a<NXT>(), stage_b<NXT>(), 0, a_row0, b_row0, fq, fsw, f0);
      mfma_rows<MODE, G, FM / 2, FM>(acc, f1);
    }
  };
  // FP8: one 16 x 16 x 128 MFMA per block and stage (32-byte fragments: chunks fq and 4 + fq),
  // so there is no second sub-step to read ahead into, and two full fragment sets do not fit
  // beside the accumulators.  One set of B fragments and a ring of four A fragments (slot i % 4
  // for block row i).  Per stage (FM = 8):
  //   rows 0, 1 column by column (B fragment 0 first), reading A rows 2, 3;
  //   rows 2 .. 4 in order, reading A rows 4 .. 7 (three rows ahead), so the stage's last read
  //   of this buffer precedes row 4's MFMAs;
  //   wait for own stage kt+1 loads and all LDS reads; barrier;
  //   row 5, then rows 6, 7 column by column, with the DMA of stage kt+2 spread over these five
  //   steps; the next stage's A rows 0, 1 are read around row 5, and each B fragment is re-read
  //   from the next stage's buffer as soon as its column of row 7 has issued (the next stage's
  //   first columns cover those reads).
  // With FM = 4 (the 256 x 128 half tile) there are no middle rows: rows 0, 1, the barrier, then
  // rows 2, 3 column by column.  Against the 32 x 32 x 64 form (two 64-byte sub-steps, both
  // fragment sets, barrier after half of the last sub-step) this measured 5-7% faster on the
  // FFN-down, FFN-up, 4096^3, 9914 x 4096^2 and 4096 x 14336 x 5376 shapes, with the same bits;
  // a variant reading A two rows ahead (barrier before rows 6, 7) gained 0-2.5%.
  const uint32_t f8_a0 = static_cast<uint32_t>(a_row0 * BKB + ((fq ^ fsw) << 4));
  const uint32_t f8_a1 = static_cast<uint32_t>(a_row0 * BKB + (((4 + fq) ^ fsw) << 4));
  const uint32_t f8_b0 = static_cast<uint32_t>(b_row0 * BKB + ((fq ^ fsw) << 4));
  const uint32_t f8_b1 = static_cast<uint32_t>(b_row0 * BKB + (((4 + fq) ^ fsw) << 4));
  auto f8_read = [&](const uint8_t* buf, uint32_t o0, uint32_t o1, int blk, Frag<MODE>& fr) {
    fr.lo = *reinterpret_cast<const v4i*>(buf + o0 + blk * Blk<MODE, G>::MD * BKB);
    fr.hi = *reinterpret_cast<const v4i*>(buf + o1 + blk * Blk<MODE, G>::MD * BKB);
  };
  Frag<MODE> f8_b[Blk<MODE, G>::FN];
  Frag<MODE> f8_ring[4];
  auto stage_f8 = [&](auto cur_tag, int64_t kt) {
    constexpr int CUR = decltype(cur_tag)::value, NXT = CUR ^ 1;
    constexpr int FN = Blk<MODE, G>::FN;
    static_assert(FM % 4 == 0, "ring slots repeat every stage");
    const uint8_t* ca = stage_a<CUR>();
    f8_read(ca, f8_a0, f8_a1, 2, f8_ring[2]);
    f8_read(ca, f8_a0, f8_a1, 3, f8_ring[3]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      mfma<MODE>(acc[0][j], f8_ring[0], f8_b[j]);
      mfma<MODE>(acc[1][j], f8_ring[1], f8_b[j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Rows 2 .. FM - 4 read A three rows ahead (row 2 also reads row 4's), so the last A read of
    // the stage precedes row FM - 4's MFMAs and the barrier can follow them.
#pragma unroll
    for (int i = 2; i < FM - 3; ++i) {
      if (i == 2 && FM > 4) f8_read(ca, f8_a0, f8_a1, 4, f8_ring[0]);
      if (i + 3 < FM) f8_read(ca, f8_a0, f8_a1, i + 3, f8_ring[(i + 3) % 4]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < FN; ++j) mfma<MODE>(acc[i][j], f8_ring[i % 4], f8_b[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_stage<0>();
    // The DMA below overwrites this buffer: every wave's reads of it must have returned.
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    stage_barrier();
    const uint8_t* na = stage_a<NXT>();
    const uint8_t* nb = stage_b<NXT>();
    // With more than four block rows, row FM - 3 runs after the barrier (in order); then the last
    // two rows column by column.
    constexpr int MIDDLE = FM > 4 ? 1 : 0, STEPS = FN + MIDDLE;
    if constexpr (MIDDLE) {
      dma_range(stage_a<CUR>(), stage_b<CUR>(), kt + 2, 0, NQ / STEPS);
      f8_read(na, f8_a0, f8_a1, 0, f8_ring[0]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < FN; ++j) mfma<MODE>(acc[FM - 3][j], f8_ring[(FM - 3) % 4], f8_b[j]);
      __builtin_amdgcn_sched_barrier(0);
      f8_read(na, f8_a0, f8_a1, 1, f8_ring[1]);
    } else {
      f8_read(na, f8_a0, f8_a1, 0, f8_ring[0]);
      f8_read(na, f8_a0, f8_a1, 1, f8_ring[1]);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      dma_range(stage_a<CUR>(), stage_b<CUR>(), kt + 2, (j + MIDDLE) * NQ / STEPS, (j + MIDDLE + 1) * NQ / STEPS);
      __builtin_amdgcn_sched_barrier(0);
      mfma<MODE>(acc[FM - 2][j], f8_ring[(FM - 2) % 4], f8_b[j]);
      mfma<MODE>(acc[FM - 1][j], f8_ring[(FM - 1) % 4], f8_b[j]);
      __builtin_amdgcn_sched_barrier(0);
      f8_read(nb, f8_b0, f8_b1, j, f8_b[j]);
    }
  };
  dma(stage_a<0>(), stage_b<0>(), 0);
  dma(stage_a<1>(), stage_b<1>(), 1);
  wait_stage<G::DMA_INSTR + G::DMA_INSTR_B>();  // stage 0 landed (own loads)
  stage_barrier();
  if constexpr (MODE == F8) {
#pragma unroll
    for (int j = 0; j < Blk<MODE, G>::FN; ++j) f8_read(stage_b<0>(), f8_b0, f8_b1, j, f8_b[j]);
    f8_read(stage_a<0>(), f8_a0, f8_a1, 0, f8_ring[0]);
    f8_read(stage_a<0>(), f8_a0, f8_a1, 1, f8_ring[1]);
  } else {
    read_frags<MODE, G>(stage_a<0>(), stage_b<0>(), 0, a_row0, b_row0, fq, fsw, f0);
  }
  for (int64_t kt = 0; kt < kt_padded; kt += 2) {
    if constexpr (MODE == F8) {
      stage_f8(I0{}, kt);
      stage_f8(I1{}, kt + 1);
    } else {
      stage(I0{}, kt);
      stage(I1{}, kt + 1);
    }
  }
  // Drain the trailing (zero) DMAs before the LDS is reused or the wave exits.
  wait_stage<0>();
  stage_barrier();
}

// Register-staged main loop for rows that are not 16-byte multiples (small, odd K): bytes
// are loaded one at a time with exact bounds, then stored to the same swizzled layout.
template <int MODE, class G>
__device__ __forceinline__ void mainloop_staged(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, int M,
                                                int N, int64_t Kb, int tile_m0, int tile_n0, AccTile<MODE, G>& acc) {
  constexpr int SUB = Traits<MODE>::sub_steps;
  constexpr int CHUNKS = BKB / 16;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  zero_acc<MODE, G>(acc);
  constexpr int ROWS_PER_PASS = G::THREADS / CHUNKS;  // chunk (t % CHUNKS) of rows t / CHUNKS + pass * ROWS_PER_PASS
  const int lc = tid % CHUNKS, lr = tid / CHUNKS;
  const int64_t kt_count = k_stages(Kb);
  int frow, fq, fsw;
  frag_lane<MODE>(lane, frow, fq, fsw);
  const int a_row0 = wm * G::WM + frow, b_row0 = wn * G::WN + frow;
  for (int64_t kt = 0; kt < kt_count; ++kt) {
    const int64_t kb = kt * BKB + lc * 16;
    for (int i = 0; i < BM / ROWS_PER_PASS; ++i) {
      const int r = lr + ROWS_PER_PASS * i;
      const int am = tile_m0 + r, bn = r < G::TN ? tile_n0 + r : N;  // rows past the tile width: zeros
      uint32_t wa[4] = {0, 0, 0, 0}, wb[4] = {0, 0, 0, 0};
      for (int e = 0; e < 16; ++e) {
        const bool kin = kb + e < Kb;
        const uint32_t va = (am < M && kin) ? A[(int64_t)am * Kb + kb + e] : 0u;
        const uint32_t vb = (bn < N && kin) ? B[(int64_t)bn * Kb + kb + e] : 0u;
        wa[e >> 2] |= va << (8 * (e & 3));
        wb[e >> 2] |= vb << (8 * (e & 3));
      }
      const int off = r * BKB + ((lc ^ swz(r)) << 4);
      *reinterpret_cast<uint4*>(stage_a<0>() + off) = make_uint4(wa[0], wa[1], wa[2], wa[3]);
      *reinterpret_cast<uint4*>(stage_b<0>() + off) = make_uint4(wb[0], wb[1], wb[2], wb[3]);
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
      FragSet<MODE, G> f;
      read_frags<MODE, G>(stage_a<0>(), stage_b<0>(), s, a_row0, b_row0, fq, fsw, f);
      mfma_rows<MODE, G, 0, Blk<MODE, G>::FM>(acc, f);
    }
    __syncthreads();
  }
}

// Lane geometry of an accumulator tile: element e of block (i, j) lies at tile row row(i, e) and
// tile column col(j).  16 x 16 blocks: lane l holds column l & 15, rows 4 (l >> 4) + e;
// 32 x 32 blocks: column l & 31, rows 8 (e >> 2) + 4 (l >> 5) + (e & 3).
// The lane index comes from an opaque copy of threadIdx.x taken after the main loop: loads that
// depend on it (scales, bias) then stay after the loop instead of being hoisted into its
// register budget (the 16 x 16 main loop uses 241 of 256 VGPRs).
__device__ __forceinline__ int tid_after_mainloop() {
  int t = threadIdx.x;
  __asm__ volatile("" : "+v"(t));
  return t;
}

template <int MODE, class G>
struct AccGeom {
  static constexpr int MD = Blk<MODE, G>::MD, FM = Blk<MODE, G>::FM, FN = Blk<MODE, G>::FN;
  static constexpr int PER = MD == 32 ? 16 : 4;  // elements per block and lane
  int r0, c0;
  __device__ __forceinline__ explicit AccGeom(int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
    r0 = wm * G::WM + (lane >> (MD == 32 ? 5 : 4)) * 4;
    c0 = wn * G::WN + (lane & (MD - 1));
  }
  __device__ __forceinline__ int row(int i, int e) const {
    return r0 + i * MD + (MD == 32 ? (e >> 2) * 8 + (e & 3) : e);
  }
  __device__ __forceinline__ int col(int j) const { return c0 + j * MD; }
};

// A tile's row and column scales, PER per thread (scale t on thread t % THREADS; [0, BM) the
// rows, [BM, BM + TN) the columns; 0 past the matrix), loaded before the main loop so that
// their latency hides behind it instead of opening the epilogue: 0.1-0.7 us less per tile
// round (A/B, same bits: 4096^3 56.1 -> 55.4 us, FFN-up 211.0 -> 209.1 us).  The loads are
// issued before the loop's first DMA, so the loop's in-order vmcnt waits cover them and their
// counts stay exact.
template <class G>
struct TileScalePrefetch {
  static constexpr int PER = (BM + G::TN + G::THREADS - 1) / G::THREADS;  // scales per thread
  float v[PER];
  __device__ __forceinline__ TileScalePrefetch(const float* __restrict__ sa, const float* __restrict__ sb, int M,
                                               int N, int m0, int n0) {
    if constexpr (PER == 1) {
      // One scale per thread: a single load from either vector (the eight-wave grids).
      const int t = threadIdx.x;
      const int m = m0 + t, n = n0 + t - BM;
      v[0] = t < BM ? (m < M ? sa[m] : 0.0f) : (t < BM + G::TN && n < N ? sb[n] : 0.0f);
    } else {
      // Thread t takes row scale t and column scale t (PER == 2: BM == TN == THREADS).
      static_assert(PER == 2 && G::THREADS == BM && G::TN == BM, "two scales per thread: one row, one column");
      const int t = threadIdx.x;
      v[0] = m0 + t < M ? sa[m0 + t] : 0.0f;
      v[1] = n0 + t < N ? sb[n0 + t] : 0.0f;
    }
  }
};

// Row and column scales of a tile, staged in the LDS after the 16-bit tile (every thread of the
// workgroup constructs it after the main loop, whose last barrier freed the LDS): from global
// memory, one coalesced load per thread, or from the prefetched values.  Lanes then read their
// scales from the LDS one block row at a time, so the epilogue holds few extra registers.
template <class G>
struct TileScales {
  const float* s;  // rows [0, BM), then columns [BM, BM + G::TN)
  __device__ __forceinline__ TileScales(const float* __restrict__ sa, const float* __restrict__ sb, int M, int N,
                                        int m0, int n0, int tid) {
    float* w = reinterpret_cast<float*>(g_lds + EPI_SCALES_OFFSET);
    for (int t = tid; t < BM + G::TN; t += G::THREADS) {
      const int m = m0 + t, n = n0 + t - BM;
      w[t] = t < BM ? (m < M ? sa[m] : 0.0f) : (n < N ? sb[n] : 0.0f);
    }
    __syncthreads();
    s = w;
  }
  __device__ __forceinline__ TileScales(const TileScalePrefetch<G>& pre, int tid) {
    float* w = reinterpret_cast<float*>(g_lds + EPI_SCALES_OFFSET);
#pragma unroll
    for (int i = 0; i < TileScalePrefetch<G>::PER; ++i) {
      const int t = tid + i * G::THREADS;
      if (t < BM + G::TN) w[t] = pre.v[i];
    }
    __syncthreads();
    s = w;
  }
  __device__ __forceinline__ float row(int r) const { return s[r]; }
  __device__ __forceinline__ float col(int c) const { return s[BM + c]; }
};

// Visit every accumulator element with its global (row, col).
template <class G, class AccT, int FM, int FN, class F>
__device__ __forceinline__ void for_each_acc(const AccT (&acc)[FM][FN], int tile_m0, int tile_n0, F&& f) {
  constexpr int MD = G::WM / FM;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  if constexpr (MD == 32) {
    const int col_in = lane & 31, row_half = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = tile_m0 + wm * G::WM + i * 32 + (r >> 2) * 8 + row_half + (r & 3);
          const int n = tile_n0 + wn * G::WN + j * 32 + col_in;
          f(m, n, acc[i][j][r]);
        }
  } else {
    const int col_in = lane & 15, row_q = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = tile_m0 + wm * G::WM + i * 16 + row_q + r;
          const int n = tile_n0 + wn * G::WN + j * 16 + col_in;
          f(m, n, acc[i][j][r]);
        }
  }
}

}  // namespace gemm
}  // namespace m5k
