// W8A8 / FP8 / BF16 / FP16 linear layers on gfx950 MFMA with fused epilogues.
//
// Contract: src/m5kernels/metal.py:158-269 (gemm) with the epilogue strings of
// metal.py:88-128:
//   quantized  C = O(float(acc) * AS[row] * BS[col])            (left to right, FP32)
//   + bias     C = O(float(acc) * AS[row] * BS[col] + Bias[..])  (before the output cast)
//   gated      branch = bf16(value); C = bf16(float(Residual) + float(branch) * float(Gate[..]))
//   float      C = O(float(acc))
// The library is compiled with -ffp-contract=off so none of these products and sums is
// fused into an FMA: the FP32 rounding sequence is exactly the one written above.
#pragma once
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "gemm_core.h"

namespace m5k {
namespace gemm {
namespace detail {

enum { EPI_NONE = 0, EPI_VECTOR = 1, EPI_TABLE = 2 };

struct EpiParams {
  const float* sa;
  const float* sb;
  void* c;
  const float* bias;
  const int32_t* bias_map;
  const uint16_t* residual;
  const uint16_t* gate;
  const int32_t* gate_map;
  int coalesced;  // 16-bit output with N % 8 == 0 and 16-byte aligned c / residual / gate
};

// RAW: write INT32 accumulators (I8 only).
// Wave grid used by every GEMM kernel of the library.
using KernelGrid = Grid8;

// The tile's scales ahead of the main loop (quantized modes with a scale epilogue; nothing for the
// others).
template <int MODE, bool RAW, class G>
__device__ __forceinline__ TileScalePrefetch<G> prefetch_scales(const EpiParams& p, int M, int N, int m0, int n0) {
  if constexpr ((MODE == I8 || MODE == F8) && !RAW) return TileScalePrefetch<G>(p.sa, p.sb, M, N, m0, n0);
  else return TileScalePrefetch<G>(nullptr, nullptr, 0, 0, 0, 0);
}

// Scale epilogue of one 256 x G::TN tile (every thread of the workgroup calls it; the LDS is
// free).  RAW writes the INT32 accumulators.  The per-row and per-column operands of the
// lane's elements (scales, bias vector) are loaded in one batch before the arithmetic, and a
// bias table's offsets and values one block row at a time, so the epilogue waits for memory a
// few times instead of once per element.
template <int MODE, int OUT_DT, int BIAS, int GATE, bool RAW, class G = KernelGrid>
__device__ __forceinline__ void epilogue(const AccTile<MODE, G>& acc, int M, int N, int m0, int n0,
                                         const EpiParams& p, const TileScalePrefetch<G>& pre) {
  using Geo = AccGeom<MODE, G>;
  constexpr bool QUANT = MODE == I8 || MODE == F8;
  const int tid = tid_after_mainloop();
  const Geo geo(tid);
  if constexpr (RAW) {
#pragma unroll
    for (int i = 0; i < Geo::FM; ++i)
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) {
          const int m = m0 + geo.row(i, e), n = n0 + geo.col(j);
          if (m < M && n < N) static_cast<int32_t*>(p.c)[(int64_t)m * N + n] = acc[i][j][e];
        }
    return;
  } else {
    float cs[QUANT ? Geo::FN : 1];
    const float* sc = nullptr;
    if constexpr (QUANT) {
      const TileScales<G> ts(pre, tid);
      sc = ts.s;
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j) cs[j] = ts.col(geo.col(j));
    }
    float bvec[BIAS == EPI_VECTOR ? Geo::FN : 1];
    if constexpr (BIAS == EPI_VECTOR) {
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j) {
        const int n = n0 + geo.col(j);
        bvec[j] = n < N ? p.bias[n] : 0.0f;
      }
    }
    // FP32 value of block row i's elements: the scale epilogue, then the bias (a bias table's
    // row offsets and values are loaded per block row, two batches).
    auto row_values = [&](int i, float (&val)[Geo::FN][Geo::PER]) {
      float rs[QUANT ? Geo::PER : 1];
      if constexpr (QUANT) {
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) rs[e] = sc[geo.row(i, e)];
      }
      float tb[BIAS == EPI_TABLE ? Geo::FN : 1][BIAS == EPI_TABLE ? Geo::PER : 1];
      if constexpr (BIAS == EPI_TABLE) {
        int64_t brow[Geo::PER];
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) {
          const int m = m0 + geo.row(i, e);
          brow[e] = m < M ? (int64_t)p.bias_map[m] * N : 0;
        }
#pragma unroll
        for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
          for (int e = 0; e < Geo::PER; ++e) {
            const int m = m0 + geo.row(i, e), n = n0 + geo.col(j);
            tb[j][e] = (m < M && n < N) ? p.bias[brow[e] + n] : 0.0f;
          }
      }
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) {
          float value;
          if constexpr (QUANT) value = (static_cast<float>(acc[i][j][e]) * rs[e]) * cs[j];
          else value = acc[i][j][e];
          if constexpr (BIAS == EPI_VECTOR) value = value + bvec[j];
          if constexpr (BIAS == EPI_TABLE) value = value + tb[j][e];
          val[j][e] = value;
        }
    };

    // 16-bit outputs: stage the rounded tile (the BF16 branch for the gated form) in the LDS the
    // main loop has released, then write whole 512-byte tile rows with 16-byte streaming stores.
    if constexpr (OUT_DT == M5K_BF16 || OUT_DT == M5K_F16) {
      if (p.coalesced) {
        uint16_t* tile = reinterpret_cast<uint16_t*>(g_lds);
#pragma unroll
        for (int i = 0; i < Geo::FM; ++i) {
          float val[Geo::FN][Geo::PER];
          row_values(i, val);
#pragma unroll
          for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
            for (int e = 0; e < Geo::PER; ++e) {
              // Entries past M or N are staged unmasked: the write-out below skips them.
              const int r = geo.row(i, e), c = geo.col(j);
              const float value = val[j][e];
              tile[r * TILE16_STRIDE + c] = static_cast<uint16_t>(
                  GATE != EPI_NONE || OUT_DT == M5K_BF16 ? f32_to_bf16_bits(value) : f32_to_f16_bits(value));
            }
        }
        __syncthreads();
        constexpr int CPR = G::TN / 8;  // 16-byte chunks per tile row
        for (int c = threadIdx.x; c < BM * CPR; c += G::THREADS) {
          const int r = c / CPR, cc = c % CPR;
          const int m = m0 + r, n = n0 + 8 * cc;
          if (m >= M || n >= N) continue;  // N % 8 == 0: a chunk is wholly in or out
          uint4 w = *reinterpret_cast<const uint4*>(tile + r * TILE16_STRIDE + 8 * cc);
          const int64_t idx = (int64_t)m * N + n;
          if constexpr (GATE != EPI_NONE) {
            const int64_t goff = GATE == EPI_TABLE ? (int64_t)p.gate_map[m] * N : 0;
            const uint4 rw = *reinterpret_cast<const uint4*>(p.residual + idx);
            const uint4 gw = *reinterpret_cast<const uint4*>(p.gate + goff + n);
            const uint32_t bs[4] = {w.x, w.y, w.z, w.w}, rs[4] = {rw.x, rw.y, rw.z, rw.w},
                           gs[4] = {gw.x, gw.y, gw.z, gw.w};
            uint32_t out[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float lo = bf16_bits_to_f32(rs[t] & 0xFFFFu) +
                               bf16_bits_to_f32(bs[t] & 0xFFFFu) * bf16_bits_to_f32(gs[t] & 0xFFFFu);
              const float hi =
                  bf16_bits_to_f32(rs[t] >> 16) + bf16_bits_to_f32(bs[t] >> 16) * bf16_bits_to_f32(gs[t] >> 16);
              out[t] = f32x2_to_bf16x2(lo, hi);
            }
            w = make_uint4(out[0], out[1], out[2], out[3]);
          }
          store_stream16(static_cast<uint16_t*>(p.c) + idx, w);
        }
        return;
      }
    }

#pragma unroll
    for (int i = 0; i < Geo::FM; ++i) {
      float val[Geo::FN][Geo::PER];
      row_values(i, val);
      // The gated form's residual and gate values of this block row, loaded in one batch.
      float res[GATE != EPI_NONE ? Geo::FN : 1][GATE != EPI_NONE ? Geo::PER : 1];
      float gte[GATE != EPI_NONE ? Geo::FN : 1][GATE != EPI_NONE ? Geo::PER : 1];
      if constexpr (GATE != EPI_NONE) {
#pragma unroll
        for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
          for (int e = 0; e < Geo::PER; ++e) {
            const int m = m0 + geo.row(i, e), n = n0 + geo.col(j);
            const bool in = m < M && n < N;
            const int64_t goff = GATE == EPI_TABLE && in ? (int64_t)p.gate_map[m] * N : 0;
            res[j][e] = in ? bf16_bits_to_f32(p.residual[(int64_t)m * N + n]) : 0.0f;
            gte[j][e] = in ? bf16_bits_to_f32(p.gate[goff + n]) : 0.0f;
          }
      }
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) {
          const int m = m0 + geo.row(i, e), n = n0 + geo.col(j);
          if (m >= M || n >= N) continue;
          const int64_t idx = (int64_t)m * N + n;
          if constexpr (GATE != EPI_NONE) {
            const float branch = round_through<M5K_BF16>(val[j][e]);
            store_elem<M5K_BF16>(p.c, idx, res[j][e] + branch * gte[j][e]);
          } else {
            store_elem<OUT_DT>(p.c, idx, val[j][e]);
          }
        }
    }
  }
}

// One 256 x G::TN output tile per workgroup.
template <int MODE, bool ALIGNED, int OUT_DT, int BIAS, int GATE, bool RAW, class G = KernelGrid>
__global__ __launch_bounds__(G::THREADS, 1) void gemm_kernel(const uint8_t* __restrict__ A,
                                                             const uint8_t* __restrict__ B, int M, int N,
                                                             int64_t Kb, EpiParams p) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + G::TN - 1) / G::TN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * G::TN;
  const TileScalePrefetch<G> pre = prefetch_scales<MODE, RAW, G>(p, M, N, m0, n0);
  AccTile<MODE, G> acc;
  if constexpr (ALIGNED) mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, 0, k_stages(Kb));
  else mainloop_staged<MODE, G>(A, B, M, N, Kb, m0, n0, acc);
  epilogue<MODE, OUT_DT, BIAS, GATE, RAW, G>(acc, M, N, m0, n0, p, pre);
}

// ---- Mixed tiles for a partial last round ---------------------------------------------------
//
// T tiles on C CUs (one workgroup per CU) take ceil(T / C) rounds; when the last round is only
// partly filled, most CUs idle through it.  The mixed launch runs the first `full` tiles of the
// raster order (a whole number of rounds) as 256 x 256 tiles and splits each remaining tile
// into two 256 x 128 halves, which take a little over half a tile's time each, so the leftover
// work runs as one shorter, better-filled round.  Each output element is still one
// workgroup's dot product over all of K: results are bit-identical to the plain launch.
// Workgroups [0, full) are the full tiles.  Workgroup full + w runs logical half
// h = xcd_logical(w), which is half h & 1 of tile full + h / 2 in the raster order.  full is
// a multiple of 8, so w keeps the hardware's XCD (w % 8 == (full + w) % 8), each XCD gets a
// contiguous run of h, and the two halves of a tile land on one XCD unless a run boundary
// falls between them.
using HalfGrid = Grid8Half;

template <int MODE, int OUT_DT, int BIAS, int GATE, bool RAW>
__global__ __launch_bounds__(KernelGrid::THREADS, 1) void gemm_mixed_kernel(const uint8_t* __restrict__ A,
                                                                            const uint8_t* __restrict__ B, int M,
                                                                            int N, int64_t Kb, int full,
                                                                            EpiParams p) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < full) {
    using G = KernelGrid;
    int tm, tn;
    band_coords(xcd_logical(bid, full), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const TileScalePrefetch<G> pre = prefetch_scales<MODE, RAW, G>(p, M, N, m0, n0);
    AccTile<MODE, G> acc;
    mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, 0, k_stages(Kb));
    epilogue<MODE, OUT_DT, BIAS, GATE, RAW, G>(acc, M, N, m0, n0, p, pre);
  } else {
    using G = HalfGrid;
    const int h = xcd_logical(bid - full, 2 * (tiles_m * tiles_n - full));
    int tm, tn;
    band_coords(full + (h >> 1), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN + (h & 1) * G::TN;
    if (n0 >= N) return;  // right half of a last tile column at most 128 wide (whole workgroup)
    const TileScalePrefetch<G> pre = prefetch_scales<MODE, RAW, G>(p, M, N, m0, n0);
    AccTile<MODE, G> acc;
    mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, 0, k_stages(Kb));
    epilogue<MODE, OUT_DT, BIAS, GATE, RAW, G>(acc, M, N, m0, n0, p, pre);
  }
}

constexpr int XCDS = 8;
// Time of a 256 x 128 tile in units of a 256 x 256 tile's (measured: 256 half tiles of
// 2048 x 4096 x 4096 INT8 in 0.57 of the 256 full tiles of 4096 x 4096 x 4096).
constexpr double kHalfTileCost = 0.56;

// Finish time, in 256 x 256 tile times, of `full` tiles (a multiple of the CU count: whole
// rounds) followed by `half` half tiles; workgroup w runs on XCD w % 8, whose CUs take its
// workgroups in order.
inline double mixed_makespan(int64_t full, int64_t half, int cus) {
  const int64_t c = cus / XCDS;
  const int64_t per = (half + XCDS - 1) / XCDS;  // the busiest XCD's half tiles
  return static_cast<double>(full / cus) + static_cast<double>((per + c - 1) / c) * kHalfTileCost;
}

// Full tiles of the mixed launch, or -1 for the plain launch.  Candidates keep the last one
// or two rounds of tiles as halves; the mixed launch is used for a predicted gain of 5% or
// more.  The full part is always whole rounds, so the half tiles start together once every
// full tile is done.  Measured on MI355X, half tiles that overlapped a partial round of full
// tiles ran slower than such a model predicts (4-8% behind the plain launch at N = 6144 and
// 14336), while the whole-round splits matched or beat it.
// M5K_GEMM_MIXED_TILES=0 in the environment selects the plain launch (read on every call).
inline int64_t mixed_full_tiles(int64_t m, int64_t n, int cus) {
  if (cus < XCDS || cus % XCDS) return -1;
  if (const char* env = std::getenv("M5K_GEMM_MIXED_TILES"); env && env[0] == '0') return -1;
  const int64_t total = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  const int64_t rounds = total / cus;
  if (total % cus == 0 || rounds > 64) return -1;  // no partial round, or one that is noise
  double best = static_cast<double>(rounds + 1) * 0.95;
  int64_t pick = -1;
  for (int64_t j = rounds; j >= 0 && j + 2 >= rounds; --j) {
    const int64_t full = j * cus;
    const double t = mixed_makespan(full, 2 * (total - full), cus);
    if (t < best) {
      best = t;
      pick = full;
    }
  }
  return pick;
}

// ---- Narrow tiles for a whole number of rounds ------------------------------------------------
//
// 256 x 224 tiles (Grid8Narrow, 16 x 16 modes) do 7/8 of a full tile's MFMAs.  Where their
// count fills whole rounds and the 256-wide count does not (N = 7168: 28 full or 32 narrow
// tile columns; at M = 4096, 448 tiles = 1.75 rounds against 512 = 2 rounds), the narrow grid
// finishes in 2 x 7/8 round times instead of 2.  Bit-identical to the plain launch for the
// same reason as the mixed launch.
constexpr double kNarrowTileCost = 0.9;  // 256 x 224 tile time / 256 x 256 tile time

// Predicted time, in 256 x 256 tile times, of the plain, mixed and narrow launches; returns
// true when the narrow launch is 5% or more ahead of both others.
inline bool narrow_pays(int64_t m, int64_t n, int cus, int64_t mixed_full) {
  if (cus <= 0) return false;
  if (const char* env = std::getenv("M5K_GEMM_NARROW_TILES"); env && env[0] == '0') return false;
  const int64_t tiles_m = (m + BM - 1) / BM;
  const int64_t plain_tiles = tiles_m * ((n + BN - 1) / BN);
  const int64_t narrow_tiles = tiles_m * ((n + Grid8Narrow::TN - 1) / Grid8Narrow::TN);
  if (plain_tiles > 64 * static_cast<int64_t>(cus)) return false;
  double other = static_cast<double>((plain_tiles + cus - 1) / cus);
  if (mixed_full >= 0) other = std::min(other, mixed_makespan(mixed_full, 2 * (plain_tiles - mixed_full), cus));
  const double narrow = static_cast<double>((narrow_tiles + cus - 1) / cus) * kNarrowTileCost;
  return narrow < 0.95 * other;
}

// The direct-to-LDS main loop needs 16-byte aligned rows and bases and 256-row windows that
// fit a 32-bit buffer offset (rows of at most 2^23 bytes); other operands take the
// register-staged loop.
inline bool dma_ok(const void* a, const void* b, int64_t kb) {
  return kb % 16 == 0 && kb <= (int64_t(1) << 23) && aligned16(a) && aligned16(b);
}

// SCHED_QUAD: plain 256 x 256 tiles on Grid4 (four waves of 128 x 128, one per SIMD, 256 AGPR
// accumulators), W8A8 only.  Never planned: on the FFN-down, FFN-up and 4096^3 GEMMs it measured
// 1.10-1.15x the time of the eight-wave grid (same bits), since a lone wave per SIMD has no
// sibling to issue MFMAs while it waits on LDS reads and stage barriers.  It stays a tuner option.
enum Schedule { SCHED_PLAIN = 0, SCHED_MIXED = 1, SCHED_NARROW = 2, SCHED_QUAD = 3 };

// A schedule forced for the calls of this host thread (m5k_gemm_set_schedule: the harness tuner),
// else one named by M5K_GEMM_SCHEDULE ("plain", "mixed", "narrow", "quad"; read on every call, for
// outside tools), else -1.  A forced mixed launch keeps the planner's full-tile count when it has
// one, else runs every tile of the last (or only) round as two halves.  Narrow applies to the
// 16 x 16 modes and quad to W8A8; the other modes run plain in their place.
inline thread_local int g_thread_schedule = -1;

inline int forced_schedule(bool md16, bool i8, int64_t m, int64_t n, int cus, int64_t& full) {
  int which = g_thread_schedule;
  if (which < 0) {
    const char* env = std::getenv("M5K_GEMM_SCHEDULE");
    if (env == nullptr || env[0] == '\0') return -1;
    if (std::strcmp(env, "plain") == 0) which = SCHED_PLAIN;
    else if (std::strcmp(env, "mixed") == 0) which = SCHED_MIXED;
    else if (std::strcmp(env, "narrow") == 0) which = SCHED_NARROW;
    else if (std::strcmp(env, "quad") == 0) which = SCHED_QUAD;
    else return -1;
  }
  full = -1;
  if (which == SCHED_PLAIN) return SCHED_PLAIN;
  if (which == SCHED_NARROW) return md16 ? SCHED_NARROW : SCHED_PLAIN;
  if (which == SCHED_QUAD) return i8 ? SCHED_QUAD : SCHED_PLAIN;
  if (which == SCHED_MIXED && cus >= XCDS && cus % XCDS == 0) {
    const int64_t total = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    full = mixed_full_tiles(m, n, cus);
    if (full < 0) full = total > cus ? (total - 1) / cus * cus : 0;
    return SCHED_MIXED;
  }
  return -1;
}

// Launch schedule of an aligned GEMM with an [m, n] output on `cus` CUs; `full` receives the
// mixed launch's full tiles (-1 otherwise).  Narrow tiles exist for the 16 x 16 modes only.
inline int plan_schedule(bool md16, bool i8, int64_t m, int64_t n, int cus, int64_t& full) {
  if (const int forced = forced_schedule(md16, i8, m, n, cus, full); forced >= 0) return forced;
  full = mixed_full_tiles(m, n, cus);
  if (md16 && narrow_pays(m, n, cus, full)) {
    full = -1;
    return SCHED_NARROW;
  }
  return full >= 0 ? SCHED_MIXED : SCHED_PLAIN;
}

template <int MODE, int OUT_DT, int BIAS, int GATE, bool RAW>
int launch(const void* a, const void* b, int64_t m, int64_t n, int64_t k, const EpiParams& p,
           hipStream_t st, const char* name) {
  const int64_t kb = k * Traits<MODE>::elem_bytes;
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  M5K_REQUIRE(tiles <= 0x7FFFFFFF, "%s: too many tiles", name);
  // The direct-to-LDS path addresses a tile's rows through 32-bit buffer windows.
  const bool aligned = dma_ok(a, b, kb);
  const dim3 grid(static_cast<unsigned>(tiles)), block(KernelGrid::THREADS);
  auto* A = static_cast<const uint8_t*>(a);
  auto* B = static_cast<const uint8_t*>(b);
  EpiParams q = p;
  q.coalesced = n % 8 == 0 && aligned16(p.c) && (p.residual == nullptr || (aligned16(p.residual) && aligned16(p.gate)));
  if (aligned) {
    int64_t full = -1;
    // The narrow 256 x 224 tile serves the 16 x 16 modes with 16-byte fragments (INT8, BF16,
    // FP16); FP8's 32-byte fragments for its seven B blocks do not fit beside the accumulators.
    constexpr bool narrow_ok = Traits<MODE>::MD == 16 && MODE != F8;
    const int sched = plan_schedule(narrow_ok, MODE == I8, m, n, device_cus(), full);
    if constexpr (narrow_ok) {
      if (sched == SCHED_NARROW) {
        using G = Grid8Narrow;
        const int64_t wgs = ((m + BM - 1) / BM) * ((n + G::TN - 1) / G::TN);
        launch_kernel(gemm_kernel<MODE, true, OUT_DT, BIAS, GATE, RAW, G>, dim3(static_cast<unsigned>(wgs)), block, st,
                      A, B, (int)m, (int)n, kb, q);
        return launch_status(name);
      }
    }
    if constexpr (MODE == I8) {
      if (sched == SCHED_QUAD) {
        launch_kernel(gemm_kernel<MODE, true, OUT_DT, BIAS, GATE, RAW, Grid4>, grid, dim3(Grid4::THREADS), st, A, B,
                      (int)m, (int)n, kb, q);
        return launch_status(name);
      }
    }
    if (sched == SCHED_MIXED) {
      const int64_t wgs = full + 2 * (tiles - full);
      launch_kernel(gemm_mixed_kernel<MODE, OUT_DT, BIAS, GATE, RAW>, dim3(static_cast<unsigned>(wgs)), block, st, A, B,
                    (int)m, (int)n, kb, static_cast<int>(full), q);
    } else {
      launch_kernel(gemm_kernel<MODE, true, OUT_DT, BIAS, GATE, RAW>, grid, block, st, A, B, (int)m, (int)n, kb, q);
    }
  } else
    launch_kernel(gemm_kernel<MODE, false, OUT_DT, BIAS, GATE, RAW>, grid, block, st, A, B, (int)m, (int)n, kb, q);
  return launch_status(name);
}

// ---- Split-K W8A8 for short M ------------------------------------------------------------
//
// With few output tiles (M of one or two tile rows) the plain launch leaves most CUs idle
// while its few workgroups stream the whole weight.  The split form gives each tile `splits`
// workgroups, each over a contiguous range of 128-byte K stages, writing raw INT32 partial tiles to
// workspace[s][M][N]; a second kernel sums the partials in split order (exact: INT32 sums of
// a bounded dot product) and applies the same FP32 epilogue as gemm_kernel, so the output
// is bit-identical to the plain launch.  P is the partial type: INT32 for INT8, FP32 for the
// FP8 split (launch_f8_splitk).
template <int MODE, class G = KernelGrid, class P = int32_t>
__global__ __launch_bounds__(G::THREADS, 1) void gemm_splitk_kernel(const uint8_t* __restrict__ A,
                                                                    const uint8_t* __restrict__ B, int M, int N,
                                                                    int64_t Kb, int splits, int64_t stages_per_split,
                                                                    P* __restrict__ partial) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + G::TN - 1) / G::TN;
  const int tile = static_cast<int>(blockIdx.x) / splits, s = static_cast<int>(blockIdx.x) % splits;
  int tm, tn;
  tile_coords(tile, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * G::TN;
  const int64_t kt_total = k_stages(Kb);
  const int64_t kt0 = s * stages_per_split;
  const int64_t kt1 = kt0 + stages_per_split < kt_total ? kt0 + stages_per_split : kt_total;
  AccTile<MODE, G> acc;
  mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, kt0, kt1 - kt0);
  P* out = partial + static_cast<int64_t>(s) * M * N;
  for_each_acc<G>(acc, m0, n0, [&](int m, int n, auto v) {
    if (m < M && n < N) out[static_cast<int64_t>(m) * N + n] = v;
  });
}

template <int OUT_DT, int BIAS, int GATE, class P = int32_t>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const P* __restrict__ partial, int splits, int M, int N,
                                                              EpiParams p) {
  const int64_t total = static_cast<int64_t>(M) * N;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * 256) {
    P v = 0;
    for (int s = 0; s < splits; ++s) v += partial[s * total + idx];
    const int m = static_cast<int>(idx / N), n = static_cast<int>(idx - static_cast<int64_t>(m) * N);
    float value = (static_cast<float>(v) * p.sa[m]) * p.sb[n];
    if constexpr (BIAS != EPI_NONE) {
      const int64_t boff = BIAS == EPI_TABLE ? (int64_t)p.bias_map[m] * N : 0;
      value = value + p.bias[boff + n];
    }
    if constexpr (GATE != EPI_NONE) {
      const int64_t goff = GATE == EPI_TABLE ? (int64_t)p.gate_map[m] * N : 0;
      const float branch = round_through<M5K_BF16>(value);
      const float res = bf16_bits_to_f32(p.residual[idx]);
      const float g = bf16_bits_to_f32(p.gate[goff + n]);
      store_elem<M5K_BF16>(p.c, idx, res + branch * g);
    } else {
      store_elem<OUT_DT>(p.c, idx, value);
    }
  }
}

template <int OUT_DT, int BIAS, int GATE>
int launch_splitk(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k, const EpiParams& p,
                  int splits, int32_t* workspace, hipStream_t st, const char* name) {
  const int64_t kt_total = k_stages(k);
  const int64_t per = (kt_total + splits - 1) / splits;
  const int used = static_cast<int>((kt_total + per - 1) / per);  // no empty split
  // 256 x 64 tiles (K <= 8192) or 256 x 128 tiles when their workgroups fit in one round, so
  // a few K ranges fill the chip and the INT32 partials (splits x M x N) stay small next to the
  // weights streamed.  Measured against 256 x 256 tiles with the split count sized to each:
  // 256 x 64 1.4-1.6x faster at K 4096-5376 (M 1-256), equal at K 16384 and 5% slower at K
  // 14336, hence its K limit; 256 x 128 1.15-1.23x faster where 256 x 64 does not fit (N 14336,
  // or K 14336-16384); at M 384-1024 the narrower tiles were 1.1-1.45x faster.
  const int cus = device_cus();
  auto fits = [&](int width) {
    return cus > 0 && ((m + BM - 1) / BM) * ((n + width - 1) / width) * used <= static_cast<int64_t>(cus);
  };
  const int tn = k <= 8192 && fits(Grid8Skinny::TN) ? Grid8Skinny::TN : fits(HalfGrid::TN) ? HalfGrid::TN : BN;
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + tn - 1) / tn);
  M5K_REQUIRE(tiles * used <= 0x7FFFFFFF, "%s: too many workgroups", name);
  const dim3 wgs(static_cast<unsigned>(tiles * used)), block(KernelGrid::THREADS);
  auto* A = reinterpret_cast<const uint8_t*>(a);
  auto* B = reinterpret_cast<const uint8_t*>(b);
  if (tn == Grid8Skinny::TN)
    gemm_splitk_kernel<I8, Grid8Skinny><<<wgs, block, 0, st>>>(A, B, (int)m, (int)n, k, used, per, workspace);
  else if (tn == HalfGrid::TN)
    gemm_splitk_kernel<I8, HalfGrid><<<wgs, block, 0, st>>>(A, B, (int)m, (int)n, k, used, per, workspace);
  else
    gemm_splitk_kernel<I8><<<wgs, block, 0, st>>>(A, B, (int)m, (int)n, k, used, per, workspace);
  if (int rc = launch_status(name)) return rc;
  const int64_t blocks = (m * n + 255) / 256;
  const unsigned grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
  splitk_epilogue_kernel<OUT_DT, BIAS, GATE><<<dim3(grid), dim3(256), 0, st>>>(workspace, used, (int)m, (int)n, p);
  return launch_status(name);
}

template <int OUT_DT>
int launch_i8_splitk(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k, const EpiParams& p,
                     int splits, int32_t* workspace, hipStream_t st, const char* name) {
  if (p.bias) {
    return p.bias_map ? launch_splitk<OUT_DT, EPI_TABLE, EPI_NONE>(a, b, m, n, k, p, splits, workspace, st, name)
                      : launch_splitk<OUT_DT, EPI_VECTOR, EPI_NONE>(a, b, m, n, k, p, splits, workspace, st, name);
  }
  if (p.residual) {
    return p.gate_map ? launch_splitk<M5K_BF16, EPI_NONE, EPI_TABLE>(a, b, m, n, k, p, splits, workspace, st, name)
                      : launch_splitk<M5K_BF16, EPI_NONE, EPI_VECTOR>(a, b, m, n, k, p, splits, workspace, st, name);
  }
  return launch_splitk<OUT_DT, EPI_NONE, EPI_NONE>(a, b, m, n, k, p, splits, workspace, st, name);
}

// FP8 split-K: FP32 partial tiles, summed in split order by the same epilogue kernel.  The
// 256 x 64 tile's waves hold two 16-row blocks, fewer than FP8's stage schedule takes, so the
// split tiles are 256 x 128 where their workgroups fit in one round, else 256 x 256.  Each K
// range is its own FP32 accumulation, so the output can differ from the unsplit launch in the
// last bits of the FP32 sum (FP8's accumulation order is not pinned); it is deterministic.
template <int OUT_DT>
int launch_f8_splitk(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k, const EpiParams& p,
                     int splits, float* workspace, hipStream_t st, const char* name) {
  const int64_t kt_total = k_stages(k);
  const int64_t per = (kt_total + splits - 1) / splits;
  const int used = static_cast<int>((kt_total + per - 1) / per);  // no empty split
  const int cus = device_cus();
  const bool half = cus > 0 && ((m + BM - 1) / BM) * ((n + HalfGrid::TN - 1) / HalfGrid::TN) * used <= cus;
  const int tn = half ? HalfGrid::TN : BN;
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + tn - 1) / tn);
  M5K_REQUIRE(tiles * used <= 0x7FFFFFFF, "%s: too many workgroups", name);
  const dim3 wgs(static_cast<unsigned>(tiles * used)), block(KernelGrid::THREADS);
  if (half)
    gemm_splitk_kernel<F8, HalfGrid, float><<<wgs, block, 0, st>>>(a, b, (int)m, (int)n, k, used, per, workspace);
  else
    gemm_splitk_kernel<F8, KernelGrid, float><<<wgs, block, 0, st>>>(a, b, (int)m, (int)n, k, used, per, workspace);
  if (int rc = launch_status(name)) return rc;
  const int64_t blocks = (m * n + 255) / 256;
  const unsigned grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
  splitk_epilogue_kernel<OUT_DT, EPI_NONE, EPI_NONE, float>
      <<<dim3(grid), dim3(256), 0, st>>>(workspace, used, (int)m, (int)n, p);
  return launch_status(name);
}

inline int check_shape(int64_t m, int64_t n, int64_t k, const char* name) {
  M5K_REQUIRE(m > 0 && n > 0 && k > 0, "%s: empty shape m=%lld n=%lld k=%lld", name, (long long)m,
              (long long)n, (long long)k);
  M5K_REQUIRE(m <= 0x7FFFFFFF && n <= 0x7FFFFFFF, "%s: m or n exceeds int32", name);
  return M5K_OK;
}

template <int MODE, int OUT_DT>
int launch_plain(const void* a, const void* b, int64_t m, int64_t n, int64_t k, const EpiParams& p,
                 hipStream_t st, const char* name) {
  if (p.residual) {
    return p.gate_map ? launch<MODE, M5K_BF16, EPI_NONE, EPI_TABLE, false>(a, b, m, n, k, p, st, name)
                      : launch<MODE, M5K_BF16, EPI_NONE, EPI_VECTOR, false>(a, b, m, n, k, p, st, name);
  }
  return launch<MODE, OUT_DT, EPI_NONE, EPI_NONE, false>(a, b, m, n, k, p, st, name);
}

template <int OUT_DT>
int launch_i8(const void* a, const void* b, int64_t m, int64_t n, int64_t k, const EpiParams& p,
              hipStream_t st) {
  const char* name = "m5k_gemm_i8";
  if (p.bias) {
    return p.bias_map ? launch<I8, OUT_DT, EPI_TABLE, EPI_NONE, false>(a, b, m, n, k, p, st, name)
                      : launch<I8, OUT_DT, EPI_VECTOR, EPI_NONE, false>(a, b, m, n, k, p, st, name);
  }
  return launch_plain<I8, OUT_DT>(a, b, m, n, k, p, st, name);
}

}  // namespace detail
}  // namespace gemm
}  // namespace m5k

