// Q/K projection + per-head RMSNorm + split-half RoPE with head-major BF16 output.
//
// Contract: qk_rope.py:120-203 with the arithmetic of shaders/qk_rope_projection.metal:26-33
// and shaders/qk_rope_body.metal:1-20.  For one row m and head h (128 channels):
//   z[d]  = bf16(projection)            INT8: bf16((float(acc) * sa[m]) * sb[n]);  BF16: bf16(acc)
//   inv   = 1 / sqrt(sum_d z[d]^2 / 128 + eps)
//   u[d]  = (z[d] * inv) * gamma[d]
//   d < R:      y[d] = u[d] * c[j] - u[d+R] * s[j]      (j = d)
//   R <= d < 2R: y[d] = u[d] * c[j] + u[d-R] * s[j]     (j = d - R)
//   d >= 2R:    y[d] = u[d]
//   Y[h, m, d] = bf16(y[d]);  c, s = cos/sin[m, j] (bf16)
// Every product and sum is a separate FP32 operation (the library is built without FMA
// contraction).
//
// The fused kernel runs the GEMM main loop for a 256-row x 2-head tile, stages the BF16
// projection in the (then free) LDS, and normalizes each (row, head) with a group
// of 16 lanes (8 channels each, one 16-byte read and one 16-byte head-major store per lane).
// The staged kernel runs the same per-(row, head) routine on a BF16 [M,N] projection in HBM,
// so the two paths agree bit for bit whenever their projections do.
#include "gemm_launch.h"

namespace m5k {
namespace qk {
namespace {

using namespace m5k::gemm;
using m5k::gemm::detail::KernelGrid;

constexpr int HEAD = 128;

struct QkParams {
  const uint16_t* gamma;  // bf16 [128] (Q gamma in the grouped layout)
  const uint16_t* cos;    // bf16 [M, R]
  const uint16_t* sin;    // bf16 [M, R]
  int rope_half;          // R in [0, 64]
  float eps;
  uint16_t* y;            // bf16 [N/128, M, 128] (Q output in the grouped layout)
  // Grouped Q/K/V layout: weight rows [heads, 3, 128]; 128-column block c is head c / 3,
  // stream c % 3 (0 = Q, 1 = K, 2 = V).  V is the BF16 projection itself.
  int grouped;
  const uint16_t* k_gamma;  // bf16 [128]
  uint16_t* k_out;          // bf16 [heads, M, 128]
  uint16_t* v_out;          // bf16 [heads, M, 128]
};

// Destination of 128-column block `block`: head index, output tensor and gamma (nullptr for V).
struct BlockDst {
  int head;
  uint16_t* out;
  const uint16_t* gamma;
};

__device__ __forceinline__ BlockDst block_dst(const QkParams& p, int block) {
  if (!p.grouped) return BlockDst{block, p.y, p.gamma};
  const int head = block / 3, stream = block - 3 * head;
  return stream == 0 ? BlockDst{head, p.y, p.gamma}
         : stream == 1 ? BlockDst{head, p.k_out, p.k_gamma}
                       : BlockDst{head, p.v_out, nullptr};
}

// Normalize + rotate one (row, head).  lg in [0,16) owns channels [8 lg, 8 lg + 8); z holds
// them; partner(d) returns channel d of the same (row, head).  All 16 lanes of the group must
// call together (width-16 exchanges).
template <class Partner>
__device__ __forceinline__ void norm_rope_16(const float (&z)[8], Partner partner, const QkParams& p, int64_t row,
                                             int64_t m_rows, int head, int lg) {
  float ss = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) ss += z[t] * z[t];
  ss += __shfl_xor(ss, 1, 16);
  ss += __shfl_xor(ss, 2, 16);
  ss += __shfl_xor(ss, 4, 16);
  ss += __shfl_xor(ss, 8, 16);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(HEAD) + p.eps);
  const int R = p.rope_half;
  const uint16_t* crow = p.cos + row * R;
  const uint16_t* srow = p.sin + row * R;
  uint32_t packed[4];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int d = 8 * lg + t;
    float v = (z[t] * inv) * bf16_bits_to_f32(p.gamma[d]);
    if (d < 2 * R) {
      const bool lower = d < R;
      const int pair = lower ? d + R : d - R;
      const int j = lower ? d : d - R;
      const float pv = (partner(pair) * inv) * bf16_bits_to_f32(p.gamma[pair]);
      const float c = bf16_bits_to_f32(crow[j]), s = bf16_bits_to_f32(srow[j]);
      v = lower ? (v * c) - (pv * s) : (v * c) + (pv * s);
    }
    const uint32_t bits = f32_to_bf16_bits(v);
    if (t & 1) packed[t >> 1] |= bits << 16;
    else packed[t >> 1] = bits;
  }
  uint16_t* out = p.y + (static_cast<int64_t>(head) * m_rows + row) * HEAD + 8 * lg;
  store_stream16(out, make_uint4(packed[0], packed[1], packed[2], packed[3]));
}

// Fast path for rope_half % 8 == 0 (R = 48 and 64 included): a lane's 8 channels are either
// all rotated-lower (d < R), all rotated-upper (R <= d < 2R) or all unrotated, the partner of
// channel d lives on lane lg +- R/8 at the same register index, and cos/sin of the lane's
// channels are 8 consecutive BF16 values (one 16-byte load each).  u[d] is computed once by
// its owner and fetched by the partner lane: the same FP32 expression as norm_rope_16, so the
// two paths give identical bits.
struct LaneRope {
  float gam[8];  // gamma of the lane's channels
  int src;       // partner lane within the 16-lane group
  bool rot, lower;
  float sgn;     // -1 for the lower half of the rotated channels, else +1
};

__device__ __forceinline__ LaneRope lane_rope(const QkParams& p, const uint16_t* gamma, int lg) {
  LaneRope r;
  const uint4 g = *reinterpret_cast<const uint4*>(gamma + 8 * lg);
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    r.gam[2 * t] = __uint_as_float(gw[t] << 16);
    r.gam[2 * t + 1] = __uint_as_float(gw[t] & 0xFFFF0000u);
  }
  const int R = p.rope_half, d0 = 8 * lg;
  r.rot = d0 < 2 * R;
  r.lower = d0 < R;
  r.src = !r.rot ? lg : r.lower ? lg + R / 8 : lg - R / 8;
  r.sgn = r.lower ? -1.0f : 1.0f;
  return r;
}

// cos and sin of the lane's 8 channels for `row` (zeros for unrotated lanes).
__device__ __forceinline__ void lane_cos_sin(const QkParams& p, const LaneRope& r, int64_t row, int lg, uint4& c,
                                             uint4& s) {
  if (r.rot) {
    const int j0 = r.lower ? 8 * lg : 8 * lg - p.rope_half;
    const int64_t off = row * p.rope_half + j0;
    c = *reinterpret_cast<const uint4*>(p.cos + off);
    s = *reinterpret_cast<const uint4*>(p.sin + off);
  } else {
    c = make_uint4(0, 0, 0, 0);
    s = make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void unpack8_bf16(const uint4& w, float (&v)[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    v[2 * t] = __uint_as_float(ws[t] << 16);
    v[2 * t + 1] = __uint_as_float(ws[t] & 0xFFFF0000u);
  }
}

// Sum over each 16-lane row, the same pairings as xor butterflies 1, 2, 4, 8: quad_perm
// [1,0,3,2] and [2,3,0,1] are xor 1 and 2; after them every lane of a quad holds the same bits,
// so row_half_mirror (lane i <- 7 - i) adds the same quad as xor 4 and row_mirror (lane
// i <- 15 - i) the same half-row as xor 8.  The sums commute, so all 16 lanes end with the
// bits the xor butterflies give.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x141>(v);
  v += dpp_move<0x140>(v);
  return v;
}

// Sum of squares of one (row, head) held as z[8] per lane of its 16-lane group, in every lane.
__device__ __forceinline__ float head_sumsq(const float (&z)[8]) {
  float ss = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) ss += z[t] * z[t];
  return row16_sum(ss);
}

__device__ __forceinline__ float head_inv(float ss, float eps) {
  return 1.0f / sqrtf(ss / static_cast<float>(HEAD) + eps);
}

// Lane k's value of each 16-lane row (row_newbcast:k), for k known after unrolling.
__device__ __forceinline__ float row16_bcast(float v, int k) {
  switch (k) {
    case 0: return dpp_move<0x150>(v);
    case 1: return dpp_move<0x151>(v);
    case 2: return dpp_move<0x152>(v);
    case 3: return dpp_move<0x153>(v);
    case 4: return dpp_move<0x154>(v);
    case 5: return dpp_move<0x155>(v);
    case 6: return dpp_move<0x156>(v);
    case 7: return dpp_move<0x157>(v);
    case 8: return dpp_move<0x158>(v);
    case 9: return dpp_move<0x159>(v);
    case 10: return dpp_move<0x15A>(v);
    case 11: return dpp_move<0x15B>(v);
    case 12: return dpp_move<0x15C>(v);
    case 13: return dpp_move<0x15D>(v);
    case 14: return dpp_move<0x15E>(v);
    default: return dpp_move<0x15F>(v);
  }
}

// Normalize (by the head's inverse RMS `inv`) and rotate one (row, head) held as z[8] per
// lane; returns the packed BF16 output.  HALF8: rope_half == 64, every partner lane is lg ^ 8
// (one row_ror:8 DPP move).
template <bool HALF8>
__device__ __forceinline__ uint4 rope_apply(const float (&z)[8], const LaneRope& r, const uint4& cw,
                                            const uint4& sw, float inv) {
  float u[8], c[8], s[8];
  unpack8_bf16(cw, c);
  unpack8_bf16(sw, s);
#pragma unroll
  for (int t = 0; t < 8; ++t) u[t] = (z[t] * inv) * r.gam[t];
  // All partner values first, then branch-free arithmetic: fma(-+1, b, a) is the single
  // rounding of a - b (lower half) or a + b (upper half), the same bits as the subtract or add.
  float pu[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) pu[t] = HALF8 ? dpp_move<0x128>(u[t]) : __shfl(u[t], r.src, 16);
  // With rope_half == 64 every channel of a 128-wide head is rotated (8 lg < 128), so only the
  // general layout keeps the unrotated lanes' values.
  float y[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float rotated = __builtin_fmaf(r.sgn, pu[t] * s[t], u[t] * c[t]);
    y[t] = HALF8 || r.rot ? rotated : u[t];
  }
  return make_uint4(f32x2_to_bf16x2(y[0], y[1]), f32x2_to_bf16x2(y[2], y[3]), f32x2_to_bf16x2(y[4], y[5]),
                    f32x2_to_bf16x2(y[6], y[7]));
}

template <bool HALF8>
__device__ __forceinline__ uint4 norm_rope_fast(const float (&z)[8], const LaneRope& r, const uint4& cw,
                                                const uint4& sw, float eps) {
  return rope_apply<HALF8>(z, r, cw, sw, head_inv(head_sumsq(z), eps));
}

// Epilogue of one 256 x G::TN projection tile (G::TN = 256: two heads, or 128: one head), called
// by every thread after the main loop: the BF16 projection is staged in the LDS the loop has
// released, then 16-lane groups normalize and rotate (row, head) pairs.
template <int MODE, class G>
__device__ __forceinline__ void qk_tile_epilogue(const AccTile<MODE, G>& acc, int M, int N, int m0, int n0,
                                                 const TileScalePrefetch<G>& pre, const QkParams& p, int fast) {
  static_assert(G::TN % HEAD == 0, "projection tiles hold whole heads");
  constexpr int HPT = G::TN / HEAD;  // heads per tile
  // Everything the epilogue loads depends on the lane index taken here, after the main loop,
  // so no epilogue value is hoisted into the loop's register budget (with the interleaved
  // fragment reads the loop uses 241 of 256 VGPRs).
  int tid_after = threadIdx.x;
  __asm__ volatile("" : "+v"(tid_after));
  const int group = tid_after >> 4, lg = tid_after & 15;
  constexpr int GROUPS = G::THREADS / 16;  // 32 groups of 16 lanes
  constexpr int ROWS_PER_GROUP = BM / GROUPS;
  const int heads_here = min(G::TN, N - n0) / HEAD;  // N is a multiple of 128

  // BF16 projection tile [256 rows][G::TN cols] in LDS (row stride TILE16_STRIDE).  The main
  // loop ended with a drained DMA and a barrier, so the stage ring is free.
  uint16_t* tile = reinterpret_cast<uint16_t*>(g_lds);
  {
    using Geo = AccGeom<MODE, G>;
    const Geo geo(tid_after);
    float cs[Geo::FN];
    const float* sc = nullptr;
    if constexpr (MODE == I8) {
      const TileScales<G> ts(pre, tid_after);
      sc = ts.s;
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j) cs[j] = ts.col(geo.col(j));
    }
#pragma unroll
    for (int i = 0; i < Geo::FM; ++i) {
      float rs[Geo::PER];
      if constexpr (MODE == I8) {
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) rs[e] = sc[geo.row(i, e)];
      }
#pragma unroll
      for (int j = 0; j < Geo::FN; ++j)
#pragma unroll
        for (int e = 0; e < Geo::PER; ++e) {
          // Entries past M or N are staged unmasked: no (row, head) pair reads them.
          const int r = geo.row(i, e), c = geo.col(j);
          float value;
          if constexpr (MODE == I8) value = (static_cast<float>(acc[i][j][e]) * rs[e]) * cs[j];
          else value = acc[i][j][e];
          tile[r * TILE16_STRIDE + c] = static_cast<uint16_t>(f32_to_bf16_bits(value));
        }
    }
  }
  // Fast path: issue the cos/sin loads of the group's first LOOKAHEAD rows once the accumulators
  // are staged (their registers are free then); the barrier below covers their latency, and each
  // later row's loads go out LOOKAHEAD rows ahead of its use.  The pair words are read from the
  // staged tile when needed rather than held.  Holding all eight rows' tables and all sixteen pair
  // words spilled 35 VGPRs to scratch; this form uses 228 VGPRs and no scratch, same bits (C5
  // fused projection 162.6 -> 160.2 us, one box).
  LaneRope lr, lrk;  // Q (or single-projection) gamma; K gamma in the grouped layout
  constexpr int LOOKAHEAD = 4;  // rows of cos/sin in flight ahead of the row being rotated
  uint4 cw[ROWS_PER_GROUP], sw[ROWS_PER_GROUP];
  int row0 = m0 + group;
  __asm__ volatile("" : "+v"(row0));
  auto load_cs = [&](int i) {
    const int row = row0 + GROUPS * i;
    if (row < M) lane_cos_sin(p, lr, row, lg, cw[i], sw[i]);
  };
  if (fast) {
    lr = lane_rope(p, p.gamma, lg);
    if (p.grouped) lrk = lane_rope(p, p.k_gamma, lg);
#pragma unroll
    for (int i = 0; i < LOOKAHEAD; ++i) load_cs(i);
  }

  __syncthreads();

  if (fast) {
    // The group's (row, head) pairs, pair k = HPT i + h, at most one per lane.  A first pass
    // forms every pair's sum of squares and lane k keeps pair k's, so each lane takes one
    // square root and division; the second broadcasts pair k's inverse from lane k.  Pairs of
    // rows past M are read from the staged tile (inside it) and store nothing.
    constexpr int PAIRS = ROWS_PER_GROUP * HPT;
    static_assert(PAIRS <= 16, "one (row, head) pair per lane of the group");
    auto pair_words = [&](int i, int h) {
      return *reinterpret_cast<const uint4*>(tile + (group + GROUPS * i) * TILE16_STRIDE + h * HEAD + 8 * lg);
    };
    float ss_mine = 0.0f;
#pragma unroll
    for (int i = 0; i < ROWS_PER_GROUP; ++i) {
#pragma unroll
      for (int h = 0; h < HPT; ++h) {
        const int k = HPT * i + h;
        float z[8];
        unpack8_bf16(pair_words(i, h), z);
        const float ss = head_sumsq(z);
        ss_mine = lg == k ? ss : ss_mine;
      }
    }
    const float inv_mine = head_inv(ss_mine, p.eps);
#pragma unroll
    for (int i = 0; i < ROWS_PER_GROUP; ++i) {
      if (i + LOOKAHEAD < ROWS_PER_GROUP) load_cs(i + LOOKAHEAD);
      __builtin_amdgcn_sched_barrier(0);
      const int row = m0 + group + GROUPS * i;
      if (row >= M) continue;  // uniform across the 16-lane group
#pragma unroll
      for (int h = 0; h < HPT; ++h) {
        if (h >= heads_here) continue;
        const int k = HPT * i + h;
        const BlockDst d = block_dst(p, n0 / HEAD + h);  // uniform across the group
        uint16_t* dst = d.out + (static_cast<int64_t>(d.head) * M + row) * HEAD + 8 * lg;
        const uint4 wk = pair_words(i, h);
        if (d.gamma == nullptr) {  // V: the rounded projection
          store_stream16(dst, wk);
          continue;
        }
        float z[8];
        unpack8_bf16(wk, z);
        const LaneRope& rr = d.gamma == p.gamma ? lr : lrk;
        const float inv = row16_bcast(inv_mine, k);
        store_stream16(dst, p.rope_half == 64 ? rope_apply<true>(z, rr, cw[i], sw[i], inv)
                                              : rope_apply<false>(z, rr, cw[i], sw[i], inv));
      }
    }
    return;
  }
  for (int q = group; q < BM * HPT; q += GROUPS) {
    const int local_row = q / HPT, local_head = q % HPT;
    const int row = m0 + local_row;
    const int block = n0 / HEAD + local_head;
    if (row >= M || block * HEAD >= N) continue;  // uniform across the 16-lane group
    const uint16_t* src = tile + local_row * TILE16_STRIDE + local_head * HEAD;
    const BlockDst d = block_dst(p, block);
    if (d.gamma == nullptr) {
      store_stream16(d.out + (static_cast<int64_t>(d.head) * M + row) * HEAD + 8 * lg,
                     *reinterpret_cast<const uint4*>(src + 8 * lg));
      continue;
    }
    QkParams ps = p;
    ps.gamma = d.gamma;
    ps.y = d.out;
    float z[8];
    unpack8_bf16(*reinterpret_cast<const uint4*>(src + 8 * lg), z);
    norm_rope_16(z, [&](int dd) { return bf16_bits_to_f32(src[dd]); }, ps, row, M, d.head, lg);
  }
}

// The INT8 tile's scales ahead of the main loop (the BF16 projection has none).
template <int MODE, class G>
__device__ __forceinline__ TileScalePrefetch<G> qk_prefetch_scales(const float* __restrict__ sa,
                                                                   const float* __restrict__ sb, int M, int N, int m0,
                                                                   int n0) {
  if constexpr (MODE == I8) return TileScalePrefetch<G>(sa, sb, M, N, m0, n0);
  else return TileScalePrefetch<G>(nullptr, nullptr, 0, 0, 0, 0);
}

template <int MODE, bool ALIGNED>
__global__ __launch_bounds__(KernelGrid::THREADS, 1) void qk_fused_kernel(const uint8_t* __restrict__ A,
                                                                          const uint8_t* __restrict__ B, int M, int N,
                                                                          int64_t Kb, const float* __restrict__ sa,
                                                                          const float* __restrict__ sb, QkParams p,
                                                                          int fast) {
  using G = KernelGrid;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const TileScalePrefetch<G> pre = qk_prefetch_scales<MODE, G>(sa, sb, M, N, m0, n0);
  AccTile<MODE, G> acc;
  if constexpr (ALIGNED) mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, 0, k_stages(Kb));
  else mainloop_staged<MODE, G>(A, B, M, N, Kb, m0, n0, acc);
  qk_tile_epilogue<MODE, G>(acc, M, N, m0, n0, pre, p, fast);
}

// The mixed schedule of the GEMM library (gemm_mixed_kernel) for the fused projection: the
// first `full` tiles of the raster order (whole rounds) as 256 x 256 tiles, every other tile
// as two 256 x 128 halves of one head each, so a partial last round runs as one shorter,
// better-filled round.  Each output is one workgroup's dot product over all of K, so the bits
// equal the plain launch's.
template <int MODE>
__global__ __launch_bounds__(KernelGrid::THREADS, 1) void qk_mixed_kernel(const uint8_t* __restrict__ A,
                                                                          const uint8_t* __restrict__ B, int M, int N,
                                                                          int64_t Kb, int full,
                                                                          const float* __restrict__ sa,
                                                                          const float* __restrict__ sb, QkParams p,
                                                                          int fast) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < full) {
    using G = KernelGrid;
    int tm, tn;
    band_coords(xcd_logical(bid, full), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const TileScalePrefetch<G> pre = qk_prefetch_scales<MODE, G>(sa, sb, M, N, m0, n0);
    AccTile<MODE, G> acc;
    mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, 0, k_stages(Kb));
    qk_tile_epilogue<MODE, G>(acc, M, N, m0, n0, pre, p, fast);
  } else {
    using G = gemm::detail::HalfGrid;
    const int h = xcd_logical(bid - full, 2 * (tiles_m * tiles_n - full));
    int tm, tn;
    band_coords(full + (h >> 1), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN + (h & 1) * G::TN;
    if (n0 >= N) return;  // right half of a last tile column one head wide (whole workgroup)
    const TileScalePrefetch<G> pre = qk_prefetch_scales<MODE, G>(sa, sb, M, N, m0, n0);
    AccTile<MODE, G> acc;
    mainloop_dma<MODE, G>(A, B, M, N, Kb, m0, n0, acc, 0, k_stages(Kb));
    qk_tile_epilogue<MODE, G>(acc, M, N, m0, n0, pre, p, fast);
  }
}

// Staged postprocess of a BF16 [M, N] projection: one 16-lane group per (row, head), consecutive
// groups walking the heads of a row (coalesced 256-byte reads).
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const uint16_t* __restrict__ P, int64_t M, int64_t N,
                                                           QkParams p, int fast) {
  const int64_t heads = N / HEAD;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int lg = threadIdx.x & 15;
  if (q >= M * heads) return;  // whole 16-lane groups leave together
  const int64_t row = q / heads;
  const int head = static_cast<int>(q - row * heads);
  const uint16_t* src = P + row * N + static_cast<int64_t>(head) * HEAD;
  float z[8];
  unpack8_bf16(*reinterpret_cast<const uint4*>(src + 8 * lg), z);
  if (fast) {
    const LaneRope lr = lane_rope(p, p.gamma, lg);
    uint4 cw, sw;
    lane_cos_sin(p, lr, row, lg, cw, sw);
    const uint4 out = p.rope_half == 64 ? norm_rope_fast<true>(z, lr, cw, sw, p.eps)
                                        : norm_rope_fast<false>(z, lr, cw, sw, p.eps);
    store_stream16(p.y + (static_cast<int64_t>(head) * M + row) * HEAD + 8 * lg, out);
    return;
  }
  norm_rope_16(z, [&](int d) { return bf16_bits_to_f32(src[d]); }, p, row, M, head, lg);
}

// The fast path needs whole 8-channel lanes per RoPE half and 16-byte aligned tables.
inline int fast_rope(const QkParams& p) {
  return p.rope_half % 8 == 0 && aligned16(p.gamma) && (!p.grouped || aligned16(p.k_gamma)) &&
         (p.rope_half == 0 || (aligned16(p.cos) && aligned16(p.sin)));
}

template <int MODE>
int launch_fused(const void* a, const void* b, int64_t m, int64_t n, int64_t k, const float* sa, const float* sb,
                 const QkParams& p, hipStream_t st) {
  const int64_t kb = k * Traits<MODE>::elem_bytes;
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  const bool aligned = gemm::detail::dma_ok(a, b, kb);
  const dim3 grid(static_cast<unsigned>(tiles)), block(KernelGrid::THREADS);
  auto* A = static_cast<const uint8_t*>(a);
  auto* B = static_cast<const uint8_t*>(b);
  const int fast = fast_rope(p);
  if (aligned) {
    // The GEMM library's schedule for this output shape; 256 x 224 tiles do not hold whole
    // heads, so the narrow schedule is not offered here.
    int64_t full = -1;
    if (gemm::detail::plan_schedule(false, false, m, n, device_cus(), full) == gemm::detail::SCHED_MIXED) {
      const int64_t wgs = full + 2 * (tiles - full);
      qk_mixed_kernel<MODE><<<dim3(static_cast<unsigned>(wgs)), block, 0, st>>>(A, B, (int)m, (int)n, kb,
                                                                               static_cast<int>(full), sa, sb, p, fast);
    } else {
      qk_fused_kernel<MODE, true><<<grid, block, 0, st>>>(A, B, (int)m, (int)n, kb, sa, sb, p, fast);
    }
  } else {
    qk_fused_kernel<MODE, false><<<grid, block, 0, st>>>(A, B, (int)m, (int)n, kb, sa, sb, p, fast);
  }
  return launch_status("m5k_projection_qk_rope");
}

int check_norm_args(int64_t m, int64_t n, const void* gamma, const void* cos, const void* sin, int rope_half,
                    float epsilon, const void* y, const char* name) {
  M5K_REQUIRE(m > 0 && n > 0 && n % HEAD == 0, "%s: need M > 0 and N a positive multiple of 128", name);
  M5K_REQUIRE(m <= 0x7FFFFFFF && n <= 0x7FFFFFFF, "%s: M or N exceeds int32", name);
  M5K_REQUIRE(gamma && y && (rope_half == 0 || (cos && sin)), "%s: null pointer", name);
  M5K_REQUIRE(rope_half >= 0 && rope_half <= HEAD / 2, "%s: rope_half %d not in [0, 64]", name, rope_half);
  M5K_REQUIRE(epsilon > 0.0f, "%s: epsilon must be positive", name);
  M5K_REQUIRE(aligned16(y), "%s: y must be 16-byte aligned", name);
  return M5K_OK;
}

}  // namespace
}  // namespace qk
}  // namespace m5k

using namespace m5k;
using namespace m5k::qk;

extern "C" int m5k_projection_qk_rope(const void* a, const void* b, int ab_dtype, int64_t m, int64_t n, int64_t k,
                                      const float* a_scales, const float* b_scales, const void* gamma,
                                      const void* cos, const void* sin, int rope_half, float epsilon, void* y,
                                      void* stream) {
  clear_error();
  const char* name = "m5k_projection_qk_rope";
  if (int rc = check_norm_args(m, n, gamma, cos, sin, rope_half, epsilon, y, name)) return rc;
  M5K_REQUIRE(a && b && k > 0, "%s: null operand or empty K", name);
  QkParams p{static_cast<const uint16_t*>(gamma), static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
             rope_half, epsilon, static_cast<uint16_t*>(y), 0, nullptr, nullptr, nullptr};
  hipStream_t st = as_stream(stream);
  if (ab_dtype == M5K_I8) {
    M5K_REQUIRE(a_scales && b_scales, "%s: INT8 needs a_scales and b_scales", name);
    M5K_REQUIRE(k <= 131071, "%s: K exceeds the INT32 worst-case bound 131071", name);
    return launch_fused<I8>(a, b, m, n, k, a_scales, b_scales, p, st);
  }
  M5K_REQUIRE(ab_dtype == M5K_BF16, "%s: operands must be INT8 or BF16", name);
  return launch_fused<BF16>(a, b, m, n, k, nullptr, nullptr, p, st);
}

extern "C" int m5k_qk_norm_rope(const void* projected, int64_t m, int64_t n, const void* gamma, const void* cos,
                                const void* sin, int rope_half, float epsilon, void* y, void* stream) {
  clear_error();
  const char* name = "m5k_qk_norm_rope";
  if (int rc = check_norm_args(m, n, gamma, cos, sin, rope_half, epsilon, y, name)) return rc;
  M5K_REQUIRE(projected && aligned16(projected), "%s: projection must be a 16-byte aligned pointer", name);
  QkParams p{static_cast<const uint16_t*>(gamma), static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
             rope_half, epsilon, static_cast<uint16_t*>(y), 0, nullptr, nullptr, nullptr};
  const int64_t groups = m * (n / HEAD);
  const int64_t blocks = (groups + 15) / 16;
  M5K_REQUIRE(blocks <= 0x7FFFFFFF, "%s: input too large", name);
  qk_norm_rope_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(projected), m, n, p, fast_rope(p));
  return launch_status(name);
}

extern "C" int m5k_projection_qkv_rope(const void* a, const void* b, int ab_dtype, int64_t m, int64_t heads, int64_t k,
                                       const float* a_scales, const float* b_scales, const void* q_gamma,
                                       const void* k_gamma, const void* cos, const void* sin, int rope_half,
                                       float epsilon, void* q_out, void* k_out, void* v_out, void* stream) {
  clear_error();
  const char* name = "m5k_projection_qkv_rope";
  M5K_REQUIRE(heads > 0 && heads * 3 * HEAD <= 0x7FFFFFFF, "%s: bad head count %lld", name, (long long)heads);
  const int64_t n = heads * 3 * HEAD;
  if (int rc = check_norm_args(m, n, q_gamma, cos, sin, rope_half, epsilon, q_out, name)) return rc;
  M5K_REQUIRE(a && b && k > 0 && k_gamma && k_out && v_out, "%s: null pointer or empty K", name);
  M5K_REQUIRE(aligned16(k_out) && aligned16(v_out), "%s: outputs must be 16-byte aligned", name);
  QkParams p{static_cast<const uint16_t*>(q_gamma), static_cast<const uint16_t*>(cos),
             static_cast<const uint16_t*>(sin),     rope_half,
             epsilon,                               static_cast<uint16_t*>(q_out),
             1,                                     static_cast<const uint16_t*>(k_gamma),
             static_cast<uint16_t*>(k_out),         static_cast<uint16_t*>(v_out)};
  hipStream_t st = as_stream(stream);
  if (ab_dtype == M5K_I8) {
    M5K_REQUIRE(a_scales && b_scales, "%s: INT8 needs a_scales and b_scales", name);
    M5K_REQUIRE(k <= 131071, "%s: K exceeds the INT32 worst-case bound 131071", name);
    return launch_fused<I8>(a, b, m, n, k, a_scales, b_scales, p, st);
  }
  M5K_REQUIRE(ab_dtype == M5K_BF16, "%s: operands must be INT8 or BF16", name);
  return launch_fused<BF16>(a, b, m, n, k, nullptr, nullptr, p, st);
}
