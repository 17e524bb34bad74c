// HBM streaming ceiling for a row kernel's traffic mix (diagnostic library libm5k_diag.so; not
// part of the C ABI in include/m5k.h and not used by any op).
//
// The kernel moves the bytes of a row kernel and does nothing else: it reads one or two input
// arrays of `n16` 16-byte chunks and writes an optional full-size output (16 bytes per chunk, the
// residual update R_next or an FP32-to-BF16 stand-in) and an optional half-size output (8 bytes
// per chunk, the INT8 codes of BF16 input).  Each output word is an XOR of the input words, so no
// load or store can be dropped.  Read once, written once, 16-byte vector accesses, a grid-stride
// loop over 4 chunks per thread per step with every load issued before the first store; plain,
// or with non-temporal stores (and loads).  Timed
// over independent input sets, it gives the streaming rate that the same read/write mix reaches
// with no compute, against which the row kernels' streaming rates are read.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// POLICY 0: plain loads and stores; 1: non-temporal stores; 2: non-temporal loads and stores.
template <int POLICY>
__device__ __forceinline__ uint4 load16(const uint4* p) {
  if constexpr (POLICY == 2) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *p;
  }
}
template <int POLICY>
__device__ __forceinline__ void store16(uint4* p, uint4 v) {
  if constexpr (POLICY >= 1) __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
  else *p = v;
}
template <int POLICY>
__device__ __forceinline__ void store8(uint2* p, uint2 v) {
  if constexpr (POLICY >= 1) __builtin_nontemporal_store(u32x2{v.x, v.y}, reinterpret_cast<u32x2*>(p));
  else *p = v;
}

template <int POLICY>
__global__ __launch_bounds__(kThreads) void stream_mix_kernel(const uint4* __restrict__ in0,
                                                               const uint4* __restrict__ in1,
                                                               uint4* __restrict__ out_full,
                                                               uint2* __restrict__ out_half, int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x; base < n16;
       base += stride * kUnroll) {
    uint4 a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = base + static_cast<int64_t>(u) * kThreads;
      a[u] = c < n16 ? load16<POLICY>(in0 + c) : make_uint4(0, 0, 0, 0);
      b[u] = (in1 != nullptr && c < n16) ? load16<POLICY>(in1 + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = base + static_cast<int64_t>(u) * kThreads;
      if (c >= n16) continue;
      const uint4 r = make_uint4(a[u].x ^ b[u].x, a[u].y ^ b[u].y, a[u].z ^ b[u].z, a[u].w ^ b[u].w);
      if (out_full != nullptr) store16<POLICY>(out_full + c, r);
      if (out_half != nullptr) store8<POLICY>(out_half + c, make_uint2(r.x ^ r.y, r.z ^ r.w));
    }
  }
}

}  // namespace

// in0 (required) and in1 (optional) hold n16 16-byte chunks; out_full (optional) n16 chunks,
// out_half (optional) n16 8-byte chunks.  grid_blocks > 0 workgroups of 256 threads; policy 0
// (plain), 1 (non-temporal stores) or 2 (non-temporal loads and stores).  Returns 0 or a HIP
// error code (1 for invalid arguments).
extern "C" int m5k_diag_stream_mix(const void* in0, const void* in1, void* out_full, void* out_half, int64_t n16,
                                   int grid_blocks, int policy, void* stream) {
  if (!in0 || n16 <= 0 || grid_blocks <= 0 || (!out_full && !out_half) || policy < 0 || policy > 2) return 1;
  const dim3 grid(static_cast<unsigned>(grid_blocks)), block(kThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* a = static_cast<const uint4*>(in0);
  const auto* b = static_cast<const uint4*>(in1);
  auto* full = static_cast<uint4*>(out_full);
  auto* half = static_cast<uint2*>(out_half);
  if (policy == 0) stream_mix_kernel<0><<<grid, block, 0, st>>>(a, b, full, half, n16);
  else if (policy == 1) stream_mix_kernel<1><<<grid, block, 0, st>>>(a, b, full, half, n16);
  else stream_mix_kernel<2><<<grid, block, 0, st>>>(a, b, full, half, n16);
  return static_cast<int>(hipGetLastError());
}
