// qk_rope.hip -- the attention path's producer and the synthetic-input generator.
//
// qk_norm_rope_kernel restates the reference's QK-norm + RoPE shader (src/webgpu/ops.ts:104-150)
// for packed varlen rows: per 128-wide head vector, RMSNorm (eps, optional gain), then NeoX
// rotate-half RoPE (rot[d] = d < 64 ? -n[d+64] : n[d-64]) with the host-built cos/sin table of
// model.ts:76-81.  Positions restart at every sequence boundary (the reference used
// token % sequence, ops.ts:146, which is the same thing for its padded layout).  f32 arithmetic
// as the reference's; it either rewrites a block of heads in place or reads the Q and K blocks
// of a qkvRaw row and writes compact Q and K, as the reference's producer does.
//
// fill_normal_kernel draws N(0,1) fp16 values from a counter-based SplitMix64 stream
// (Box-Muller on output pairs) so the GPU can generate 28 layers of Q/K/V in HBM quickly.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qk_rope.h"

namespace qattn {

__device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

__device__ inline uint64_t rand_u64(uint64_t seed, uint64_t i) {
  return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

// Round-to-nearest-even f32 -> f16 through the hardware conversion (v_cvt_f16_f32 is RNE).
__device__ inline half_t to_half(float x) { return (half_t)x; }

__global__ void fill_normal_kernel(half_t* dst, int64_t rows, int64_t row_elems,
                                   int64_t row_stride, uint64_t seed) {
  const int64_t npairs = (rows * row_elems + 1) / 2;
  const int64_t total = rows * row_elems;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < npairs;
       j += (int64_t)gridDim.x * blockDim.x) {
    const double u1 = (double)((rand_u64(seed, 2 * j) >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(rand_u64(seed, 2 * j + 1) >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double th = 6.283185307179586 * u2;
    double s, c;
    sincos(th, &s, &c);
    const int64_t e0 = 2 * j, e1 = 2 * j + 1;
    dst[(e0 / row_elems) * row_stride + (e0 % row_elems)] = to_half((float)(r * c));
    if (e1 < total) dst[(e1 / row_elems) * row_stride + (e1 % row_elems)] = to_half((float)(r * s));
  }
}

// QK RMSNorm + RoPE, f32 (the reference shader's arithmetic, ops.ts:125-147).  One wavefront =
// one token: its head vectors go four at a time to the four 16-lane groups (lane j of a group
// holds elements 8j..8j+7 of its vector: 16-byte loads and stores), every vector's load issued
// before the first is used.  The token's cos/sin row and the gains are read once per lane for
// all its vectors.  The sum of squares is reduced over the 16 lanes by xor-shuffles in a fixed
// order; the rotate-half partner of element d (d +- 64) sits in lane j ^ 8 at the same slot.
// Positions restart at every sequence boundary; the launch covers up to kRopeSeqs sequences whose
// offsets come by value, the token's sequence found by one ballot over them.
template <int ITERS>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
  typedef half_t h8v __attribute__((ext_vector_type(8)));
  const int lane = threadIdx.x & 63, grp = lane >> 4, j = lane & 15;
  const int t = a.cu[0] + (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= a.cu[a.nseq]) return;
  // Sequence of token t: the number of sequences that end at or before it (the ends are read
  // first, counted after the row's loads are issued).
  const int end = lane < a.nseq ? a.cu[lane + 1] : 0x7fffffff;
  h8v x[ITERS];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int h = 4 * it + grp;
    const bool isq = h < a.split;
    x[it] = *reinterpret_cast<const h8v*>(a.in + (int64_t)t * a.in_stride + (isq ? a.in_col_q : a.in_col_k) +
                                          (isq ? h : h - a.split) * 128 + 8 * j);
  }
  float4 wq[2] = {{1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}}, wk[2] = {wq[0], wq[1]};
  if (a.weight_q) {
    wq[0] = reinterpret_cast<const float4*>(a.weight_q)[2 * j];
    wq[1] = reinterpret_cast<const float4*>(a.weight_q)[2 * j + 1];
  }
  if (a.weight_k) {
    wk[0] = reinterpret_cast<const float4*>(a.weight_k)[2 * j];
    wk[1] = reinterpret_cast<const float4*>(a.weight_k)[2 * j + 1];
  }
  const int s = __popcll(__ballot(end <= t));
  const int pos = t - a.cu[s];
  const float4* cs = reinterpret_cast<const float4*>(a.rope + (int64_t)pos * 64 + 8 * (j & 7));
  float4 c4[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) c4[e] = cs[e];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int h = 4 * it + grp;
    const bool isq = h < a.split;
    float v[8], ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (float)x[it][e];
      ss = fmaf(v[e], v[e], ss);
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 16);
    const float inv = __frsqrt_rn(ss / 128.0f + a.eps);
    float n[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float4 g = isq ? wq[e >> 2] : wk[e >> 2];
      n[e] = v[e] * inv * ((e & 3) == 0 ? g.x : (e & 3) == 1 ? g.y : (e & 3) == 2 ? g.z : g.w);
    }
    h8v r;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float4 c = c4[e >> 1];  // (cos, sin) of slots e and e+1
      const float p0 = __shfl_xor(n[e], 8, 16), p1 = __shfl_xor(n[e + 1], 8, 16);
      const float rot0 = j < 8 ? -p0 : p0, rot1 = j < 8 ? -p1 : p1;
      r[e] = (half_t)(n[e] * c.x + rot0 * c.y);
      r[e + 1] = (half_t)(n[e + 1] * c.z + rot1 * c.w);
    }
    half_t* dst = isq ? a.out_q + (int64_t)t * a.out_stride_q + h * 128
                      : a.out_k + (int64_t)t * a.out_stride_k + (h - a.split) * 128;
    *reinterpret_cast<h8v*>(dst + 8 * j) = r;
  }
}

// Row r of dst gets N(0,1) draws keyed by the token id ids[r]: element c is draw c of the
// stream seeded with seed + ids[r] * 0xD1B54A32D192ED03 (same pairing as fill_normal_kernel).
__global__ void fill_token_rows_kernel(half_t* dst, const int32_t* ids, int64_t rows,
                                       int64_t row_elems, int64_t row_stride, uint64_t seed) {
  const int64_t pairs_per_row = (row_elems + 1) / 2;
  const int64_t total = rows * pairs_per_row;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = g / pairs_per_row, j = g % pairs_per_row;
    const uint64_t s = seed + (uint64_t)(uint32_t)ids[r] * 0xD1B54A32D192ED03ULL;
    const double u1 = (double)((rand_u64(s, 2 * j) >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(rand_u64(s, 2 * j + 1) >> 11) * 0x1.0p-53;
    const double rr = sqrt(-2.0 * log(u1));
    double sn, cs;
    sincos(6.283185307179586 * u2, &sn, &cs);
    dst[r * row_stride + 2 * j] = to_half((float)(rr * cs));
    if (2 * j + 1 < row_elems) dst[r * row_stride + 2 * j + 1] = to_half((float)(rr * sn));
  }
}

hipError_t launch_fill_token_rows(half_t* dst, const int32_t* ids, int64_t rows, int64_t row_elems,
                                  int64_t row_stride, uint64_t seed, hipStream_t stream) {
  const int64_t total = rows * ((row_elems + 1) / 2);
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_token_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, dst, ids,
                     rows, row_elems, row_stride, seed);
  return hipGetLastError();
}

hipError_t launch_fill_normal(half_t* dst, int64_t rows, int64_t row_elems, int64_t row_stride,
                              uint64_t seed, hipStream_t stream) {
  const int64_t npairs = (rows * row_elems + 1) / 2;
  if (npairs <= 0) return hipSuccess;
  int64_t blocks = (npairs + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, dst, rows,
                     row_elems, row_stride, seed);
  return hipGetLastError();
}

// One launch per kRopeSeqs sequences, one wavefront per token; a.heads (a multiple of 4, at most
// kRopeMaxHeads) picks the instantiation.  cu: host copy of the nseq + 1 offsets.
hipError_t launch_qk_norm_rope(RopeArgs a, const int32_t* cu, int nseq, hipStream_t stream) {
  if (a.heads < 4 || a.heads % 4 || a.heads > kRopeMaxHeads || a.split % 4) return hipErrorInvalidValue;
  for (int s0 = 0; s0 < nseq; s0 += kRopeSeqs) {
    const int n = nseq - s0 < kRopeSeqs ? nseq - s0 : kRopeSeqs;
    a.nseq = n;
    for (int i = 0; i <= n; ++i) a.cu[i] = cu[s0 + i];
    const int64_t tokens = (int64_t)cu[s0 + n] - cu[s0];
    if (tokens <= 0) continue;
    const dim3 grid((unsigned)((tokens + 3) / 4)), block(256);
    switch (a.heads / 4) {
      case 1: hipLaunchKernelGGL(qk_norm_rope_kernel<1>, grid, block, 0, stream, a); break;
      case 2: hipLaunchKernelGGL(qk_norm_rope_kernel<2>, grid, block, 0, stream, a); break;
      case 3: hipLaunchKernelGGL(qk_norm_rope_kernel<3>, grid, block, 0, stream, a); break;
      case 4: hipLaunchKernelGGL(qk_norm_rope_kernel<4>, grid, block, 0, stream, a); break;
      case 5: hipLaunchKernelGGL(qk_norm_rope_kernel<5>, grid, block, 0, stream, a); break;
      case 6: hipLaunchKernelGGL(qk_norm_rope_kernel<6>, grid, block, 0, stream, a); break;
      case 7: hipLaunchKernelGGL(qk_norm_rope_kernel<7>, grid, block, 0, stream, a); break;
      default: hipLaunchKernelGGL(qk_norm_rope_kernel<8>, grid, block, 0, stream, a); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace qattn
