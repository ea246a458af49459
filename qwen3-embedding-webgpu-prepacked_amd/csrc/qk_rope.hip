// qk_rope.hip -- the attention path's producer and the synthetic-input generator.
//
// qk_norm_rope_kernel restates the reference's QK-norm + RoPE shader (src/webgpu/ops.ts:104-150)
// for packed varlen rows: per 128-wide head vector, RMSNorm (eps, optional gain), then NeoX
// rotate-half RoPE (rot[d] = d < 64 ? -n[d+64] : n[d-64]) with the host-built cos/sin table of
// model.ts:76-81.  Positions restart at every sequence boundary (the reference used
// token % sequence, ops.ts:146, which is the same thing for its padded layout).  It computes
// in f64 with a fixed summation order so the result is reproducible bit for bit on any
// device; one thread owns one head vector (this kernel is not on the timed path).
//
// fill_normal_kernel draws N(0,1) fp16 values from a counter-based SplitMix64 stream
// (Box-Muller on output pairs) so the GPU can generate 28 layers of Q/K/V in HBM quickly.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qattn {

typedef _Float16 half_t;

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

__global__ void qk_norm_rope_kernel(half_t* x, int64_t row_stride, int64_t col0, int heads,
                                    const int32_t* cu, int nseq, const float* weight, double eps,
                                    const float* rope_cos, const float* rope_sin) {
  const int64_t T = cu[nseq];
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * heads) return;
  const int64_t t = idx / heads;
  const int h = (int)(idx % heads);
  int lo = 0, hi = nseq - 1;  // sequence holding token t
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int64_t pos = t - cu[lo];
  half_t* v = x + t * row_stride + col0 + (int64_t)h * 128;
  double ss = 0.0;
  for (int d = 0; d < 128; ++d) {
    const double xd = (double)(float)v[d];
    ss = ss + xd * xd;  // products of halves are exact in f64; fixed order
  }
  const double inv = 1.0 / sqrt(ss / 128.0 + eps);
  float n[128];
  for (int d = 0; d < 128; ++d) {
    const double w = weight ? (double)weight[d] : 1.0;
    n[d] = (float)(((double)(float)v[d] * inv) * w);
  }
  for (int d = 0; d < 128; ++d) {
    const int i = d & 63;
    const float rot = d < 64 ? -n[d + 64] : n[d - 64];
    // Both products are exact in f64, so fused or unfused evaluation rounds identically.
    const double r = (double)n[d] * (double)rope_cos[pos * 64 + i] +
                     (double)rot * (double)rope_sin[pos * 64 + i];
    v[d] = to_half((float)r);
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

hipError_t launch_qk_norm_rope(half_t* x, int64_t row_stride, int64_t col0, int heads,
                               const int32_t* cu_dev, int nseq, int64_t T, const float* weight,
                               double eps, const float* rope_cos, const float* rope_sin,
                               hipStream_t stream) {
  const int64_t n = T * heads;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, stream,
                     x, row_stride, col0, heads, cu_dev, nseq, weight, eps, rope_cos, rope_sin);
  return hipGetLastError();
}

}  // namespace qattn
