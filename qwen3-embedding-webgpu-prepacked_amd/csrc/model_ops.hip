// model_ops.hip -- the row-wise kernels of the Qwen3-Embedding-0.6B forward around the attention
// path: Q6_K token-embedding lookup, residual add + RMSNorm, SwiGLU.  All are HBM-bound
// streaming kernels (a few bytes of arithmetic per byte moved): rows are read and written with
// 16-byte vector accesses, one wavefront (or one thread per 8 columns) per row, no LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_common.h"
#include "model_ops.h"

namespace qattn {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// ---- Q6_K token embedding (EmbeddingLookupKernel, ops.ts:381-423) ------------------------------
// A Q6_K block holds 256 values in 210 bytes: ql[128] (low nibbles), qh[64] (2 high bits each),
// 16 int8 scales, f16 d.  Value i = 128 h + 32 quad + l (h < 2, quad < 4, l < 32) is
//   q = (ql[64 h + l + 32 (quad & 1)] >> (quad >= 2 ? 4 : 0) & 15) | ((qh[32 h + l] >> 2 quad) & 3) << 4
//   value = f16(f32(d) * f32(scales[8 h + l / 16 + 2 quad]) * f32(q - 32))
// (ops.ts:390-401; the CPU decoder quantization.ts:46-70 is the same map).  One thread per 8
// consecutive values (same h, quad, scale), 128 threads per token row of 1024.
__global__ __launch_bounds__(256) void embed_q6k_kernel(const int32_t* ids, int64_t tokens, const uint8_t* table,
                                                         int64_t vocab, int width, half_t* out, int64_t out_stride) {
  const int per_row = width / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * per_row) return;
  const int64_t t = i / per_row;
  const int c0 = (int)(i - t * per_row) * 8;
  const int32_t id = ids[t];
  h8 v;
  if (id < 0 || id >= vocab) {
    // Out-of-range ids (rejected by the plan on the host) give zeros instead of a wild read.
    v = h8{};
  } else {
    const uint8_t* blk = table + ((int64_t)id * (width / 256) + c0 / 256) * kQ6KBlockBytes;
    const int within = c0 & 255, h = within >> 7, pos = within & 127, quad = pos >> 5, l0 = pos & 31;
    const uint8_t* ql = blk + 64 * h + 32 * (quad & 1) + l0;
    const uint8_t* qh = blk + 128 + 32 * h + l0;
    const float scale = (float)(int8_t)blk[192 + 8 * h + l0 / 16 + 2 * quad];
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[208] | (blk[209] << 8)));
    const float ds = d * scale;
    const int lo_shift = quad >= 2 ? 4 : 0, hi_shift = 2 * quad;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int q = ((ql[j] >> lo_shift) & 15) | (((qh[j] >> hi_shift) & 3) << 4);
      v[j] = (_Float16)(ds * (float)(q - 32));
    }
  }
  *reinterpret_cast<h8*>(out + t * out_stride + c0) = v;
}

// ---- residual add + RMSNorm (RmsNormKernel, ops.ts:21-72) -------------------------------------
// One wavefront per row; lane l owns columns 8l + 512j.  With a residual: v = f32(x) + f32(r),
// x <- f16(v) (the residual stream is updated in place, ops.ts:41), and the sum of squares takes
// the unrounded v (ops.ts:42); without: v = f32(x).  normalized = f16(f32(x) * inv * w) with the
// stored (rounded) x and inv = 1 / sqrt(sum / width + eps) (ops.ts:52-55).  residual_at(c) gives
// the residual's 8 values at columns c..c+7 (from memory, or from a projection's split-K sums),
// so both kernels below run the same arithmetic in the same order.
template <bool RESIDUAL, typename ResidualAt>
__device__ inline void rmsnorm_row(half_t* xr, ResidualAt residual_at, const float* weight, half_t* out_row,
                                   int width, float eps, int lane) {
  constexpr int kMaxChunks = kRmsMaxWidth / 512;
  h8 xs[kMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    const int c = 8 * lane + 512 * j;
    if (c < width) {
      h8 a = *reinterpret_cast<const h8*>(xr + c);
      if (RESIDUAL) {
        const h8 b = residual_at(c);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float s = (float)a[e] + (float)b[e];
          ss += s * s;
          a[e] = (_Float16)s;
        }
        *reinterpret_cast<h8*>(xr + c) = a;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)a[e] * (float)a[e];
      }
      xs[j] = a;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float inv = 1.f / sqrtf(ss / (float)width + eps);
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    const int c = 8 * lane + 512 * j;
    if (c < width) {
      const float4 w0 = *reinterpret_cast<const float4*>(weight + c);
      const float4 w1 = *reinterpret_cast<const float4*>(weight + c + 4);
      const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      h8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (_Float16)((float)xs[j][e] * inv * w[e]);
      *reinterpret_cast<h8*>(out_row + c) = o;
    }
  }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(half_t* x, const half_t* residual, const float* weight,
                                                      half_t* out, int64_t rows, int width, int64_t x_stride,
                                                      int64_t r_stride, int64_t out_stride, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  half_t* xr = x + row * x_stride;
  if (residual) {
    const half_t* rr = residual + row * r_stride;
    rmsnorm_row<true>(xr, [&](int c) { return *reinterpret_cast<const h8*>(rr + c); }, weight, out + row * out_stride,
                      width, eps, lane);
  } else {
    rmsnorm_row<false>(xr, [](int) { return h8{}; }, weight, out + row * out_stride, width, eps, lane);
  }
}

// A projection's split-K sums as the residual: r = f16(part[0] + part[1] + ...) in chunk order
// (part: chunks x rows x width fp32, the layout and sums of q4_reduce_kernel), then
// rmsnorm_row as above: bit for bit the projection's output followed by rmsnorm_kernel.
__global__ __launch_bounds__(256) void reduce_rmsnorm_kernel(const float* part, int chunks, half_t* x,
                                                             const float* weight, half_t* out, int64_t rows,
                                                             int width, int64_t x_stride, int64_t out_stride,
                                                             float eps) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const size_t plane = (size_t)rows * (size_t)width;
  const float* pr = part + (size_t)row * width;
  auto sums = [&](int c) {
    f4 s0 = *reinterpret_cast<const f4*>(pr + c), s1 = *reinterpret_cast<const f4*>(pr + c + 4);
    for (int ch = 1; ch < chunks; ++ch) {
      s0 = s0 + *reinterpret_cast<const f4*>(pr + (size_t)ch * plane + c);
      s1 = s1 + *reinterpret_cast<const f4*>(pr + (size_t)ch * plane + c + 4);
    }
    return h8{(_Float16)s0[0], (_Float16)s0[1], (_Float16)s0[2], (_Float16)s0[3],
              (_Float16)s1[0], (_Float16)s1[1], (_Float16)s1[2], (_Float16)s1[3]};
  };
  rmsnorm_row<true>(x + row * x_stride, sums, weight, out + row * out_stride, width, eps, lane);
}

// ---- SwiGLU (SwiGLUKernel, ops.ts:74-102) ------------------------------------------------------
// out[r][c] = f16(silu(g) * u), g = f32(gate_up[r][c]), u = f32(gate_up[r][width + c]),
// silu(g) = g / (1 + exp(-g)) in f32.  One thread per 8 columns.
__global__ __launch_bounds__(256) void swiglu_kernel(const half_t* gate_up, int64_t gu_stride, half_t* out,
                                                     int64_t out_stride, int64_t rows, int width) {
  const int per_row = width / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * per_row) return;
  const int64_t r = i / per_row;
  const int c = (int)(i - r * per_row) * 8;
  const h8 g = *reinterpret_cast<const h8*>(gate_up + r * gu_stride + c);
  const h8 u = *reinterpret_cast<const h8*>(gate_up + r * gu_stride + width + c);
  h8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = swiglu_value(g[e], u[e]);
  *reinterpret_cast<h8*>(out + r * out_stride + c) = o;
}

}  // namespace

hipError_t launch_embed_q6k(const int32_t* ids, int64_t tokens, const uint8_t* table, int64_t vocab, int width,
                            half_t* out, int64_t out_stride, hipStream_t stream) {
  const int64_t threads = tokens * (width / 8);
  if (threads <= 0) return hipSuccess;
  hipLaunchKernelGGL(embed_q6k_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, ids, tokens,
                     table, vocab, width, out, out_stride);
  return hipGetLastError();
}

hipError_t launch_reduce_rmsnorm(const float* part, int chunks, int rows, int width, const RowNorm& norm,
                                 hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(reduce_rmsnorm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, part, chunks,
                     norm.x, norm.weight, norm.out, (int64_t)rows, width, norm.x_stride, norm.out_stride, norm.eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(half_t* x, const half_t* residual, const float* weight, half_t* out, int64_t rows,
                          int width, int64_t x_stride, int64_t r_stride, int64_t out_stride, float eps,
                          hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, residual, weight,
                     out, rows, width, x_stride, r_stride, out_stride, eps);
  return hipGetLastError();
}

hipError_t launch_swiglu(const half_t* gate_up, int64_t gu_stride, half_t* out, int64_t out_stride, int64_t rows,
                         int width, hipStream_t stream) {
  const int64_t threads = rows * (width / 8);
  if (threads <= 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, gate_up,
                     gu_stride, out, out_stride, rows, width);
  return hipGetLastError();
}

}  // namespace qattn
