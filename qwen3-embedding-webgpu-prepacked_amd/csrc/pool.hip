// pool.hip -- last-token pool + L2 normalisation, the consumer of the attention path.
//
// Restates the reference's LastTokenPoolKernel (src/webgpu/ops.ts:347-379): for batch entry b it
// reads row b*S + lengths[b] - 1 of the fp16 hidden state (ops.ts:357), sums the squares in f32
// (ops.ts:358-361), and writes f32(x) * inverseSqrt(sum) (ops.ts:362-363).  Here sequences are
// packed (cu_seqlens), so the row is cu_seqlens[i+1] - 1, and the host passes the rows by value.
//
// One wavefront per sequence (the reference uses a 256-thread workgroup and an LDS tree): each
// lane reads 8 consecutive halves (16 B) per 512-wide chunk, the squares are summed in f32 per
// lane and then across the wave with xor shuffles, and each lane writes its 8 scaled values as two
// 16 B stores.  The whole launch moves nseq * width * 6 bytes: it is latency-bound, not a
// bandwidth or matrix-core problem, so rows up to kPoolRegChunks * 512 wide (the model's 1024 and
// the attention output's 2048) are held in registers: all loads issue at once and the row is read
// once.  Wider rows take a second read for the output pass.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qattn {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPoolMaxRows = 256;   // sequences per launch (rows passed by value)
constexpr int kPoolRegChunks = 8;  // 512-wide chunks held in registers (width <= 4096)

struct PoolRows {
  int32_t row[kPoolMaxRows];  // last row of sequence base + j, or -1 for an empty sequence
};

__global__ __launch_bounds__(64) void pool_last_l2_kernel(const _Float16* __restrict__ x, int64_t row_stride,
                                                          int width, float* __restrict__ out,
                                                          int64_t out_row_stride, int base, PoolRows rows) {
  const int j = blockIdx.x;
  const int lane = threadIdx.x;
  const int r = rows.row[j];
  float* dst = out + (int64_t)(base + j) * out_row_stride;
  if (r < 0) {  // empty sequence: no last token
    for (int c = lane * 8; c < width; c += 512) {
      reinterpret_cast<f4*>(dst + c)[0] = f4{0.f, 0.f, 0.f, 0.f};
      reinterpret_cast<f4*>(dst + c)[1] = f4{0.f, 0.f, 0.f, 0.f};
    }
    return;
  }
  const _Float16* src = x + (int64_t)r * row_stride;
  float sum = 0.f;
  if (width <= kPoolRegChunks * 512) {
    h8 v[kPoolRegChunks];
#pragma unroll
    for (int k = 0; k < kPoolRegChunks; ++k) {
      const int c = lane * 8 + 512 * k;
      v[k] = c < width ? *reinterpret_cast<const h8*>(src + c) : h8{};
    }
#pragma unroll
    for (int k = 0; k < kPoolRegChunks; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) sum = fmaf((float)v[k][e], (float)v[k][e], sum);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float inv = 1.0f / __builtin_sqrtf(sum);  // as below: 0 -> inf -> NaN outputs
#pragma unroll
    for (int k = 0; k < kPoolRegChunks; ++k) {
      const int c = lane * 8 + 512 * k;
      if (c < width) {
        reinterpret_cast<f4*>(dst + c)[0] = f4{(float)v[k][0] * inv, (float)v[k][1] * inv, (float)v[k][2] * inv,
                                               (float)v[k][3] * inv};
        reinterpret_cast<f4*>(dst + c)[1] = f4{(float)v[k][4] * inv, (float)v[k][5] * inv, (float)v[k][6] * inv,
                                               (float)v[k][7] * inv};
      }
    }
    return;
  }
  for (int c = lane * 8; c < width; c += 512) {
    const h8 v = *reinterpret_cast<const h8*>(src + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) sum = fmaf((float)v[e], (float)v[e], sum);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  // inverseSqrt(sum): an all-zero row gives inf and 0 * inf = NaN, as in the reference.
  const float inv = 1.0f / __builtin_sqrtf(sum);
  for (int c = lane * 8; c < width; c += 512) {
    const h8 v = *reinterpret_cast<const h8*>(src + c);
    reinterpret_cast<f4*>(dst + c)[0] = f4{(float)v[0] * inv, (float)v[1] * inv, (float)v[2] * inv, (float)v[3] * inv};
    reinterpret_cast<f4*>(dst + c)[1] = f4{(float)v[4] * inv, (float)v[5] * inv, (float)v[6] * inv, (float)v[7] * inv};
  }
}

// Launches ceil(nseq / 256) grids of one 64-thread workgroup per sequence.  cu_seqlens is host
// memory (validated by the caller); nothing is allocated.
hipError_t launch_pool_last_l2(const _Float16* x, int64_t row_stride, int width, const int32_t* cu_seqlens,
                               int nseq, float* out, int64_t out_row_stride, hipStream_t stream) {
  for (int base = 0; base < nseq; base += kPoolMaxRows) {
    const int n = nseq - base < kPoolMaxRows ? nseq - base : kPoolMaxRows;
    PoolRows rows;
    for (int j = 0; j < n; ++j) {
      const int i = base + j;
      rows.row[j] = cu_seqlens[i + 1] > cu_seqlens[i] ? cu_seqlens[i + 1] - 1 : -1;
    }
    hipLaunchKernelGGL(pool_last_l2_kernel, dim3((unsigned)n), dim3(64), 0, stream, x, row_stride, width, out,
                       out_row_stride, base, rows);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace qattn
