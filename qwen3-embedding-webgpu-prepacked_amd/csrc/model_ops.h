// model_ops.h -- launchers of the row-wise model kernels (model_ops.hip) and their limits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_common.h"

namespace qattn {

constexpr int kQ6KBlockBytes = 210;   // GGML Q6_K: 256 values (ggml block_q6_K)
constexpr int kRmsMaxWidth = 4096;    // rmsnorm_kernel: columns per row (one wavefront, 8 per lane per pass)

// out[t][c] (c < width, a multiple of 256) = token ids[t]'s row of the Q6_K table of `vocab` rows;
// ids outside [0, vocab) give zero rows.
hipError_t launch_embed_q6k(const int32_t* ids, int64_t tokens, const uint8_t* table, int64_t vocab, int width,
                            half_t* out, int64_t out_stride, hipStream_t stream);
// The residual add + RMSNorm that follows a projection, with the projection's output as the
// residual (launch_rmsnorm's other arguments).
struct RowNorm {
  half_t* x;
  int64_t x_stride;
  const float* weight;
  half_t* out;
  int64_t out_stride;
  float eps;
};
// RowNorm on a projection's split-K partial sums (part: chunks x rows x width fp32, width a
// multiple of 8 and <= kRmsMaxWidth, 16-byte aligned rows): bit for bit the projection's output
// followed by launch_rmsnorm, without writing that output.
hipError_t launch_reduce_rmsnorm(const float* part, int chunks, int rows, int width, const RowNorm& norm,
                                 hipStream_t stream);
// Residual add (residual may be NULL) + RMSNorm of `rows` rows of `width` (multiple of 8, <= kRmsMaxWidth).
hipError_t launch_rmsnorm(half_t* x, const half_t* residual, const float* weight, half_t* out, int64_t rows,
                          int width, int64_t x_stride, int64_t r_stride, int64_t out_stride, float eps,
                          hipStream_t stream);
// silu(g) * u in fp32, rounded to fp16: the one formula of swiglu_kernel and of the fused
// gate/up projection (q4_matmul.hip), so the two paths agree bit for bit.  The hardware exp2 and
// reciprocal (about 1 fp32 ulp each) are far inside the fp16 rounding of the result.
__device__ inline half_t swiglu_value(half_t g, half_t u) {
  const float gf = (float)g;
  float v = gf * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(gf * -1.44269504f)) * (float)u;
  // The product is rounded to fp32 and then to fp16 in every caller: without this the compiler
  // may fold the multiply and the conversion into one v_fma_mix (a single rounding) in one
  // kernel and not in another.
  asm volatile("" : "+v"(v));
  return (half_t)v;
}

// Bytes of fp32 partials a Q4_0 projection of this shape splits its K chunks into (0: the
// shape does not split; q4_matmul.hip).  A caller that passes a workspace of at least this size
// gets the split launch; the result is bit for bit the unsplit one's.
size_t q4_split_bytes(int M, int K, int N);

// out = silu(gate) * up for rows of [gate (width) | up (width)], width a multiple of 8.
hipError_t launch_swiglu(const half_t* gate_up, int64_t gu_stride, half_t* out, int64_t out_stride, int64_t rows,
                         int width, hipStream_t stream);

}  // namespace qattn
