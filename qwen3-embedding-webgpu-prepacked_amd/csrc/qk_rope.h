// qk_rope.h -- launch arguments of the QK-norm + RoPE producer (qk_rope.hip), shared with the
// host entry points that fill them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qattn {

typedef _Float16 half_t;

constexpr int kRopeSeqs = 64;
constexpr int kRopeMaxHeads = 32;
struct RopeArgs {
  const half_t* in;       // head h < split of row t at in + t * in_stride + in_col_q + 128 h,
                          // head h >= split at in + t * in_stride + in_col_k + 128 (h - split)
  half_t* out_q;          // head h < split of row t at out_q + t * out_stride_q + 128 h
  half_t* out_k;          // head h >= split at out_k + t * out_stride_k + 128 (h - split)
  const float* weight_q;  // gains of the first `split` heads (NULL: 1)
  const float* weight_k;  // gains of the others (NULL: 1)
  const float2* rope;     // [position][64] (cos, sin), f32 of the f64 angle (model.ts:76-81)
  int64_t in_stride, out_stride_q, out_stride_k;
  int64_t in_col_q, in_col_k;
  int32_t heads, split;   // head vectors per token: 4 * ITERS; split a multiple of 4
  float eps;
  int32_t nseq;
  int32_t cu[kRopeSeqs + 1];  // token offsets of this launch's sequences (cu[0] = first token)
};

// One launch per kRopeSeqs sequences of cu (host array of nseq + 1 offsets); the rest of `a`
// filled by the caller.
hipError_t launch_qk_norm_rope(RopeArgs a, const int32_t* cu, int nseq, hipStream_t stream);

}  // namespace qattn
