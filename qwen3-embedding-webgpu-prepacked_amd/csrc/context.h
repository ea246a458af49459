// context.h -- the library context (the opaque qattn_ctx of include/qattn.h) and the helpers every
// C-ABI source shares: error reporting, device selection, stream choice, argument checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <string>

#include "../../include/qattn.h"

struct qattn_ctx {
  int device = 0;
  int cu_count = 0;
  hipStream_t stream = nullptr;
  hipStream_t read_stream = nullptr;  // qattn_buffer_read_after's copies (waits on events only)
  void* scratch = nullptr;  // this device's copy of the static work-list array (qattn_prefill_static)
  // RoPE table of the producer, [positions][64] (cos, sin), built for `rope_theta`; grown when a
  // longer sequence arrives (the reference builds one per plan, model.ts:76-83).
  float2* rope = nullptr;
  int32_t rope_positions = 0;
  double rope_theta = 0.0;
  std::string last_error;
  std::mutex mu;
};

namespace qattn {

// Records the message as the context's (and the calling thread's) last error; returns `code`.
int fail(qattn_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

// Sets the calling thread's and (when given) the context's last error without formatting.
void set_last_error(qattn_ctx* ctx, const std::string& message);

#define HIP_TRY(ctx, expr)                                                                   \
  do {                                                                                       \
    hipError_t e_ = (expr);                                                                  \
    if (e_ != hipSuccess)                                                                    \
      return ::qattn::fail((ctx), QATTN_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

// Makes `dev` current for the scope and restores the caller's device afterwards.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

inline hipStream_t pick_stream(qattn_ctx* ctx, qattn_stream_t s) {
  return s ? reinterpret_cast<hipStream_t>(s) : ctx->stream;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Host cu_seqlens: nseq in [1, QATTN_MAX_SEQS], cu[0] = 0, non-decreasing.
int validate_cu(qattn_ctx* ctx, const int32_t* cu, int32_t nseq);

struct RowNorm;  // model_ops.h
// qattn_q4_matmul with an optional fp32 workspace for the split launch of small projections
// (api.hip; the model plan passes its own).  With `norm`, a split launch also runs that residual
// add + RMSNorm on its output straight from the partial sums (and does not write y); *normed
// says whether it did, or the caller still has to.
int q4_matmul_ws(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w, int64_t w_bytes,
                 int32_t N, void* y, int64_t ldy, qattn_stream_t stream, float* ws, size_t ws_bytes,
                 const RowNorm* norm = nullptr, bool* normed = nullptr);

}  // namespace qattn
