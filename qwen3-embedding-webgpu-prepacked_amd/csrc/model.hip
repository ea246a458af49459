// model.hip -- the Qwen3-Embedding-0.6B forward on one stream (C ABI of include/qattn.h):
// qattn_embed_q6k / qattn_rmsnorm / qattn_swiglu, and qattn_model (weights) +
// qattn_model_plan (activations, one attention run) in place of the reference's
// Qwen3WebGPUModel / Qwen3ExecutionPlan (src/webgpu/model.ts:49-255).
//
// The plan enqueues the reference's sequence of dispatches (model.ts:117-131) over a packed
// varlen batch: no padding rows, RoPE positions restart per sequence, attention restricted to
// each sequence.  Every stage is one launch of this library's gfx950 kernels; the plan keeps its
// buffers between batches and re-plans only the attention work list.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <new>
#include <vector>

#include "../../include/qattn.h"
#include "attn_common.h"
#include "context.h"
#include "model_ops.h"

using namespace qattn;

namespace {
constexpr int kHidden = QATTN_HIDDEN;
constexpr int kInter = QATTN_INTERMEDIATE;
constexpr int kQkvWidth = kQHeads * kHeadDim + 2 * kKVHeads * kHeadDim;  // 4096 (model.ts:69)
constexpr int kQWidth = kQHeads * kHeadDim;                              // 2048
constexpr int kKWidth = kKVHeads * kHeadDim;                             // 1024
constexpr int64_t kEmbdRowBytes = (int64_t)kHidden / 256 * QATTN_Q6K_BLOCK_BYTES;  // 840
// The split workspace a plan of max_tokens needs: the largest the output (K = 2048) and down
// (K = 3072) projections ask for at any batch size up to max_tokens.
size_t max_split_bytes(int32_t max_tokens) {
  size_t best = 0;
  for (int32_t M = 1; M <= max_tokens; ++M) {
    const size_t a = q4_split_bytes(M, kQWidth, kHidden), b = q4_split_bytes(M, kInter, kHidden);
    if (!a && !b && M > 64) break;  // past the split range (it ends where the tiles stop being few)
    best = std::max(best, std::max(a, b));
  }
  return best;
}
}  // namespace

struct qattn_model {
  qattn_ctx* ctx = nullptr;
  qattn_model_desc desc{};
  std::vector<qattn_layer_weights> layers;
  int64_t vocab = 0;
};

struct qattn_model_plan {
  qattn_model* model = nullptr;
  int32_t max_tokens = 0, max_seqs = 0;
  int32_t* ids = nullptr;      // device int32 [max_tokens]
  void* x = nullptr;           // residual stream     [T][1024]
  void* normalized = nullptr;  // norm output          [T][1024]
  void* qkv = nullptr;         // qkvRaw               [T][4096]
  void* q = nullptr;           // roped Q              [T][2048]
  void* k = nullptr;           // roped K              [T][1024]
  void* attn = nullptr;        // attention output     [T][2048]
  void* delta = nullptr;       // projection output    [T][1024]
  void* ffn = nullptr;         // SwiGLU output        [T][3072]
  qattn_run* run = nullptr;
  std::vector<int32_t> planned_cu;  // the batch the attention run is planned for
  float* gemm_ws = nullptr;         // fp32 partials of the split output / down projections
  size_t gemm_ws_bytes = 0;
};

extern "C" {

// ---- the row-wise stages -------------------------------------------------------------------

int qattn_embed_q6k(qattn_ctx* ctx, const int32_t* ids, int64_t tokens, const void* table, int64_t table_bytes,
                    int32_t width, void* out, int64_t out_row_stride, qattn_stream_t stream) {
  if (!ctx || !ids || !table || !out) return fail(ctx, QATTN_EINVAL, "ctx/ids/table/out is NULL");
  if (width < 256 || width % 256 || out_row_stride < width || out_row_stride % 8 || tokens < 0)
    return fail(ctx, QATTN_EINVAL, "width %d / out_row_stride %lld / tokens %lld: width a multiple of 256, "
                "stride >= width and a multiple of 8", width, (long long)out_row_stride, (long long)tokens);
  const int64_t row_bytes = (int64_t)width / 256 * QATTN_Q6K_BLOCK_BYTES;
  if (table_bytes < row_bytes || table_bytes % row_bytes)
    return fail(ctx, QATTN_EINVAL, "table_bytes %lld is not a whole number of %lld-byte rows", (long long)table_bytes,
                (long long)row_bytes);
  if (!aligned16(out) || reinterpret_cast<uintptr_t>(ids) % 4)
    return fail(ctx, QATTN_EINVAL, "out must be 16-byte and ids 4-byte aligned");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_embed_q6k(ids, tokens, static_cast<const uint8_t*>(table), table_bytes / row_bytes, width,
                                static_cast<half_t*>(out), out_row_stride, pick_stream(ctx, stream)));
  return QATTN_OK;
}

int qattn_rmsnorm(qattn_ctx* ctx, void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                  const float* weight, void* out, int64_t out_row_stride, int64_t rows, int32_t width, double eps,
                  qattn_stream_t stream) {
  if (!ctx || !x || !weight || !out) return fail(ctx, QATTN_EINVAL, "ctx/x/weight/out is NULL");
  if (width < 8 || width % 8 || width > kRmsMaxWidth || rows < 0)
    return fail(ctx, QATTN_EINVAL, "width %d: a multiple of 8 in [8, %d]", width, kRmsMaxWidth);
  if (x_row_stride < width || x_row_stride % 8 || out_row_stride < width || out_row_stride % 8 ||
      (residual && (residual_row_stride < width || residual_row_stride % 8)))
    return fail(ctx, QATTN_EINVAL, "row strides must be >= width and multiples of 8 elements");
  if (!aligned16(x) || !aligned16(out) || !aligned16(weight) || (residual && !aligned16(residual)))
    return fail(ctx, QATTN_EINVAL, "x/residual/weight/out must be 16-byte aligned");
  if (out == x) return fail(ctx, QATTN_EINVAL, "out may not alias x");
  if (!(eps >= 0.0)) return fail(ctx, QATTN_EINVAL, "eps must be >= 0");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_rmsnorm(static_cast<half_t*>(x), static_cast<const half_t*>(residual), weight,
                              static_cast<half_t*>(out), rows, width, x_row_stride, residual_row_stride, out_row_stride,
                              (float)eps, pick_stream(ctx, stream)));
  return QATTN_OK;
}

int qattn_swiglu(qattn_ctx* ctx, const void* gate_up, int64_t gate_up_row_stride, void* out, int64_t out_row_stride,
                 int64_t rows, int32_t width, qattn_stream_t stream) {
  if (!ctx || !gate_up || !out) return fail(ctx, QATTN_EINVAL, "ctx/gate_up/out is NULL");
  if (width < 8 || width % 8 || rows < 0 || gate_up_row_stride < 2 * (int64_t)width || gate_up_row_stride % 8 ||
      out_row_stride < width || out_row_stride % 8)
    return fail(ctx, QATTN_EINVAL, "width %d / strides (%lld, %lld): width a multiple of 8, gate_up stride >= "
                "2*width, out stride >= width, multiples of 8", width, (long long)gate_up_row_stride,
                (long long)out_row_stride);
  if (!aligned16(gate_up) || !aligned16(out)) return fail(ctx, QATTN_EINVAL, "gate_up/out must be 16-byte aligned");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_swiglu(static_cast<const half_t*>(gate_up), gate_up_row_stride, static_cast<half_t*>(out),
                             out_row_stride, rows, width, pick_stream(ctx, stream)));
  return QATTN_OK;
}

// ---- model (weights) -----------------------------------------------------------------------

int qattn_model_create(qattn_ctx* ctx, const qattn_model_desc* d, qattn_model** out) {
  if (!ctx || !d || !out) return fail(ctx, QATTN_EINVAL, "ctx/desc/out is NULL");
  *out = nullptr;
  if (!d->token_embd || d->token_embd_bytes < kEmbdRowBytes || d->token_embd_bytes % kEmbdRowBytes)
    return fail(ctx, QATTN_EINVAL, "token_embd: %lld bytes is not a whole number of %lld-byte Q6_K rows of %d",
                (long long)d->token_embd_bytes, (long long)kEmbdRowBytes, kHidden);
  if (!d->output_norm || !aligned16(d->output_norm))
    return fail(ctx, QATTN_EINVAL, "output_norm must be a 16-byte aligned device pointer");
  if (d->n_layers < 1 || d->n_layers > QATTN_MAX_LAYERS || !d->layers)
    return fail(ctx, QATTN_EINVAL, "n_layers %d outside [1, %d] (or layers NULL)", d->n_layers, QATTN_MAX_LAYERS);
  if (!(d->eps >= 0.0) || !(d->rope_theta > 0.0)) return fail(ctx, QATTN_EINVAL, "bad eps/rope_theta");
  if (d->mask != QATTN_MASK_CAUSAL && d->mask != QATTN_MASK_PREFIX_LOCAL)
    return fail(ctx, QATTN_EINVAL, "unknown mask kind %d", d->mask);
  if (d->mask == QATTN_MASK_PREFIX_LOCAL && (d->prefix < 0 || d->window < 0 || (d->prefix == 0 && d->window == 0)))
    return fail(ctx, QATTN_EINVAL, "prefix %d / window %d: >= 0, not both 0", d->prefix, d->window);
  if (d->flags & ~QATTN_FLAG_BATCH_INVARIANT) return fail(ctx, QATTN_EINVAL, "unknown flags 0x%x", d->flags);
  struct Gemm {
    const char* name;
    const void* w;
    int64_t bytes;
    int K, N;
  };
  for (int32_t l = 0; l < d->n_layers; ++l) {
    const qattn_layer_weights& w = d->layers[l];
    const float* gains[] = {w.attn_norm, w.attn_q_norm, w.attn_k_norm, w.ffn_norm};
    for (const float* p : gains)
      if (!p || !aligned16(p)) return fail(ctx, QATTN_EINVAL, "layer %d: norm gains must be 16-byte aligned device pointers", l);
    const Gemm gemms[] = {{"attn_qkv", w.attn_qkv, w.attn_qkv_bytes, kHidden, kQkvWidth},
                          {"attn_output", w.attn_output, w.attn_output_bytes, kQWidth, kHidden},
                          {"ffn_gate_up", w.ffn_gate_up, w.ffn_gate_up_bytes, kHidden, 2 * kInter},
                          {"ffn_down", w.ffn_down, w.ffn_down_bytes, kInter, kHidden}};
    for (const Gemm& m : gemms) {
      const int64_t need = qattn_q4_compact_bytes(m.K, m.N);
      if (!m.w || reinterpret_cast<uintptr_t>(m.w) % 4 || m.bytes < need)
        return fail(ctx, QATTN_EINVAL, "layer %d: %s needs a 4-byte aligned %d -> %d compact tensor of %lld bytes (got %lld)",
                    l, m.name, m.K, m.N, (long long)need, (long long)m.bytes);
    }
  }
  auto* m = new (std::nothrow) qattn_model();
  if (!m) return fail(ctx, QATTN_ENOMEM, "out of host memory");
  m->ctx = ctx;
  m->desc = *d;
  m->layers.assign(d->layers, d->layers + d->n_layers);
  m->desc.layers = nullptr;
  m->vocab = d->token_embd_bytes / kEmbdRowBytes;
  *out = m;
  return QATTN_OK;
}

void qattn_model_destroy(qattn_model* model) { delete model; }

}  // extern "C"

// ---- plan ----------------------------------------------------------------------------------

namespace {

void free_plan(qattn_model_plan* p) {
  if (p->run) qattn_run_destroy(p->run);  // waits for the context stream
  qattn_ctx* ctx = p->model->ctx;
  DeviceGuard g(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  void* bufs[] = {p->ids, p->x, p->normalized, p->qkv, p->q, p->k, p->attn, p->delta, p->ffn, p->gemm_ws};
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  delete p;
}

// Stage markers of qattn_model_plan_profile: an event pair around every stage.
struct Recorder {
  std::vector<hipEvent_t> events;  // begin, end per recorded stage
  std::vector<int> stage;
  hipStream_t stream = nullptr;
  hipError_t err = hipSuccess;
  void begin(int s) {
    hipEvent_t e = nullptr;
    if (err == hipSuccess) err = hipEventCreate(&e);
    if (err == hipSuccess) err = hipEventRecord(e, stream);
    events.push_back(e);
    stage.push_back(s);
  }
  void end() {
    hipEvent_t e = nullptr;
    if (err == hipSuccess) err = hipEventCreate(&e);
    if (err == hipSuccess) err = hipEventRecord(e, stream);
    events.push_back(e);
  }
  ~Recorder() {
    for (hipEvent_t e : events)
      if (e) (void)hipEventDestroy(e);
  }
};

// Everything after the checks: enqueues one batch of T tokens.
int enqueue(qattn_model_plan* p, const int32_t* cu, int32_t nseq, float* out, int64_t out_row_stride,
            hipStream_t stream, Recorder* rec) {
  const qattn_model* m = p->model;
  qattn_ctx* ctx = m->ctx;
  const qattn_model_desc& d = m->desc;
  const int64_t T = cu[nseq];
  const qattn_stream_t s = reinterpret_cast<qattn_stream_t>(stream);
  auto begin = [&](int stage) {
    if (rec) rec->begin(stage);
  };
  auto end = [&]() {
    if (rec) rec->end();
  };
  int rc;
#define STAGE_TRY(expr) \
  do {                  \
    rc = (expr);        \
    if (rc) return rc;  \
  } while (0)
  begin(QATTN_STAGE_EMBEDDING_NORM);
  STAGE_TRY(qattn_embed_q6k(ctx, p->ids, T, d.token_embd, d.token_embd_bytes, kHidden, p->x, kHidden, s));
  STAGE_TRY(qattn_rmsnorm(ctx, p->x, kHidden, nullptr, 0, m->layers[0].attn_norm, p->normalized, kHidden, T, kHidden,
                          d.eps, s));
  end();
  for (int32_t l = 0; l < d.n_layers; ++l) {
    const qattn_layer_weights& w = m->layers[l];
    const float* next_norm = l + 1 < d.n_layers ? m->layers[l + 1].attn_norm : d.output_norm;
    begin(QATTN_STAGE_QKV);
    STAGE_TRY(qattn_q4_matmul(ctx, p->normalized, kHidden, (int32_t)T, kHidden, w.attn_qkv, w.attn_qkv_bytes,
                              kQkvWidth, p->qkv, kQkvWidth, s));
    end();
    begin(QATTN_STAGE_ROPE_ATTENTION);
    STAGE_TRY(qattn_qk_norm_rope_qkv(ctx, p->qkv, kQkvWidth, p->q, kQWidth, p->k, kKWidth, cu, nseq, w.attn_q_norm,
                                     w.attn_k_norm, d.eps, d.rope_theta, s));
    STAGE_TRY(qattn_run_encode(p->run, s));
    end();
    // A split projection (small batches) runs the residual add + RMSNorm that follows it straight
    // from its partial sums; its time then falls in the projection's stage.
    const RowNorm ffn_in{static_cast<half_t*>(p->x), kHidden, w.ffn_norm, static_cast<half_t*>(p->normalized),
                         kHidden, (float)d.eps};
    bool normed = false;
    begin(QATTN_STAGE_ATTENTION_OUTPUT);
    STAGE_TRY(q4_matmul_ws(ctx, p->attn, kQWidth, (int32_t)T, kQWidth, w.attn_output, w.attn_output_bytes, kHidden,
                           p->delta, kHidden, s, p->gemm_ws, p->gemm_ws_bytes, &ffn_in, &normed));
    end();
    begin(QATTN_STAGE_POST_ATTENTION_NORM);
    if (!normed)
      STAGE_TRY(qattn_rmsnorm(ctx, p->x, kHidden, p->delta, kHidden, w.ffn_norm, p->normalized, kHidden, T, kHidden,
                              d.eps, s));
    end();
    // The gate/up projection and SwiGLU are one launch (no [T][6144] intermediate); its time is
    // the ffn_up_gate stage and the swiglu stage stays empty.
    begin(QATTN_STAGE_FFN_UP_GATE);
    STAGE_TRY(qattn_q4_matmul_swiglu(ctx, p->normalized, kHidden, (int32_t)T, kHidden, w.ffn_gate_up,
                                     w.ffn_gate_up_bytes, kInter, p->ffn, kInter, s));
    end();
    begin(QATTN_STAGE_SWIGLU);
    end();
    const RowNorm next_in{static_cast<half_t*>(p->x), kHidden, next_norm, static_cast<half_t*>(p->normalized),
                          kHidden, (float)d.eps};
    begin(QATTN_STAGE_FFN_DOWN);
    STAGE_TRY(q4_matmul_ws(ctx, p->ffn, kInter, (int32_t)T, kInter, w.ffn_down, w.ffn_down_bytes, kHidden, p->delta,
                           kHidden, s, p->gemm_ws, p->gemm_ws_bytes, &next_in, &normed));
    end();
    begin(QATTN_STAGE_POST_FFN_NORM);
    if (!normed)
      STAGE_TRY(qattn_rmsnorm(ctx, p->x, kHidden, p->delta, kHidden, next_norm, p->normalized, kHidden, T, kHidden,
                              d.eps, s));
    end();
  }
  begin(QATTN_STAGE_POOL);
  STAGE_TRY(qattn_pool_last_l2(ctx, p->normalized, kHidden, kHidden, cu, nseq, out, out_row_stride, s));
  end();
#undef STAGE_TRY
  return QATTN_OK;
}

// Checks a batch, uploads its ids and re-plans the attention run when the batch changed.
int prepare(qattn_model_plan* p, const int32_t* ids, const int32_t* cu, int32_t nseq, float* out,
            int64_t out_row_stride, hipStream_t stream) {
  const qattn_model* m = p->model;
  qattn_ctx* ctx = m->ctx;
  int rc = validate_cu(ctx, cu, nseq);
  if (rc) return rc;
  const int64_t T = cu[nseq];
  if (nseq > p->max_seqs || T > p->max_tokens)
    return fail(ctx, QATTN_EINVAL, "batch of %d sequences / %lld tokens exceeds the plan's %d / %d", nseq,
                (long long)T, p->max_seqs, p->max_tokens);
  if (!out || !aligned16(out) || out_row_stride < kHidden || out_row_stride % 4)
    return fail(ctx, QATTN_EINVAL, "out: a 16-byte aligned device pointer, row stride >= %d and a multiple of 4",
                kHidden);
  if (T > 0 && !ids) return fail(ctx, QATTN_EINVAL, "ids is NULL");
  for (int64_t t = 0; t < T; ++t)
    if (ids[t] < 0 || ids[t] >= m->vocab)
      return fail(ctx, QATTN_EINVAL, "token %lld: id %d outside the vocabulary [0, %lld)", (long long)t, ids[t],
                  (long long)m->vocab);
  DeviceGuard g(ctx->device);
  if (T > 0) HIP_TRY(ctx, hipMemcpyAsync(p->ids, ids, (size_t)T * 4, hipMemcpyHostToDevice, stream));
  if (!std::equal(p->planned_cu.begin(), p->planned_cu.end(), cu, cu + nseq + 1) ||
      p->planned_cu.size() != (size_t)nseq + 1) {
    rc = qattn_run_update(p->run, cu, nseq);
    if (rc) return rc;
    p->planned_cu.assign(cu, cu + nseq + 1);
  }
  return QATTN_OK;
}

}  // namespace

extern "C" {

int qattn_model_plan_create(qattn_model* model, int32_t max_tokens, int32_t max_seqs, qattn_model_plan** out) {
  if (!model || !out) return fail(model ? model->ctx : nullptr, QATTN_EINVAL, "model/out is NULL");
  *out = nullptr;
  qattn_ctx* ctx = model->ctx;
  if (max_tokens < 1 || max_tokens > (1 << 24) || max_seqs < 1 || max_seqs > QATTN_MAX_SEQS)
    return fail(ctx, QATTN_EINVAL, "max_tokens %d / max_seqs %d outside [1, 2^24] / [1, %d]", max_tokens, max_seqs,
                QATTN_MAX_SEQS);
  auto* p = new (std::nothrow) qattn_model_plan();
  if (!p) return fail(ctx, QATTN_ENOMEM, "out of host memory");
  p->model = model;
  p->max_tokens = max_tokens;
  p->max_seqs = max_seqs;
  {
    DeviceGuard g(ctx->device);
    const size_t T = (size_t)max_tokens;
    struct Buf {
      void** ptr;
      size_t bytes;
    } bufs[] = {{reinterpret_cast<void**>(&p->ids), T * 4},   {&p->x, T * kHidden * 2},
                {&p->normalized, T * kHidden * 2},             {&p->qkv, T * kQkvWidth * 2},
                {&p->q, T * kQWidth * 2},                      {&p->k, T * kKWidth * 2},
                {&p->attn, T * kQWidth * 2},                   {&p->delta, T * kHidden * 2},
                {&p->ffn, T * kInter * 2},
                // the largest split workspace any batch of this plan asks for (0 when none splits)
                {reinterpret_cast<void**>(&p->gemm_ws), p->gemm_ws_bytes = max_split_bytes(max_tokens)}};
    for (const Buf& b : bufs) {
      if (!b.bytes) continue;
      const hipError_t e = hipMalloc(b.ptr, b.bytes);
      if (e != hipSuccess) {
        free_plan(p);
        return fail(ctx, QATTN_ENOMEM, "plan buffers for %d tokens: %s", max_tokens, hipGetErrorString(e));
      }
    }
  }
  // The attention run reads q, k and V in place from qkvRaw (value stride 4096, offset 3072,
  // model.ts:95); planned here for one sequence of max_tokens, re-planned per batch.
  const int32_t cu[2] = {0, max_tokens};
  qattn_run_desc rd{};
  rd.q = p->q;
  rd.k = p->k;
  rd.v = p->qkv;
  rd.o = p->attn;
  rd.q_row_stride = kQWidth;
  rd.k_row_stride = kKWidth;
  rd.v_row_stride = kQkvWidth;
  rd.o_row_stride = kQWidth;
  rd.v_offset = kQWidth + kKWidth;
  rd.cu_seqlens = cu;
  rd.nseq = 1;
  rd.mask = model->desc.mask;
  rd.prefix = model->desc.prefix;
  rd.window = model->desc.window;
  rd.flags = model->desc.flags;
  int rc = qattn_run_create(ctx, &rd, &p->run);
  if (rc) {
    free_plan(p);
    return rc;
  }
  p->planned_cu.assign(cu, cu + 2);
  *out = p;
  return QATTN_OK;
}

void qattn_model_plan_destroy(qattn_model_plan* plan) {
  if (plan) free_plan(plan);
}

int qattn_model_plan_run(qattn_model_plan* plan, const int32_t* ids, const int32_t* cu_seqlens, int32_t nseq,
                         float* out, int64_t out_row_stride, qattn_stream_t stream) {
  if (!plan) return fail(nullptr, QATTN_EINVAL, "plan is NULL");
  qattn_ctx* ctx = plan->model->ctx;
  const hipStream_t st = pick_stream(ctx, stream);
  int rc = prepare(plan, ids, cu_seqlens, nseq, out, out_row_stride, st);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  return enqueue(plan, cu_seqlens, nseq, out, out_row_stride, st, nullptr);
}

int qattn_model_plan_profile(qattn_model_plan* plan, const int32_t* ids, const int32_t* cu_seqlens, int32_t nseq,
                             float* out, int64_t out_row_stride, qattn_stream_t stream,
                             float stage_ms[QATTN_STAGE_COUNT]) {
  if (!plan || !stage_ms) return fail(plan ? plan->model->ctx : nullptr, QATTN_EINVAL, "plan/stage_ms is NULL");
  qattn_ctx* ctx = plan->model->ctx;
  const hipStream_t st = pick_stream(ctx, stream);
  int rc = prepare(plan, ids, cu_seqlens, nseq, out, out_row_stride, st);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  Recorder rec;
  rec.stream = st;
  rc = enqueue(plan, cu_seqlens, nseq, out, out_row_stride, st, &rec);
  if (rc) return rc;
  if (rec.err != hipSuccess) return fail(ctx, QATTN_EHIP, "stage events: %s", hipGetErrorString(rec.err));
  HIP_TRY(ctx, hipStreamSynchronize(st));
  for (int s = 0; s < QATTN_STAGE_COUNT; ++s) stage_ms[s] = 0.f;
  for (size_t i = 0; i < rec.stage.size(); ++i) {
    float ms = 0.f;
    HIP_TRY(ctx, hipEventElapsedTime(&ms, rec.events[2 * i], rec.events[2 * i + 1]));
    stage_ms[rec.stage[i]] += ms;
  }
  return QATTN_OK;
}

}  // extern "C"
