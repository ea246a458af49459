// api.hip -- the C ABI declared in include/qattn.h: context, buffers, the attention operator
// (planner + launch), the mask check, the QK-norm/RoPE producer and the input generator.
//
// A run (CausalAttentionKernel.createRun, src/webgpu/ops.ts:327-343) validates its description,
// plans it (planner.cpp) and holds the work list in device memory for every later encode.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/qattn.h"
#include "attn_common.h"
#include "context.h"
#include "planner.h"
#include "qk_rope.h"

namespace qattn {
hipError_t launch_attn_fwd(const AttnParams& p, hipStream_t stream);
hipError_t launch_attn_merge(const AttnParams& p, hipStream_t stream);
hipError_t launch_debug_mask(int S, MaskSpec mask, uint32_t* bits, int words_per_row,
                             hipStream_t stream);
hipError_t launch_xcd_map(int* out, int n, hipStream_t stream);
hipError_t launch_fill_normal(half_t* dst, int64_t rows, int64_t row_elems, int64_t row_stride,
                              uint64_t seed, hipStream_t stream);
hipError_t launch_fill_token_rows(half_t* dst, const int32_t* ids, int64_t rows, int64_t row_elems,
                                  int64_t row_stride, uint64_t seed, hipStream_t stream);
hipError_t launch_q4_matmul(const half_t* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                            half_t* y, int64_t ldy, hipStream_t stream, float* ws, size_t ws_bytes,
                            const RowNorm* norm, bool* normed);
hipError_t launch_q4_matmul_swiglu(const half_t* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes,
                                   int n_inter, half_t* y, int64_t ldy, hipStream_t stream);
hipError_t launch_pool_last_l2(const half_t* x, int64_t row_stride, int width, const int32_t* cu_seqlens,
                               int nseq, float* out, int64_t out_row_stride, hipStream_t stream);
}  // namespace qattn

using namespace qattn;

// Work-list storage of qattn_prefill_static, the entry point that allocates no device memory:
// a fixed array in the library's own device image, one copy per GPU, held until the process
// ends.  Host code never uses its name as an address (that would be a host stand-in): each
// context resolves the device address once, with its device current, in qattn_create, and passes
// that pointer on.  1 MiB holds the work list (32-byte entries) and the slot offsets of launches
// of up to about 32000 entries -- 64-query blocks x 8 KV heads, roughly 250k tokens.
namespace {
constexpr size_t kScratchBytes = (size_t)1 << 20;
}
static __device__ __align__(256) char scratch[kScratchBytes];

// A run keeps two plan images (work list, split items' chunk-0 entries, slot offsets) so that a
// re-plan never writes the image a launch may still be reading: the installed plan lives in
// image `cur`, a re-plan fills image cur ^ 1 and then switches.  An encode only notes its stream
// in `streams[cur]` (no per-launch event: an event record between back-to-back launches costs
// 2.5-3.5 us each on MI355X).  When a re-plan retires image i it records one event on each of
// those streams (`fences[i]`), after every launch that read the image; the re-plan that later
// overwrites image i waits for exactly those events -- in the engine's steady state they completed
// long before -- instead of for the device.
struct qattn_run {
  qattn_ctx* ctx = nullptr;
  AttnParams params{};         // launch arguments of the installed plan (image `cur`)
  void* plan_dev[2] = {nullptr, nullptr};
  size_t plan_capacity[2] = {0, 0};  // bytes at plan_dev[i]
  std::vector<hipStream_t> streams[2];  // streams that launched image i since it was installed
  std::vector<hipEvent_t> fences[2];    // recorded on those streams when image i was retired
  int cur = -1;                // image of the installed plan (-1: none yet)
  void* split_dev = nullptr;   // the chunks' partial results (merged by a second kernel); one
                               // workspace: launches of one run are ordered on the device
  int32_t partial_capacity = 0;  // partial-result records at split_dev
  qattn_run_desc desc{};       // the description it was created with (cu_seqlens: not kept)
  int32_t max_len = 0;         // longest sequence
  qattn_run_info info{};
};

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace qattn {

int fail(qattn_ctx* ctx, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  set_last_error(ctx, buf);
  return code;
}

void set_last_error(qattn_ctx* ctx, const std::string& message) {
  g_last_error = message;
  if (ctx) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->last_error = message;
  }
}

int validate_cu(qattn_ctx* ctx, const int32_t* cu, int32_t nseq) {
  if (!cu) return fail(ctx, QATTN_EINVAL, "cu_seqlens is NULL");
  if (nseq < 1 || nseq > QATTN_MAX_SEQS)
    return fail(ctx, QATTN_EINVAL, "nseq=%d outside [1, %d]", nseq, QATTN_MAX_SEQS);
  if (cu[0] != 0) return fail(ctx, QATTN_EINVAL, "cu_seqlens[0]=%d, expected 0", cu[0]);
  for (int32_t i = 0; i < nseq; ++i)
    if (cu[i + 1] < cu[i])
      return fail(ctx, QATTN_EINVAL, "cu_seqlens not non-decreasing at %d (%d > %d)", i, cu[i],
                  cu[i + 1]);
  return QATTN_OK;
}

}  // namespace qattn

namespace {

int validate_desc(qattn_ctx* ctx, const qattn_run_desc* d) {
  if (!d) return fail(ctx, QATTN_EINVAL, "desc is NULL");
  if (!d->q || !d->k || !d->v || !d->o) return fail(ctx, QATTN_EINVAL, "q/k/v/o must be non-NULL");
  if (!aligned16(d->q) || !aligned16(d->k) || !aligned16(d->v) || !aligned16(d->o) ||
      (d->o_last && !aligned16(d->o_last)))
    return fail(ctx, QATTN_EINVAL, "q/k/v/o/o_last must be 16-byte aligned");
  if (d->q_row_stride < kQHeads * kHeadDim || d->o_row_stride < kQHeads * kHeadDim ||
      d->k_row_stride < kKVHeads * kHeadDim || d->v_row_stride < kKVHeads * kHeadDim)
    return fail(ctx, QATTN_EINVAL,
                "row strides too small (q %lld, k %lld, v %lld, o %lld; need q,o >= 2048 and "
                "k,v >= 1024)",
                (long long)d->q_row_stride, (long long)d->k_row_stride,
                (long long)d->v_row_stride, (long long)d->o_row_stride);
  if ((d->q_row_stride | d->k_row_stride | d->v_row_stride | d->o_row_stride | d->v_offset) & 7)
    return fail(ctx, QATTN_EINVAL, "row strides and v_offset must be multiples of 8 elements");
  if (d->v_offset < 0) return fail(ctx, QATTN_EINVAL, "v_offset must be >= 0");
  if (d->flags & ~QATTN_FLAG_BATCH_INVARIANT) return fail(ctx, QATTN_EINVAL, "unknown flags 0x%x", d->flags);
  if (d->mask != QATTN_MASK_CAUSAL && d->mask != QATTN_MASK_PREFIX_LOCAL)
    return fail(ctx, QATTN_EINVAL, "unknown mask kind %d", d->mask);
  if (d->mask == QATTN_MASK_PREFIX_LOCAL) {
    if (d->prefix < 0 || d->window < 0)
      return fail(ctx, QATTN_EINVAL, "prefix (%d) and window (%d) must be >= 0", d->prefix, d->window);
    if (d->prefix == 0 && d->window == 0)
      return fail(ctx, QATTN_EINVAL, "prefix and window are both 0: no query would see a key");
  }
  int rc = validate_cu(ctx, d->cu_seqlens, d->nseq);
  if (rc) return rc;
  const int64_t T = d->cu_seqlens[d->nseq];
  if (T >= ((int64_t)1 << 31)) return fail(ctx, QATTN_EINVAL, "too many tokens (%lld)", (long long)T);
  // The kernel addresses one sequence's rows (plus up to one 64-row tile past its end, which the
  // buffer range check zero-fills) with 32-bit byte offsets.
  const int64_t max_stride = std::max(std::max(d->q_row_stride, d->k_row_stride),
                                      std::max(d->v_row_stride, d->o_row_stride));
  for (int32_t s = 0; s < d->nseq; ++s) {
    const int64_t L = d->cu_seqlens[s + 1] - d->cu_seqlens[s];
    if ((L + kTileK) * max_stride * 2 >= ((int64_t)1 << 31))
      return fail(ctx, QATTN_EINVAL, "sequence %d: %lld tokens x row stride %lld exceeds 2 GiB", s,
                  (long long)L, (long long)max_stride);
  }
  return QATTN_OK;
}


}  // namespace

extern "C" {

int qattn_abi_version(void) { return QATTN_ABI_VERSION; }

const char* qattn_last_error(const qattn_ctx* ctx) {
  if (ctx) return ctx->last_error.c_str();
  return g_last_error.c_str();
}

int qattn_create(int device, qattn_ctx** out) {
  if (!out) return fail(nullptr, QATTN_EINVAL, "out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) return fail(nullptr, QATTN_ENODEV, "no HIP device (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(nullptr, QATTN_EINVAL, "device %d outside [0, %d)", device, n);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(nullptr, QATTN_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, QATTN_ENODEV, "device %d is %s; this library is built for gfx950 only",
                device, prop.gcnArchName);
  auto* ctx = new (std::nothrow) qattn_ctx();
  if (!ctx) return fail(nullptr, QATTN_ENOMEM, "out of host memory");
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  DeviceGuard g(device);
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return fail(nullptr, QATTN_EHIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  e = hipStreamCreateWithFlags(&ctx->read_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(nullptr, QATTN_EHIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  e = hipGetSymbolAddress(&ctx->scratch, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ctx->scratch) {
    (void)hipStreamDestroy(ctx->read_stream);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(nullptr, QATTN_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  }
  *out = ctx;
  return QATTN_OK;
}

void qattn_destroy(qattn_ctx* ctx) {
  if (!ctx) return;
  {
    DeviceGuard g(ctx->device);
    if (ctx->stream) {
      (void)hipStreamSynchronize(ctx->stream);
      (void)hipStreamDestroy(ctx->stream);
    }
    if (ctx->read_stream) {
      (void)hipStreamSynchronize(ctx->read_stream);
      (void)hipStreamDestroy(ctx->read_stream);
    }
    if (ctx->rope) (void)hipFree(ctx->rope);
  }
  delete ctx;
}

qattn_stream_t qattn_stream(qattn_ctx* ctx) { return ctx ? ctx->stream : nullptr; }

int qattn_synchronize(qattn_ctx* ctx) {
  if (!ctx) return fail(nullptr, QATTN_EINVAL, "ctx is NULL");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return QATTN_OK;
}

int qattn_device_name(qattn_ctx* ctx, char* buf, size_t len, int* cu_count) {
  if (!ctx) return fail(nullptr, QATTN_EINVAL, "ctx is NULL");
  hipDeviceProp_t prop;
  HIP_TRY(ctx, hipGetDeviceProperties(&prop, ctx->device));
  if (buf && len) {
    std::strncpy(buf, prop.gcnArchName, len - 1);
    buf[len - 1] = 0;
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  return QATTN_OK;
}

// ---- buffers ----------------------------------------------------------------------------------

int qattn_buffer_alloc(qattn_ctx* ctx, size_t bytes, void** dptr) {
  if (!ctx || !dptr) return fail(ctx, QATTN_EINVAL, "ctx/dptr is NULL");
  *dptr = nullptr;
  DeviceGuard g(ctx->device);
  hipError_t e = hipMalloc(dptr, bytes ? bytes : 16);
  if (e != hipSuccess) return fail(ctx, QATTN_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  return QATTN_OK;
}

int qattn_buffer_free(qattn_ctx* ctx, void* dptr) {
  if (!ctx) return fail(nullptr, QATTN_EINVAL, "ctx is NULL");
  if (!dptr) return QATTN_OK;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  HIP_TRY(ctx, hipFree(dptr));
  return QATTN_OK;
}

int qattn_buffer_write(qattn_ctx* ctx, void* dst, size_t offset, const void* src, size_t bytes) {
  if (!ctx || !dst || (!src && bytes)) return fail(ctx, QATTN_EINVAL, "NULL argument");
  if (!bytes) return QATTN_OK;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipMemcpyAsync(static_cast<char*>(dst) + offset, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return QATTN_OK;
}

int qattn_buffer_read(qattn_ctx* ctx, const void* src, size_t offset, void* dst, size_t bytes) {
  if (!ctx || !src || (!dst && bytes)) return fail(ctx, QATTN_EINVAL, "NULL argument");
  if (!bytes) return QATTN_OK;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipMemcpyAsync(dst, static_cast<const char*>(src) + offset, bytes, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return QATTN_OK;
}

int qattn_buffer_read_after(qattn_ctx* ctx, qattn_event_t after, const void* src, size_t offset, void* dst,
                            size_t bytes) {
  if (!ctx || !after || !src || (!dst && bytes)) return fail(ctx, QATTN_EINVAL, "NULL argument");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipStreamWaitEvent(ctx->read_stream, reinterpret_cast<hipEvent_t>(after), 0));
  if (bytes)
    HIP_TRY(ctx, hipMemcpyAsync(dst, static_cast<const char*>(src) + offset, bytes, hipMemcpyDeviceToHost,
                                ctx->read_stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->read_stream));
  return QATTN_OK;
}

int qattn_buffer_fill_u16(qattn_ctx* ctx, void* dst, uint16_t value, size_t count) {
  if (!ctx || (!dst && count)) return fail(ctx, QATTN_EINVAL, "NULL argument");
  if (!count) return QATTN_OK;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipMemsetD16Async(reinterpret_cast<hipDeviceptr_t>(dst), value, count, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return QATTN_OK;
}

// ---- attention operator -----------------------------------------------------------------------

}  // extern "C"

extern "C" {

int qattn_plan_describe(const qattn_run_desc* desc, int32_t* items, int32_t capacity,
                        int32_t* count, qattn_run_info* info) {
  if (!count) return fail(nullptr, QATTN_EINVAL, "count is NULL");
  Plan plan;
  qattn_run_info inf{};
  int rc = validate_desc(nullptr, desc);
  if (rc) return rc;
  plan_work(desc, kDefaultSlots, &plan, &inf, nullptr);
  *count = (int32_t)plan.items.size();
  if (info) *info = inf;
  if (items) {
    if (capacity < (int32_t)plan.items.size())
      return fail(nullptr, QATTN_EINVAL, "capacity %d < %zu work entries", capacity, plan.items.size());
    static_assert(sizeof(WorkItem) == 8 * sizeof(int32_t), "work entry is 8 int32");
    std::memcpy(items, plan.items.data(), plan.items.size() * sizeof(WorkItem));
  }
  return QATTN_OK;
}

int qattn_plan_slots(const qattn_run_desc* desc, int32_t max_slots, int32_t* slot_begin,
                     int32_t capacity, int32_t* nslots) {
  if (!nslots) return fail(nullptr, QATTN_EINVAL, "nslots is NULL");
  Plan plan;
  int rc = validate_desc(nullptr, desc);
  if (rc) return rc;
  plan_work(desc, max_slots > 0 ? max_slots : kDefaultSlots, &plan, nullptr, nullptr);
  *nslots = (int32_t)plan.slot_begin.size() - 1;
  if (slot_begin) {
    if (capacity < (int32_t)plan.slot_begin.size())
      return fail(nullptr, QATTN_EINVAL, "capacity %d < %zu slot offsets", capacity, plan.slot_begin.size());
    std::memcpy(slot_begin, plan.slot_begin.data(), plan.slot_begin.size() * sizeof(int32_t));
  }
  return QATTN_OK;
}

}  // extern "C"

namespace {

// qattn_debug_fail_allocs: device allocations of install_plan still to fail.
std::atomic<int32_t> g_fail_allocs{0};
hipError_t plan_malloc(void** p, size_t bytes) {
  int32_t n = g_fail_allocs.load();
  while (n > 0)
    if (g_fail_allocs.compare_exchange_weak(n, n - 1)) return hipErrorOutOfMemory;
  return hipMalloc(p, bytes);
}

// Records, on every stream that launched image i since it was installed, an event after those
// launches (fences[i]), and forgets the streams: image i's launches are then covered by its fences.
hipError_t retire_image(qattn_run* run, int i) {
  for (hipStream_t s : run->streams[i]) {
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ev, s);
    if (e != hipSuccess) {
      if (ev) (void)hipEventDestroy(ev);
      return e;
    }
    run->fences[i].push_back(ev);
  }
  run->streams[i].clear();
  return hipSuccess;
}

// Waits until no launch that reads image i (already retired) is still running.
hipError_t wait_image(qattn_run* run, int i) {
  auto& f = run->fences[i];
  while (!f.empty()) {
    const hipError_t e = hipEventSynchronize(f.back());
    if (e != hipSuccess) return e;
    (void)hipEventDestroy(f.back());
    f.pop_back();
  }
  return hipSuccess;
}

// Plans a validated description into `run` as one transaction: the new plan image goes to the
// image slot the installed plan does not use (after the launches that last read that slot have
// finished), growing it or the split workspace only when they are too small; the run switches to
// the new plan only once everything has succeeded.  On any failure the installed plan, its
// launch arguments and every buffer they point to stay as they were, so later encodes stay valid.
// The only device-wide wait left is hipFree's, and only when a buffer must grow.
int install_plan(qattn_run* run, const qattn_run_desc* d) {
  qattn_ctx* ctx = run->ctx;
  Plan plan;
  qattn_run_info info{};
  MaskSpec mask{};
  plan_work(d, std::max(1, ctx->cu_count) * kBlocksPerCU, &plan, &info, &mask);
  // One upload: the entries, the split items' chunk-0 entries, then the slot offsets (32-byte
  // entries keep the offsets aligned).
  const size_t items_bytes = plan.items.size() * sizeof(WorkItem);
  const size_t heads_bytes = plan.split_heads.size() * sizeof(WorkItem);
  const size_t slots_bytes = plan.slot_begin.size() * sizeof(int32_t);
  std::vector<char> image(items_bytes + heads_bytes + slots_bytes);
  if (items_bytes) std::memcpy(image.data(), plan.items.data(), items_bytes);
  if (heads_bytes) std::memcpy(image.data() + items_bytes, plan.split_heads.data(), heads_bytes);
  std::memcpy(image.data() + items_bytes + heads_bytes, plan.slot_begin.data(), slots_bytes);
  DeviceGuard g(ctx->device);
  const int next = run->cur < 0 ? 0 : run->cur ^ 1;
  // Fences for the installed plan's launches so far (waited on by the re-plan after this one);
  // extra fences from an update that fails later are harmless.
  if (run->cur >= 0) HIP_TRY(ctx, retire_image(run, run->cur));
  HIP_TRY(ctx, wait_image(run, next));
  if (image.size() > run->plan_capacity[next]) {
    void* grown = nullptr;
    hipError_t e = plan_malloc(&grown, image.size());
    if (e != hipSuccess) return fail(ctx, QATTN_ENOMEM, "hipMalloc(work list): %s", hipGetErrorString(e));
    if (run->plan_dev[next]) (void)hipFree(run->plan_dev[next]);  // unused: waited for above
    run->plan_dev[next] = grown;
    run->plan_capacity[next] = image.size();
  }
  if (plan.partials > run->partial_capacity) {
    // The installed plan may have launches in flight on this workspace: wait for them, then move
    // it to a larger one, which serves the installed plan as well as the new one.
    if (run->cur >= 0) HIP_TRY(ctx, wait_image(run, run->cur));
    void* grown = nullptr;
    hipError_t e = plan_malloc(&grown, (size_t)plan.partials * kPartialBytes);
    if (e != hipSuccess)
      return fail(ctx, QATTN_ENOMEM, "split workspace (%d chunks): %s", plan.partials, hipGetErrorString(e));
    if (run->split_dev) (void)hipFree(run->split_dev);
    run->split_dev = grown;
    run->partial_capacity = plan.partials;
    run->params.partials = static_cast<float*>(grown);
  }
  // Synchronous from pageable host memory: the image is on the device when this returns, and
  // the copy waits for nothing else on the device.
  HIP_TRY(ctx, hipMemcpy(run->plan_dev[next], image.data(), image.size(), hipMemcpyHostToDevice));
  // Commit.
  AttnParams p{};
  fill_params(&p, d, mask, info.slots, run->plan_dev[next], items_bytes, heads_bytes);
  p.partials = static_cast<float*>(run->split_dev);
  p.n_splits = plan.splits;
  run->params = p;
  run->cur = next;
  run->info = info;
  run->max_len = 0;
  for (int32_t s = 0; s < d->nseq; ++s) run->max_len = std::max(run->max_len, d->cu_seqlens[s + 1] - d->cu_seqlens[s]);
  run->desc = *d;
  run->desc.cu_seqlens = nullptr;
  run->desc.nseq = 0;
  return QATTN_OK;
}

// Enqueues `p` (the run's launch arguments, or a variant of them) on `stream` and notes the
// stream as one that reads image `cur` (a fence goes there when the image is retired).
int launch_run(qattn_run* run, const AttnParams& p, hipStream_t stream, bool merge) {
  qattn_ctx* ctx = run->ctx;
  auto& used = run->streams[run->cur];
  if (std::find(used.begin(), used.end(), stream) == used.end()) used.push_back(stream);
  HIP_TRY(ctx, launch_attn_fwd(p, stream));
  if (merge) HIP_TRY(ctx, launch_attn_merge(p, stream));
  return QATTN_OK;
}

void free_run(qattn_run* run) {
  DeviceGuard g(run->ctx->device);
  for (int i = 0; i < 2; ++i) {
    if (retire_image(run, i) != hipSuccess)
      for (hipStream_t s : run->streams[i]) (void)hipStreamSynchronize(s);
    (void)wait_image(run, i);
  }
  for (int i = 0; i < 2; ++i)
    if (run->plan_dev[i]) (void)hipFree(run->plan_dev[i]);
  if (run->split_dev) (void)hipFree(run->split_dev);
  delete run;
}

}  // namespace

extern "C" {

int qattn_run_create(qattn_ctx* ctx, const qattn_run_desc* d, qattn_run** out) {
  if (!ctx || !out) return fail(ctx, QATTN_EINVAL, "ctx/out is NULL");
  *out = nullptr;
  int rc = validate_desc(ctx, d);
  if (rc) return rc;
  auto* run = new (std::nothrow) qattn_run();
  if (!run) return fail(ctx, QATTN_ENOMEM, "out of host memory");
  run->ctx = ctx;
  rc = install_plan(run, d);
  if (rc) {
    free_run(run);
    return rc;
  }
  *out = run;
  return QATTN_OK;
}

int qattn_run_update(qattn_run* run, const int32_t* cu_seqlens, int32_t nseq) {
  if (!run) return fail(nullptr, QATTN_EINVAL, "run is NULL");
  qattn_run_desc d = run->desc;
  d.cu_seqlens = cu_seqlens;
  d.nseq = nseq;
  int rc = validate_desc(run->ctx, &d);
  if (rc) return rc;
  return install_plan(run, &d);
}

int qattn_run_encode(qattn_run* run, qattn_stream_t stream) {
  if (!run) return fail(nullptr, QATTN_EINVAL, "run is NULL");
  qattn_ctx* ctx = run->ctx;
  DeviceGuard g(ctx->device);
  return launch_run(run, run->params, pick_stream(ctx, stream), true);
}

int qattn_run_rebind(qattn_run* run, const void* q, const void* k, const void* v, void* o,
                     void* o_last) {
  if (!run) return fail(nullptr, QATTN_EINVAL, "run is NULL");
  if (!q || !k || !v || !o) return fail(run->ctx, QATTN_EINVAL, "q/k/v/o must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || (o_last && !aligned16(o_last)))
    return fail(run->ctx, QATTN_EINVAL, "q/k/v/o/o_last must be 16-byte aligned");
  if ((o_last != nullptr) != (run->desc.o_last != nullptr))
    return fail(run->ctx, QATTN_EINVAL, "o_last presence must match the run's description");
  AttnParams& p = run->params;
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v) + run->desc.v_offset;
  p.o = static_cast<half_t*>(o);
  p.o_last = static_cast<half_t*>(o_last);
  run->desc.q = q;
  run->desc.k = k;
  run->desc.v = v;
  run->desc.o = o;
  run->desc.o_last = o_last;
  return QATTN_OK;
}

void qattn_run_destroy(qattn_run* run) {
  if (run) free_run(run);
}

int qattn_run_get_info(const qattn_run* run, qattn_run_info* info) {
  if (!run || !info) return fail(nullptr, QATTN_EINVAL, "NULL argument");
  *info = run->info;
  return QATTN_OK;
}

int qattn_prefill(qattn_ctx* ctx, const qattn_run_desc* desc, qattn_stream_t stream) {
  qattn_run* run = nullptr;
  int rc = qattn_run_create(ctx, desc, &run);
  if (rc) return rc;
  rc = qattn_run_encode(run, stream);
  if (rc == QATTN_OK) {
    DeviceGuard g(ctx->device);
    hipError_t e = hipStreamSynchronize(pick_stream(ctx, stream));
    if (e != hipSuccess) rc = fail(ctx, QATTN_EHIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  }
  qattn_run_destroy(run);
  return rc;
}

int qattn_prefill_static(qattn_ctx* ctx, const qattn_run_desc* desc, qattn_stream_t stream) {
  if (!ctx) return fail(nullptr, QATTN_EINVAL, "ctx is NULL");
  if (!desc) return fail(ctx, QATTN_EINVAL, "desc is NULL");
  if (!ctx->scratch) return fail(ctx, QATTN_EHIP, "the static work list has no device address");
  // Batch-invariant plan: no split-K, so no partial results -- the work list is all it stores.
  qattn_run_desc d = *desc;
  d.flags |= QATTN_FLAG_BATCH_INVARIANT;
  Plan plan;
  qattn_run_info info{};
  MaskSpec mask{};
  int rc = validate_desc(ctx, &d);
  if (rc) return rc;
  plan_work(&d, std::max(1, ctx->cu_count) * kBlocksPerCU, &plan, &info, &mask);
  const size_t items_bytes = plan.items.size() * sizeof(WorkItem);
  const size_t slots_bytes = plan.slot_begin.size() * sizeof(int32_t);
  if (items_bytes + slots_bytes > kScratchBytes)
    return fail(ctx, QATTN_EINVAL,
                "%zu work entries exceed the static work list (%zu bytes, about %zu entries); use "
                "qattn_prefill or qattn_run_create",
                plan.items.size(), kScratchBytes, (kScratchBytes - 513 * sizeof(int32_t)) / sizeof(WorkItem));
  std::vector<char> host(items_bytes + slots_bytes);
  if (items_bytes) std::memcpy(host.data(), plan.items.data(), items_bytes);
  std::memcpy(host.data() + items_bytes, plan.slot_begin.data(), slots_bytes);
  AttnParams p{};
  fill_params(&p, &d, mask, info.slots, ctx->scratch, items_bytes, 0);
  DeviceGuard g(ctx->device);
  hipStream_t st = pick_stream(ctx, stream);
  HIP_TRY(ctx, hipMemcpyAsync(ctx->scratch, host.data(), host.size(), hipMemcpyHostToDevice, st));
  HIP_TRY(ctx, launch_attn_fwd(p, st));
  // Also keeps `host` alive until the copy has run, and the work list until the kernel is done.
  HIP_TRY(ctx, hipStreamSynchronize(st));
  return QATTN_OK;
}

// ---- mask check -------------------------------------------------------------------------------

int qattn_debug_xcd_map(qattn_ctx* ctx, int32_t n, int32_t* host_out) {
  if (!ctx || !host_out || n <= 0 || n > (1 << 20)) return fail(ctx, QATTN_EINVAL, "bad arguments");
  DeviceGuard g(ctx->device);
  int* dev = nullptr;
  HIP_TRY(ctx, hipMalloc(&dev, (size_t)n * sizeof(int)));
  hipError_t e = launch_xcd_map(dev, n, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(host_out, dev, (size_t)n * sizeof(int), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (e != hipSuccess) return fail(ctx, QATTN_EHIP, "xcd map: %s", hipGetErrorString(e));
  return QATTN_OK;
}

int qattn_debug_mask(qattn_ctx* ctx, int32_t L, int32_t mask, int32_t prefix, int32_t window,
                     uint32_t* host_bits) {
  if (!ctx) return fail(nullptr, QATTN_EINVAL, "ctx is NULL");
  if (L > 0 && !host_bits) return fail(ctx, QATTN_EINVAL, "host_bits is NULL");
  if (L < 0 || L > (1 << 20)) return fail(ctx, QATTN_EINVAL, "L=%d outside [0, 2^20]", L);
  if (mask != QATTN_MASK_CAUSAL && mask != QATTN_MASK_PREFIX_LOCAL)
    return fail(ctx, QATTN_EINVAL, "unknown mask kind %d", mask);
  if (mask == QATTN_MASK_PREFIX_LOCAL && (prefix < 0 || window < 0 || (prefix == 0 && window == 0)))
    return fail(ctx, QATTN_EINVAL, "bad prefix/window (%d, %d)", prefix, window);
  if (L == 0) return QATTN_OK;
  const int words = (L + 31) / 32;
  const size_t bytes = (size_t)words * L * sizeof(uint32_t);
  DeviceGuard g(ctx->device);
  uint32_t* dev = nullptr;
  HIP_TRY(ctx, hipMalloc(&dev, bytes));
  const MaskSpec m{mask, mask == QATTN_MASK_PREFIX_LOCAL ? prefix : 0, mask == QATTN_MASK_PREFIX_LOCAL ? window : 0};
  hipError_t e = hipMemsetAsync(dev, 0, bytes, ctx->stream);
  if (e == hipSuccess) e = launch_debug_mask(L, m, dev, words, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(host_bits, dev, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (e != hipSuccess) return fail(ctx, QATTN_EHIP, "debug mask: %s", hipGetErrorString(e));
  return QATTN_OK;
}

int qattn_debug_run_mask(qattn_run* run, uint32_t* host_bits, int64_t capacity_words,
                         int32_t* words_per_row) {
  if (!run) return fail(nullptr, QATTN_EINVAL, "run is NULL");
  qattn_ctx* ctx = run->ctx;
  const int32_t words = (run->max_len + 31) / 32;
  if (words_per_row) *words_per_row = words;
  if (!host_bits) return QATTN_OK;
  const int64_t T = run->info.tokens;
  const int64_t need = (int64_t)kQHeads * T * words;
  if (capacity_words < need)
    return fail(ctx, QATTN_EINVAL, "capacity %lld words < %lld (16 heads x %lld rows x %d)",
                (long long)capacity_words, (long long)need, (long long)T, words);
  if (need == 0) return QATTN_OK;
  DeviceGuard g(ctx->device);
  uint32_t* dev = nullptr;
  HIP_TRY(ctx, hipMalloc(&dev, (size_t)need * sizeof(uint32_t)));
  AttnParams p = run->params;
  p.o_last = nullptr;
  p.maskbits = dev;
  p.mask_rows = (int32_t)T;
  p.mask_words = words;
  // The attention kernel's mask variant, then (split plans) the merge kernel, so the output rows
  // are written as by qattn_run_encode.
  hipError_t e = hipMemsetAsync(dev, 0, (size_t)need * sizeof(uint32_t), ctx->stream);
  int rc = e == hipSuccess ? launch_run(run, p, ctx->stream, true) : QATTN_OK;
  if (e == hipSuccess && rc == QATTN_OK)
    e = hipMemcpyAsync(host_bits, dev, (size_t)need * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess && rc == QATTN_OK) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (rc != QATTN_OK) return rc;
  if (e != hipSuccess) return fail(ctx, QATTN_EHIP, "run mask: %s", hipGetErrorString(e));
  return QATTN_OK;
}

int qattn_debug_run_timeline(qattn_run* run, uint32_t* host_stamps, int64_t capacity_words, int32_t* slots) {
  if (!run) return fail(nullptr, QATTN_EINVAL, "run is NULL");
  qattn_ctx* ctx = run->ctx;
  const int32_t n = run->params.n_slots;
  if (slots) *slots = n;
  if (!host_stamps) return QATTN_OK;
  const int64_t need = (int64_t)n * kTimelineStamps;
  if (capacity_words < need)
    return fail(ctx, QATTN_EINVAL, "capacity %lld words < %lld (%d slots x %d stamps)", (long long)capacity_words,
                (long long)need, n, kTimelineStamps);
  if (need == 0) return QATTN_OK;
  DeviceGuard g(ctx->device);
  uint32_t* dev = nullptr;
  HIP_TRY(ctx, hipMalloc(&dev, (size_t)need * sizeof(uint32_t)));
  AttnParams p = run->params;
  p.timeline = dev;
  // The attention kernel's timeline variant, then (split plans) the merge kernel, so the output
  // rows are written as by qattn_run_encode.
  hipError_t e = hipMemsetAsync(dev, 0, (size_t)need * sizeof(uint32_t), ctx->stream);
  int rc = e == hipSuccess ? launch_run(run, p, ctx->stream, true) : QATTN_OK;
  if (e == hipSuccess && rc == QATTN_OK)
    e = hipMemcpyAsync(host_stamps, dev, (size_t)need * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess && rc == QATTN_OK) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (rc != QATTN_OK) return rc;
  if (e != hipSuccess) return fail(ctx, QATTN_EHIP, "run timeline: %s", hipGetErrorString(e));
  return QATTN_OK;
}

void qattn_debug_fail_allocs(int32_t n) { g_fail_allocs.store(n > 0 ? n : 0); }

int qattn_plan_mask(int32_t L, int32_t mask, int32_t prefix, int32_t window, uint32_t* host_bits) {
  if (L < 0 || L > (1 << 20)) return fail(nullptr, QATTN_EINVAL, "L=%d outside [0, 2^20]", L);
  if (L > 0 && !host_bits) return fail(nullptr, QATTN_EINVAL, "host_bits is NULL");
  if (mask != QATTN_MASK_CAUSAL && mask != QATTN_MASK_PREFIX_LOCAL)
    return fail(nullptr, QATTN_EINVAL, "unknown mask kind %d", mask);
  if (mask == QATTN_MASK_PREFIX_LOCAL && (prefix < 0 || window < 0 || (prefix == 0 && window == 0)))
    return fail(nullptr, QATTN_EINVAL, "bad prefix/window (%d, %d)", prefix, window);
  const MaskSpec m{mask, mask == QATTN_MASK_PREFIX_LOCAL ? prefix : 0, mask == QATTN_MASK_PREFIX_LOCAL ? window : 0};
  const int words = (L + 31) / 32;
  std::memset(host_bits, 0, (size_t)words * L * sizeof(uint32_t));
  for (int q = 0; q < L; ++q) kept_keys_row(q, L, m, host_bits + (size_t)q * words, words);
  return QATTN_OK;
}

// ---- producer + generator ---------------------------------------------------------------------

namespace {
// The context's RoPE table covering `positions` positions for `theta` (model.ts:76-81: angle =
// pos * theta^(-i/64) in f64, cos / sin rounded to f32), rebuilt only when it must grow or theta
// changes.  A rebuild uploads synchronously; every other call only reads it.
int rope_table(qattn_ctx* ctx, int32_t positions, double theta, const float2** out) {
  std::lock_guard<std::mutex> lock(ctx->mu);
  if (ctx->rope && ctx->rope_positions >= positions && ctx->rope_theta == theta) {
    *out = ctx->rope;
    return QATTN_OK;
  }
  const int32_t n = std::max(positions, std::max(ctx->rope_positions, 1024));
  std::vector<float2> table((size_t)n * 64);
  for (int32_t pos = 0; pos < n; ++pos)
    for (int i = 0; i < 64; ++i) {
      const double angle = (double)pos * std::pow(theta, -(double)i / 64.0);
      table[(size_t)pos * 64 + i] = float2{(float)std::cos(angle), (float)std::sin(angle)};
    }
  DeviceGuard g(ctx->device);
  float2* dev = nullptr;
  hipError_t e = hipMalloc(&dev, table.size() * sizeof(float2));
  if (e != hipSuccess) {
    ctx->last_error = std::string("RoPE table: ") + hipGetErrorString(e);
    g_last_error = ctx->last_error;
    return QATTN_ENOMEM;
  }
  e = hipMemcpy(dev, table.data(), table.size() * sizeof(float2), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    ctx->last_error = std::string("RoPE table upload: ") + hipGetErrorString(e);
    g_last_error = ctx->last_error;
    return QATTN_EHIP;
  }
  if (ctx->rope) (void)hipFree(ctx->rope);  // waits for the device to be idle first
  ctx->rope = dev;
  ctx->rope_positions = n;
  ctx->rope_theta = theta;
  *out = dev;
  return QATTN_OK;
}

int32_t longest(const int32_t* cu, int32_t nseq) {
  int32_t m = 0;
  for (int32_t s = 0; s < nseq; ++s) m = std::max(m, cu[s + 1] - cu[s]);
  return m;
}
}  // namespace

int qattn_qk_norm_rope(qattn_ctx* ctx, void* x, int64_t row_stride, int64_t col0, int32_t heads,
                       const int32_t* cu_seqlens, int32_t nseq, const float* weight, double eps,
                       double theta, qattn_stream_t stream) {
  if (!ctx || !x) return fail(ctx, QATTN_EINVAL, "ctx/x is NULL");
  if (heads < 4 || heads % 4 || heads > 32 || col0 < 0 || col0 % 8 || row_stride % 8 ||
      row_stride < col0 + (int64_t)heads * kHeadDim)
    return fail(ctx, QATTN_EINVAL, "bad heads/col0/row_stride (%d, %lld, %lld): heads a multiple of 4 in [4, 32], "
                "col0 and row_stride multiples of 8", heads, (long long)col0, (long long)row_stride);
  if (!aligned16(x) || (weight && reinterpret_cast<uintptr_t>(weight) % 16))
    return fail(ctx, QATTN_EINVAL, "x must be 16-byte aligned (weight too)");
  if (!(eps >= 0.0) || !(theta > 0.0)) return fail(ctx, QATTN_EINVAL, "bad eps/theta");
  int rc = validate_cu(ctx, cu_seqlens, nseq);
  if (rc) return rc;
  if (cu_seqlens[nseq] == 0) return QATTN_OK;
  const float2* table = nullptr;
  rc = rope_table(ctx, longest(cu_seqlens, nseq), theta, &table);
  if (rc) return rc;
  RopeArgs a{};
  a.in = static_cast<const half_t*>(x);
  a.out_q = a.out_k = static_cast<half_t*>(x) + col0;
  a.weight_q = a.weight_k = weight;
  a.rope = table;
  a.in_stride = a.out_stride_q = a.out_stride_k = row_stride;
  a.in_col_q = a.in_col_k = col0;
  a.heads = a.split = heads;
  a.eps = (float)eps;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_qk_norm_rope(a, cu_seqlens, nseq, pick_stream(ctx, stream)));
  return QATTN_OK;
}

int qattn_qk_norm_rope_qkv(qattn_ctx* ctx, const void* qkv, int64_t qkv_row_stride, void* q,
                           int64_t q_row_stride, void* k, int64_t k_row_stride,
                           const int32_t* cu_seqlens, int32_t nseq, const float* q_weight,
                           const float* k_weight, double eps, double theta, qattn_stream_t stream) {
  if (!ctx || !qkv || !q || !k) return fail(ctx, QATTN_EINVAL, "ctx/qkv/q/k is NULL");
  if (qkv_row_stride < 3072 || qkv_row_stride % 8 || q_row_stride < 2048 || q_row_stride % 8 ||
      k_row_stride < 1024 || k_row_stride % 8)
    return fail(ctx, QATTN_EINVAL, "strides (qkv %lld, q %lld, k %lld): >= 3072 / 2048 / 1024, multiples of 8",
                (long long)qkv_row_stride, (long long)q_row_stride, (long long)k_row_stride);
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) ||
      (q_weight && reinterpret_cast<uintptr_t>(q_weight) % 16) || (k_weight && reinterpret_cast<uintptr_t>(k_weight) % 16))
    return fail(ctx, QATTN_EINVAL, "qkv/q/k (and weights) must be 16-byte aligned");
  if (!(eps >= 0.0) || !(theta > 0.0)) return fail(ctx, QATTN_EINVAL, "bad eps/theta");
  int rc = validate_cu(ctx, cu_seqlens, nseq);
  if (rc) return rc;
  if (cu_seqlens[nseq] == 0) return QATTN_OK;
  const float2* table = nullptr;
  rc = rope_table(ctx, longest(cu_seqlens, nseq), theta, &table);
  if (rc) return rc;
  RopeArgs a{};
  a.in = static_cast<const half_t*>(qkv);
  a.out_q = static_cast<half_t*>(q);
  a.out_k = static_cast<half_t*>(k);
  a.weight_q = q_weight;
  a.weight_k = k_weight;
  a.rope = table;
  a.in_stride = qkv_row_stride;
  a.out_stride_q = q_row_stride;
  a.out_stride_k = k_row_stride;
  a.in_col_q = 0;                   // Q block of the qkvRaw row (model.ts:69)
  a.in_col_k = kQHeads * kHeadDim;  // K block
  a.heads = kQHeads + kKVHeads;     // 24 head vectors per token (the reference's dispatch, ops.ts:158)
  a.split = kQHeads;
  a.eps = (float)eps;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_qk_norm_rope(a, cu_seqlens, nseq, pick_stream(ctx, stream)));
  return QATTN_OK;
}

// ---- projection: Q4_0 tile32-compact dequant-GEMM -------------------------------------------------

int64_t qattn_q4_compact_bytes(int32_t K, int32_t N) {
  if (K < 32 || K % 32 || N < 1) return -1;
  return (int64_t)((N + 31) / 32) * (K / 32) * 32 * 20;
}

namespace {
// The checks both Q4_0 GEMM entry points share: N weight rows, y rows of at least `out_cols`.
int check_q4_args(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w, int64_t w_bytes,
                  int32_t N, int32_t out_cols, const void* y, int64_t ldy) {
  if (!ctx || !x || !w || !y) return fail(ctx, QATTN_EINVAL, "ctx/x/w/y is NULL");
  if (M < 0 || N < 1 || K < 32 || K % 32)
    return fail(ctx, QATTN_EINVAL, "shape M=%d K=%d N=%d: M >= 0, N >= 1, K a positive multiple of 32", M, K, N);
  if (ldx < K || ldx % 8 || ldy < out_cols || ldy % 8)
    return fail(ctx, QATTN_EINVAL, "ldx/ldy (%lld, %lld): >= K / %d and multiples of 8 elements", (long long)ldx,
                (long long)ldy, out_cols);
  const int64_t need = qattn_q4_compact_bytes(K, N);
  if (w_bytes < need || w_bytes > 0x7FFFFFFFll)
    return fail(ctx, QATTN_EINVAL, "w_bytes %lld: a %dx%d tile32-compact tensor holds %lld bytes (< 2 GiB)",
                (long long)w_bytes, N, K, (long long)need);
  if (((int64_t)M + 128) * ldx * 2 > 0x7FFFFFFFll || (int64_t)M * ldy * 2 > 0x7FFFFFFFll)
    return fail(ctx, QATTN_EINVAL, "x or y rows beyond 2 GiB (32-bit buffer offsets)");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16 || reinterpret_cast<uintptr_t>(w) % 4)
    return fail(ctx, QATTN_EINVAL, "x/y not 16-byte or w not 4-byte aligned");
  return QATTN_OK;
}
}  // namespace

}  // extern "C"

namespace qattn {
// qattn_q4_matmul with an optional split workspace (the model plan's): launches with few tiles
// split their K chunks over workgroups when ws holds q4_split_bytes.
int q4_matmul_ws(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w, int64_t w_bytes,
                 int32_t N, void* y, int64_t ldy, qattn_stream_t stream, float* ws, size_t ws_bytes,
                 const RowNorm* norm, bool* normed) {
  if (normed) *normed = false;
  const int rc = check_q4_args(ctx, x, ldx, M, K, w, w_bytes, N, N, y, ldy);
  if (rc != QATTN_OK) return rc;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_q4_matmul(static_cast<const half_t*>(x), ldx, M, K, static_cast<const uint8_t*>(w),
                                (uint32_t)w_bytes, N, static_cast<half_t*>(y), ldy, pick_stream(ctx, stream), ws,
                                ws_bytes, norm, normed));
  return QATTN_OK;
}
}  // namespace qattn

extern "C" {

int qattn_q4_matmul(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w,
                    int64_t w_bytes, int32_t N, void* y, int64_t ldy, qattn_stream_t stream) {
  return qattn::q4_matmul_ws(ctx, x, ldx, M, K, w, w_bytes, N, y, ldy, stream, nullptr, 0);
}

int qattn_q4_matmul_swiglu(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w,
                           int64_t w_bytes, int32_t n_inter, void* y, int64_t ldy, qattn_stream_t stream) {
  if (n_inter < 64 || n_inter % 64 || n_inter > (1 << 29))
    return fail(ctx, QATTN_EINVAL, "n_inter %d: a positive multiple of 64", n_inter);
  const int rc = check_q4_args(ctx, x, ldx, M, K, w, w_bytes, 2 * n_inter, n_inter, y, ldy);
  if (rc != QATTN_OK) return rc;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_q4_matmul_swiglu(static_cast<const half_t*>(x), ldx, M, K, static_cast<const uint8_t*>(w),
                                       (uint32_t)w_bytes, n_inter, static_cast<half_t*>(y), ldy,
                                       pick_stream(ctx, stream)));
  return QATTN_OK;
}

// ---- consumer: last-token pool + L2 normalisation ----------------------------------------------

int qattn_pool_last_l2(qattn_ctx* ctx, const void* x, int64_t row_stride, int32_t width,
                       const int32_t* cu_seqlens, int32_t nseq, float* out, int64_t out_row_stride,
                       qattn_stream_t stream) {
  if (!ctx || !x || !out) return fail(ctx, QATTN_EINVAL, "ctx/x/out is NULL");
  if (width < 8 || width % 8 || row_stride < width || row_stride % 8)
    return fail(ctx, QATTN_EINVAL, "width/row_stride (%d, %lld): width >= 8, both multiples of 8 elements, "
                "row_stride >= width", width, (long long)row_stride);
  if (out_row_stride < width || out_row_stride % 4)
    return fail(ctx, QATTN_EINVAL, "out_row_stride %lld: >= width and a multiple of 4", (long long)out_row_stride);
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail(ctx, QATTN_EINVAL, "x/out not 16-byte aligned");
  int rc = validate_cu(ctx, cu_seqlens, nseq);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_pool_last_l2(static_cast<const half_t*>(x), row_stride, width, cu_seqlens, nseq, out,
                                   out_row_stride, pick_stream(ctx, stream)));
  return QATTN_OK;
}

int qattn_fill_normal(qattn_ctx* ctx, void* dst, int64_t rows, int64_t row_elems,
                      int64_t row_stride, uint64_t seed, qattn_stream_t stream) {
  if (!ctx || !dst) return fail(ctx, QATTN_EINVAL, "ctx/dst is NULL");
  if (rows < 0 || row_elems < 0 || row_stride < row_elems)
    return fail(ctx, QATTN_EINVAL, "bad rows/row_elems/row_stride");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_fill_normal(static_cast<half_t*>(dst), rows, row_elems, row_stride, seed,
                                  pick_stream(ctx, stream)));
  return QATTN_OK;
}

int qattn_fill_token_rows(qattn_ctx* ctx, void* dst, const int32_t* ids, int64_t rows,
                          int64_t row_elems, int64_t row_stride, uint64_t seed,
                          qattn_stream_t stream) {
  if (!ctx || !dst || (!ids && rows)) return fail(ctx, QATTN_EINVAL, "NULL argument");
  if (rows < 0 || row_elems < 0 || row_stride < row_elems)
    return fail(ctx, QATTN_EINVAL, "bad rows/row_elems/row_stride");
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, launch_fill_token_rows(static_cast<half_t*>(dst), ids, rows, row_elems, row_stride,
                                      seed, pick_stream(ctx, stream)));
  return QATTN_OK;
}

int qattn_gen_qkv(qattn_ctx* ctx, uint32_t config, uint32_t layer, const int32_t* cu_seqlens,
                  int32_t nseq, void* q, int64_t q_row_stride, void* k, int64_t k_row_stride,
                  void* v, int64_t v_row_stride, qattn_stream_t stream) {
  if (!ctx || !q || !k || !v) return fail(ctx, QATTN_EINVAL, "NULL argument");
  int rc = validate_cu(ctx, cu_seqlens, nseq);
  if (rc) return rc;
  if (q_row_stride < 2048 || k_row_stride < 1024 || v_row_stride < 1024)
    return fail(ctx, QATTN_EINVAL, "row strides too small");
  const int64_t T = cu_seqlens[nseq];
  const uint64_t base = 0x51574E3300000000ULL | ((uint64_t)(config & 0xff) << 16) | ((uint64_t)(layer & 0xff) << 8);
  rc = qattn_fill_normal(ctx, q, T, 2048, q_row_stride, base | 0, stream);
  if (!rc) rc = qattn_fill_normal(ctx, k, T, 1024, k_row_stride, base | 1, stream);
  if (!rc) rc = qattn_fill_normal(ctx, v, T, 1024, v_row_stride, base | 2, stream);
  if (!rc) rc = qattn_qk_norm_rope(ctx, q, q_row_stride, 0, 16, cu_seqlens, nseq, nullptr, 1e-6, 1e6, stream);
  if (!rc) rc = qattn_qk_norm_rope(ctx, k, k_row_stride, 0, 8, cu_seqlens, nseq, nullptr, 1e-6, 1e6, stream);
  return rc;
}

// ---- timing -------------------------------------------------------------------------------------

int qattn_event_create(qattn_ctx* ctx, qattn_event_t* ev) {
  if (!ctx || !ev) return fail(ctx, QATTN_EINVAL, "NULL argument");
  DeviceGuard g(ctx->device);
  hipEvent_t e = nullptr;
  HIP_TRY(ctx, hipEventCreate(&e));
  *ev = e;
  return QATTN_OK;
}

int qattn_event_record(qattn_event_t ev, qattn_stream_t stream) {
  if (!ev) return fail(nullptr, QATTN_EINVAL, "event is NULL");
  HIP_TRY(nullptr, hipEventRecord(reinterpret_cast<hipEvent_t>(ev), reinterpret_cast<hipStream_t>(stream)));
  return QATTN_OK;
}

int qattn_event_elapsed_ms(qattn_event_t a, qattn_event_t b, float* ms) {
  if (!a || !b || !ms) return fail(nullptr, QATTN_EINVAL, "NULL argument");
  HIP_TRY(nullptr, hipEventSynchronize(reinterpret_cast<hipEvent_t>(b)));
  HIP_TRY(nullptr, hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(a), reinterpret_cast<hipEvent_t>(b)));
  return QATTN_OK;
}

int qattn_event_synchronize(qattn_event_t ev) {
  if (!ev) return fail(nullptr, QATTN_EINVAL, "event is NULL");
  HIP_TRY(nullptr, hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev)));
  return QATTN_OK;
}

int qattn_event_destroy(qattn_event_t ev) {
  if (!ev) return QATTN_OK;
  HIP_TRY(nullptr, hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  return QATTN_OK;
}

}  // extern "C"
