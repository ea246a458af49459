/*
 * qattn.h -- C ABI of the MI355X (gfx950) causal GQA prefill attention library.
 *
 * Drop-in for the attention path of the reference engine (paths are relative to the reference
 * checkout, shihanqu/qwen3-embedding-webgpu-prepacked):
 *
 *   reference                                           | this ABI
 *   ----------------------------------------------------+-------------------------------------
 *   requestWebGPUDevice()              device.ts:6-24   | qattn_create / qattn_destroy
 *   createBufferWithData / createBuffer device.ts:26-37 | qattn_buffer_alloc / _write / _read
 *   CausalAttentionKernel.createRun    ops.ts:327-343   | qattn_run_create
 *   CausalAttentionKernel.encode       ops.ts:344       | qattn_run_encode
 *   plan.destroy() of run.ownedBuffers model.ts:108-111 | qattn_run_destroy
 *   tiled flash attention shader       ops.ts:168-241   | kernel behind qattn_run_encode
 *   mask predicate + tile skip         ops.ts:205-220   | qattn_debug_run_mask (executed), _debug_mask
 *   QKNormRopeKernel                   ops.ts:104-166   | qattn_qk_norm_rope_qkv (_rope in place)
 *   RoPE table                         model.ts:76-83   | cached per context by the producer
 *   last-token row of poolShader       ops.ts:357       | qattn_run_desc.o_last
 *   LastTokenPoolKernel (L2 norm)      ops.ts:347-379   | qattn_pool_last_l2
 *   compact Q4_0 batch matmul   quant-matmul.ts:267-307 | qattn_q4_matmul
 *   EmbeddingLookupKernel (Q6_K)       ops.ts:381-423   | qattn_embed_q6k
 *   RmsNormKernel (residual + norm)    ops.ts:21-72     | qattn_rmsnorm
 *   SwiGLUKernel                       ops.ts:74-102    | qattn_swiglu
 *   gate/up matmul + SwiGLUKernel      model.ts:126-127 | qattn_q4_matmul_swiglu (fused)
 *   Qwen3WebGPUModel (weights)         model.ts:185-255 | qattn_model_create / _destroy
 *   Qwen3ExecutionPlan (28 layers)     model.ts:49-139  | qattn_model_plan_create / _run / _destroy
 *   Qwen3ExecutionPlan.profile()       model.ts:141-182 | qattn_model_plan_profile
 *
 * Fixed model geometry (model.ts:18-23, ops.ts:196): 16 query heads, 8 KV heads (query head h
 * reads KV head h/2), head_dim 128, scale 1/sqrt(128), fp16 storage, fp32 accumulation.
 *
 * Conventions: every function returns QATTN_OK (0) or a negative status; the message of the
 * last failure is available from qattn_last_error(ctx) (thread-local when ctx is NULL).
 * Arguments are validated on the host before any launch.  A context owns one HIP stream
 * created with the default priority; `stream == NULL` in an entry point means that stream.
 * Device pointers are plain `void*` device addresses (from qattn_buffer_alloc or any other HIP
 * allocation on the same device).
 */
#ifndef QATTN_H
#define QATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 4: qattn_qk_norm_rope_qkv, qattn_run_update; qattn_qk_norm_rope takes heads in multiples of 4
 * 5: the model forward: qattn_embed_q6k, qattn_rmsnorm, qattn_swiglu, qattn_model_*,
 *    qattn_model_plan_*
 * 6: qattn_q4_matmul_swiglu; the model plan's FFN gate/up projection and SwiGLU are one launch
 * 7: qattn_run_update no longer waits for the device (two work-list images per run);
 *    qattn_debug_fail_allocs
 * 8: qattn_debug_run_timeline
 * 9: qattn_buffer_read_after, qattn_event_synchronize */
#define QATTN_ABI_VERSION 9

#define QATTN_Q_HEADS 16
#define QATTN_KV_HEADS 8
#define QATTN_HEAD_DIM 128
#define QATTN_MAX_SEQS 65536

enum qattn_status {
  QATTN_OK = 0,
  QATTN_EINVAL = -1, /* bad argument (shape, stride, alignment, cu_seqlens, mask) */
  QATTN_EHIP = -2,   /* HIP runtime error */
  QATTN_ENOMEM = -3, /* device or host allocation failed */
  QATTN_ENODEV = -4  /* no usable gfx950 device */
};

enum qattn_mask_kind {
  QATTN_MASK_CAUSAL = 0,       /* k <= q */
  QATTN_MASK_PREFIX_LOCAL = 1  /* k <= q && (k < prefix || q - k < window): ops.ts:206,220 */
};

typedef struct qattn_ctx qattn_ctx;
typedef struct qattn_run qattn_run;
typedef void* qattn_stream_t; /* a hipStream_t */

/* ---- device context  (replaces requestWebGPUDevice, device.ts:6-24) --------------------- */
int qattn_create(int device, qattn_ctx** out);
void qattn_destroy(qattn_ctx* ctx);
const char* qattn_last_error(const qattn_ctx* ctx);
int qattn_abi_version(void);
qattn_stream_t qattn_stream(qattn_ctx* ctx);
int qattn_synchronize(qattn_ctx* ctx);
/* gcnArchName (e.g. "gfx950:sramecc+:xnack-") and the CU count of the context's device. */
int qattn_device_name(qattn_ctx* ctx, char* buf, size_t len, int* cu_count);

/* ---- device buffers  (replaces createBuffer / createBufferWithData, device.ts:26-37, and
 *      queue.writeBuffer / mapAsync readback, model.ts:115-116,135) ----------------------- */
typedef void* qattn_event_t; /* a HIP event (qattn_event_create, timing section below) */
int qattn_buffer_alloc(qattn_ctx* ctx, size_t bytes, void** dptr);
int qattn_buffer_free(qattn_ctx* ctx, void* dptr);
/* Synchronous on the context stream. */
int qattn_buffer_write(qattn_ctx* ctx, void* dst, size_t offset, const void* src, size_t bytes);
int qattn_buffer_read(qattn_ctx* ctx, const void* src, size_t offset, void* dst, size_t bytes);
int qattn_buffer_fill_u16(qattn_ctx* ctx, void* dst, uint16_t value, size_t count);
/* The readback of one submit (the reference copies the embeddings into its readback buffer in the
 * same submit and maps it, model.ts:133-135): copies `bytes` from src + offset to host memory dst
 * once the work recorded before event `after` (qattn_event_record on the context stream) has
 * finished, on a stream of the context's own for readbacks, so work enqueued on the context stream
 * after that event (the next batch) is not waited for.  Blocks until the copy is done; safe to call
 * from another host thread while this one enqueues, as long as src stays allocated and ctx alive
 * until it returns. */
int qattn_buffer_read_after(qattn_ctx* ctx, qattn_event_t after, const void* src, size_t offset,
                            void* dst, size_t bytes);

/* ---- attention operator  (replaces CausalAttentionKernel, ops.ts:318-345) ---------------- */
typedef struct qattn_run_desc {
  /* fp16 device tensors.  Token t of the packed batch is row t.  Head h of Q/O is the 128
   * halves at element t*row_stride + h*128; KV head g of K at t*k_row_stride + g*128 and of V at
   * v_offset + t*v_row_stride + g*128 (the reference reads V in place from qkvRaw with
   * value_stride 4096 / value_offset 3072, model.ts:95).  Pointers 16-byte aligned; strides and
   * v_offset multiples of 8 elements; q/o strides >= 2048, k/v strides >= 1024. */
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t q_row_stride, k_row_stride, v_row_stride, o_row_stride, v_offset;
  /* Host array of nseq+1 non-decreasing token offsets starting at 0: sequence i is rows
   * cu_seqlens[i] .. cu_seqlens[i+1]-1 and attends only within itself (positions restart at 0).
   * Replaces the reference's padded [batch, sequence] layout (ops.ts:200,213).  Copied. */
  const int32_t* cu_seqlens;
  int32_t nseq;
  int32_t mask;    /* enum qattn_mask_kind */
  int32_t prefix;  /* PREFIX_LOCAL: keys 0..prefix-1 always visible (reference 176) */
  int32_t window;  /* PREFIX_LOCAL: keys q-window+1..q visible (reference 432) */
  /* Optional fp16 [nseq][16*128] device output: row i receives O of token cu_seqlens[i+1]-1,
   * the row the reference's last-token pool reads (ops.ts:357).  NULL to skip. */
  void* o_last;
  /* enum qattn_run_flags (0: defaults). */
  int32_t flags;
} qattn_run_desc;

enum qattn_run_flags {
  /* Never split an item's key tiles across workgroups (split-K).  Every output row is then
   * computed by one pass in a fixed order, so a sequence gives bitwise the same result alone or
   * in any batch, as the reference does; without the flag the planner may split long items to
   * balance the GPU, and results stay deterministic for a given batch but may differ from another
   * batch's in the last fp16 bit. */
  QATTN_FLAG_BATCH_INVARIANT = 1
};

/* Plans the launch (validates, builds the work list of (sequence, kv_head, query block) items,
 * spreads it over persistent workgroups -- "slots", two per compute unit -- longest first with
 * each KV head's items on one XCD, splitting long items' key tiles over several slots unless
 * QATTN_FLAG_BATCH_INVARIANT, uploads it) and returns a run that owns its device work list and
 * split-K workspace. */
int qattn_run_create(qattn_ctx* ctx, const qattn_run_desc* desc, qattn_run** out);
/* Enqueues the attention kernel of a run on `stream` (NULL: the context stream), followed by the
 * split-K merge kernel when the plan splits items.  Launches of one run must not overlap on the
 * device (one stream, or streams the caller orders): a split plan's launches share the run's
 * partial-result workspace. */
int qattn_run_encode(qattn_run* run, qattn_stream_t stream);
/* Re-points a run at other tensors of the same shape (layers sharing one packing). */
int qattn_run_rebind(qattn_run* run, const void* q, const void* k, const void* v, void* o,
                     void* o_last);
/* Re-plans a run for new sequence lengths: same tensors, strides, mask and flags, new cu_seqlens
 * (validated as by qattn_run_create).  The reference creates a run per (batch, sequence) plan
 * shape and rebuilds its uniforms per batch (embedding-engine.ts:70-75, ops.ts:327-343); a
 * varlen batch changes the work list, so one run kept at capacity takes every batch of a plan.
 * The run keeps two work-list images: the new plan is uploaded (synchronously) into the one the
 * installed plan does not use, after waiting only for the earlier launches of this run that read
 * that image -- never for the device or other streams -- and the run switches to it once the
 * upload succeeded.  To know when those launches end, the update records an event on each stream
 * the installed plan was encoded on: those streams must still exist when the run is updated or
 * destroyed.  Device memory is allocated only when the work list or the split workspace
 * outgrows every earlier one (and hipFree of the outgrown buffer may then wait for the device).
 * On failure the run keeps its previous plan, intact and usable.  The tensors must hold the new
 * token count. */
int qattn_run_update(qattn_run* run, const int32_t* cu_seqlens, int32_t nseq);
void qattn_run_destroy(qattn_run* run);

typedef struct qattn_run_info {
  int64_t tokens;           /* sum of sequence lengths */
  int64_t pairs;            /* retained (query, key) pairs summed over sequences */
  int64_t flops;            /* 4 * 128 * 16 * pairs: QK^T and PV over all query heads */
  int64_t bytes;            /* 12288 * tokens (+ 4096 per sequence with o_last): Q,K,V,O fp16 */
  int32_t work_items;       /* (sequence, kv_head, 64-query block) items */
  int32_t block_queries;    /* query positions per work item */
  int64_t tile_pairs;       /* (query, key) pairs inside the MFMA tiles computed, per query head */
  int32_t slots;            /* persistent workgroups launched (each runs a list of entries) */
  int32_t split_items;      /* items whose key tiles are spread over several entries (split-K) */
} qattn_run_info;
int qattn_run_get_info(const qattn_run* run, qattn_run_info* info);

/* Host-only planning (no device needed): validates `desc` exactly as qattn_run_create does and
 * reports the work list a run on an MI355X (256 compute units, 512 slots) would upload: entries
 * grouped by slot, heaviest first within a slot.  Each entry is eight int32:
 * {first token of the sequence, sequence length, query block, sequence<<4 | kv_head,
 *  first key tile, end key tile (indices into the item's visited key tiles), split, part}.
 * An item spread over several entries (chunks, split-K) has split >= 0 (shared by its chunks) and
 * part = chunk index | chunk count << 4 | first partial-result index << 8; otherwise split = -1,
 * part = 0 and the entry covers all of the item's tiles.  `items` may be NULL (count only);
 * `*count` receives the number of entries, `info` (optional) the run's figures.  Fails with
 * QATTN_EINVAL if `capacity` (entries) is too small for a non-NULL `items`.
 * Replaces the reference's dispatch-size computation (ops.ts:329-343). */
int qattn_plan_describe(const qattn_run_desc* desc, int32_t* items, int32_t capacity,
                        int32_t* count, qattn_run_info* info);
/* The slot structure of the same plan for at most `max_slots` workgroups (<= 0: 512): slot b
 * runs entries slot_begin[b] .. slot_begin[b+1]-1 of qattn_plan_describe's list and is dispatched
 * to XCD b % 8.  `*nslots` receives the slot count; `slot_begin` (optional, `capacity` >=
 * nslots + 1 entries) the offsets. */
int qattn_plan_slots(const qattn_run_desc* desc, int32_t max_slots, int32_t* slot_begin,
                     int32_t capacity, int32_t* nslots);

/* One-shot: create, encode, wait for completion, destroy. */
int qattn_prefill(qattn_ctx* ctx, const qattn_run_desc* desc, qattn_stream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): qattn_prefill with no
 * device allocation or free.  The plan is always batch-invariant (no split-K), so the output is
 * bitwise that of qattn_prefill with QATTN_FLAG_BATCH_INVARIANT set.  Its work list goes to a
 * fixed 1 MiB array in the library's device image (one per GPU, kept until the process ends):
 * launches of more than about 32000 work entries (64-query blocks x 8 KV heads, roughly 250k
 * tokens) are rejected with QATTN_EINVAL.  Every call on one GPU uses that GPU's array, so calls
 * that overlap on one GPU (other threads or streams) race; each call waits for its stream before
 * returning.  Host-side planning uses host memory only. */
int qattn_prefill_static(qattn_ctx* ctx, const qattn_run_desc* desc, qattn_stream_t stream);

/* ---- mask check  (same device predicate and key-tile iterator as the attention kernel) ---- */
/* Diagnostic, no counterpart in the reference: the XCD (hardware XCC_ID) that each of n
 * workgroups of a launch shaped like the attention kernel's runs on.  The planner keeps each KV
 * head's work on slots b with one value of b % 8, expecting round-robin dispatch (workgroup b on
 * XCD b % number-of-XCDs) to keep that head's K/V in one L2; this makes the expectation testable.
 * (Only locality depends on it, not results.) */
int qattn_debug_xcd_map(qattn_ctx* ctx, int32_t n, int32_t* host_out);

/* Writes the retained-key bitmask of one sequence of length L to host memory: word
 * q*ceil(L/32) + k/32, bit k%32 set iff the attention kernel visits key k for query q and keeps
 * it.  Must equal the reference predicate ops.ts:205-209,219-220 bit for bit. */
int qattn_debug_mask(qattn_ctx* ctx, int32_t L, int32_t mask, int32_t prefix, int32_t window,
                     uint32_t* host_bits);

/* Failure injection, no counterpart in the reference: the next n device allocations that
 * qattn_run_create / qattn_run_update make for a work list or split workspace fail as if the
 * device were out of memory (QATTN_ENOMEM).  n = 0 cancels.  Lets tests drive the error paths
 * of a re-plan; process-wide, not for production use. */
void qattn_debug_fail_allocs(int32_t n);

/* Host evaluation of the same iteration code (attn_common.h is compiled for host and device):
 * no device needed.  Same output layout as qattn_debug_mask. */
int qattn_plan_mask(int32_t L, int32_t mask, int32_t prefix, int32_t window, uint32_t* host_bits);

/* The retained-key set the attention kernel itself executes for a run (mask predicate
 * ops.ts:205-209,219-220): runs the run's plan once through a variant of the attention kernel
 * that also records, for every query head h, packed row t and key k of t's sequence, bit k%32
 * of word host_bits[(h*T + t)*W + k/32] iff the masked score it computed for (t, k) is finite
 * (T = tokens, W = *words_per_row = ceil(longest sequence / 32)).  The run's output buffers are
 * written as by qattn_run_encode (split plans: the merge kernel runs too; o_last excepted).
 * host_bits NULL: only *words_per_row.
 * Allocates a device buffer and synchronizes; a diagnostic, not for the hot path. */
int qattn_debug_run_mask(qattn_run* run, uint32_t* host_bits, int64_t capacity_words,
                         int32_t* words_per_row);
/* Phase timeline of one launch of a run -- no reference counterpart (a profiling aid for the
 * attention kernel, as the reference's profile() times whole stages, model.ts:141-182).  Runs the
 * kernel's timeline variant (same output rows; split plans: the merge kernel too) and returns
 * 128 uint32 per slot (workgroup) b at host_stamps[128 b]: s_memrealtime ticks (100 MHz) at
 * 0 start, 1 first loads landed, and per entry e < 15 of the slot at 2 + 8 e: +0 entry top,
 * +1 after its first tile's barrier, +2 after its last tile's barrier, +3 after that tile issued
 * the next entry's loads, +4 after the entry's last PV, +5 after the hand-over wait, +6 after
 * the rows were staged (partials stored) and the next S(0) issued, +7 after the row stores
 * (entries past 14 overwrite entry 14's); 127 end.  Unreached stamps are 0.  *slots receives
 * the slot count; host_stamps NULL: only *slots.  capacity_words >= 128 * slots.
 * Allocates a device buffer and synchronizes; a diagnostic, not for the hot path. */
int qattn_debug_run_timeline(qattn_run* run, uint32_t* host_stamps, int64_t capacity_words,
                             int32_t* slots);

/* ---- producer: QK RMSNorm + RoPE  (replaces QKNormRopeKernel, ops.ts:104-166) ------------- */
/* Reads the Q block (16 heads, columns 0..2047) and K block (8 heads, 2048..3071) of each qkvRaw
 * row (model.ts:69; row t at qkv + t*qkv_row_stride) and writes compact Q [T,16,128] and K
 * [T,8,128] (row strides q_row_stride >= 2048, k_row_stride >= 1024): per 128-wide head vector,
 * RMSNorm with eps and gain (q_weight / k_weight: f32[128] device arrays, NULL for 1), then NeoX
 * rotate-half RoPE with theta at the token's position inside its sequence -- the reference's
 * createRun(input, qWeight, kWeight, qOutput, kOutput, tokens, sequence, epsilon, ropeTable,
 * inputStride) (ops.ts:157-165), in f32 as its shader.  The RoPE table (model.ts:76-83) is
 * built once per context and rebuilt only when a longer sequence or another theta arrives;
 * otherwise the call only enqueues (one launch per 64 sequences).  Pointers 16-byte aligned,
 * strides multiples of 8 elements. */
int qattn_qk_norm_rope_qkv(qattn_ctx* ctx, const void* qkv, int64_t qkv_row_stride, void* q,
                           int64_t q_row_stride, void* k, int64_t k_row_stride,
                           const int32_t* cu_seqlens, int32_t nseq, const float* q_weight,
                           const float* k_weight, double eps, double theta, qattn_stream_t stream);
/* The same math in place on one block of `heads` head vectors (a multiple of 4) per row, at
 * element t*row_stride + col0 + h*128 (col0, row_stride multiples of 8), one gain for all. */
int qattn_qk_norm_rope(qattn_ctx* ctx, void* x, int64_t row_stride, int64_t col0, int32_t heads,
                       const int32_t* cu_seqlens, int32_t nseq, const float* weight, double eps,
                       double theta, qattn_stream_t stream);

/* ---- projection: Q4_0 tile32-compact dequant-GEMM  (replaces the compact batch matmul, ------ */
/* ---- quant-matmul.ts:267-307, over the layout of packQ40Tile32, prepacked/format.ts:64-96) -- */
/* Bytes of an N x K weight tensor in the q4_0-tile32-compact layout: ceil(N/32) tiles of K/32
 * blocks of 32 records of 20 bytes (-1 if K is not a positive multiple of 32 or N < 1). */
int64_t qattn_q4_compact_bytes(int32_t K, int32_t N);
/* y[m*ldy + n] = f16(sum over k < K of x[m*ldx + k] * W(n, k)) for m < M, n < N, where
 * W(n, k) = f16(scale * (q - 8)) from record ((n/32)*(K/32) + k/32)*32 + n%32 of `w`: the f16
 * scale in bytes 0-1, element j of the 32-column block in the low nibble of byte 4+j, element
 * j+16 in its high nibble (the reference's dequant, quant-matmul.ts:99-108).  Products and sums
 * in fp32 (the reference accumulates in f16).  x, y: fp16 device rows, 16-byte aligned, ldx >= K
 * and ldy >= N multiples of 8 elements; w: device, 4-byte aligned, w_bytes >=
 * qattn_q4_compact_bytes(K, N).  Enqueued on `stream` (NULL: the context stream); allocates
 * nothing. */
int qattn_q4_matmul(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w,
                    int64_t w_bytes, int32_t N, void* y, int64_t ldy, qattn_stream_t stream);
/* The FFN's gate/up projection and SwiGLU in one launch (the reference runs its compact matmul
 * into a [T, 2 n_inter] buffer, then SwiGLUKernel, model.ts:126-127, ops.ts:74-102):
 * y[m*ldy + j] = qattn_swiglu's value of (g, u) = (G[m][j], G[m][n_inter + j]) for j < n_inter,
 * where G is what qattn_q4_matmul writes for the 2 n_inter-row weight `w` (gate rows, then up
 * rows).  The same fp16 roundings and formula, so the result equals qattn_q4_matmul followed by
 * qattn_swiglu bit for bit, without the [M, 2 n_inter] intermediate.  n_inter a positive
 * multiple of 64; ldy >= n_inter; the other rules of qattn_q4_matmul with N = 2 n_inter. */
int qattn_q4_matmul_swiglu(qattn_ctx* ctx, const void* x, int64_t ldx, int32_t M, int32_t K, const void* w,
                           int64_t w_bytes, int32_t n_inter, void* y, int64_t ldy, qattn_stream_t stream);

/* ---- consumer: last-token pool + L2 norm  (replaces LastTokenPoolKernel, ops.ts:347-379) --- */
/* For each sequence i < nseq: out[i*out_row_stride + d] = f32(x[r*row_stride + d]) * s for
 * d < width, r = cu_seqlens[i+1]-1 (the reference's row b*S + lengths[b]-1 of its padded layout,
 * ops.ts:357) and s = 1/sqrt(sum over d of f32(x)^2) (ops.ts:358-363).  As in the reference there
 * is no epsilon: an all-zero row gives NaN.  An empty sequence (no last token; the reference
 * never forms one) gets a row of zeros.  x: fp16 device rows, out: f32 device rows, both 16-byte
 * aligned; width and row_stride multiples of 8 elements, out_row_stride >= width and a multiple
 * of 4.  Enqueued on `stream` (NULL: the context stream); allocates nothing. */
int qattn_pool_last_l2(qattn_ctx* ctx, const void* x, int64_t row_stride, int32_t width,
                       const int32_t* cu_seqlens, int32_t nseq, float* out, int64_t out_row_stride,
                       qattn_stream_t stream);

/* ---- the model forward around the attention path  (model.ts:18-23, 49-183) ----------------- */
#define QATTN_HIDDEN 1024       /* model.ts:18 */
#define QATTN_INTERMEDIATE 3072 /* model.ts:19 */
#define QATTN_MAX_LAYERS 28     /* model.ts:21 */
#define QATTN_Q6K_BLOCK_BYTES 210

/* out[t*out_row_stride + c] = row ids[t] of a Q6_K table, dequantised as the reference's
 * embedding shader does (ops.ts:381-412): value i = 128h + 32quad + l of a 256-value block is
 * f16(f32(d) * f32(scale[8h + l/16 + 2quad]) * f32(q - 32)), q the 6-bit code of ql / qh.  `ids`:
 * device int32 [tokens]; ids outside [0, vocab) give zero rows (the model plan rejects them on the
 * host first).  `table`: device, width/256 blocks of 210 bytes per row, vocab = table_bytes /
 * (width/256 * 210) rows; width a multiple of 256; out 16-byte aligned, out_row_stride a multiple
 * of 8 and >= width.  Enqueued on `stream`; allocates nothing. */
int qattn_embed_q6k(qattn_ctx* ctx, const int32_t* ids, int64_t tokens, const void* table,
                    int64_t table_bytes, int32_t width, void* out, int64_t out_row_stride,
                    qattn_stream_t stream);
/* Residual add + RMSNorm of `rows` fp16 rows of `width` (ops.ts:21-57): with a residual,
 * v = f32(x) + f32(residual) and x <- f16(v) in place; without, v = f32(x).  Then
 * out = f16(f32(x) * inv * weight[c]) with inv = 1/sqrt(sum(v^2)/width + eps), the sum over the
 * unrounded v as in the reference.  weight: device f32 [width]; residual may be NULL; out may
 * not alias x.  width a multiple of 8, <= 4096; pointers 16-byte aligned; strides multiples of 8
 * elements.  Enqueued on `stream`; allocates nothing. */
int qattn_rmsnorm(qattn_ctx* ctx, void* x, int64_t x_row_stride, const void* residual,
                  int64_t residual_row_stride, const float* weight, void* out,
                  int64_t out_row_stride, int64_t rows, int32_t width, double eps,
                  qattn_stream_t stream);
/* out[r][c] = f16(silu(g) * u), g = gate_up[r][c], u = gate_up[r][width + c], silu(g) =
 * g / (1 + exp(-g)) in f32 (ops.ts:74-89).  width a multiple of 8; gate_up_row_stride >=
 * 2*width, out_row_stride >= width, multiples of 8; pointers 16-byte aligned.  Enqueued on
 * `stream`; allocates nothing. */
int qattn_swiglu(qattn_ctx* ctx, const void* gate_up, int64_t gate_up_row_stride, void* out,
                 int64_t out_row_stride, int64_t rows, int32_t width, qattn_stream_t stream);

/* Device weights of one transformer layer (tensor names of the reference's prepacked file,
 * model.ts:86-106; compact tensors in the q4_0-tile32-compact layout of qattn_q4_matmul, norm
 * gains f32).  The library reads them in place and never frees them. */
typedef struct qattn_layer_weights {
  const float* attn_norm;   /* blk.N.attn_norm.weight    [1024] */
  const void* attn_qkv;     /* blk.N.attn_qkv.weight     1024 -> 4096 (Q 2048 | K 1024 | V 1024) */
  int64_t attn_qkv_bytes;
  const float* attn_q_norm; /* blk.N.attn_q_norm.weight  [128] */
  const float* attn_k_norm; /* blk.N.attn_k_norm.weight  [128] */
  const void* attn_output;  /* blk.N.attn_output.weight  2048 -> 1024 */
  int64_t attn_output_bytes;
  const float* ffn_norm;    /* blk.N.ffn_norm.weight     [1024] */
  const void* ffn_gate_up;  /* blk.N.ffn_gate_up.weight  1024 -> 6144 (gate 3072 | up 3072) */
  int64_t ffn_gate_up_bytes;
  const void* ffn_down;     /* blk.N.ffn_down.weight     3072 -> 1024 */
  int64_t ffn_down_bytes;
} qattn_layer_weights;

typedef struct qattn_model_desc {
  const void* token_embd;   /* token_embd.weight: Q6_K [vocab][1024] (4 blocks of 210 B per row) */
  int64_t token_embd_bytes;
  const float* output_norm; /* output_norm.weight [1024] */
  int32_t n_layers;         /* 1 .. QATTN_MAX_LAYERS (the model has 28) */
  const qattn_layer_weights* layers; /* host array of n_layers; copied */
  double eps;               /* RMSNorm epsilon (model.ts:22: 1e-6) */
  double rope_theta;        /* model.ts:23: 1e6 */
  int32_t mask;             /* attention mask (enum qattn_mask_kind; the model uses PREFIX_LOCAL) */
  int32_t prefix, window;   /* 176, 432 (ops.ts:206) */
  int32_t flags;            /* the attention run's enum qattn_run_flags: QATTN_FLAG_BATCH_INVARIANT
                             * makes a sequence's embedding bitwise independent of its batch (every
                             * other stage is row-wise or per sequence already) */
} qattn_model_desc;

typedef struct qattn_model qattn_model;
typedef struct qattn_model_plan qattn_model_plan;

/* Checks and keeps the weight pointers (no copies of the tensors). */
int qattn_model_create(qattn_ctx* ctx, const qattn_model_desc* desc, qattn_model** out);
void qattn_model_destroy(qattn_model* model);

/* An execution plan for up to max_tokens packed tokens in up to max_seqs sequences: owns the
 * activations (residual stream, normalised rows, qkvRaw, q, k, attention output, FFN buffers --
 * model.ts:62-75) and one attention run, re-planned per batch.  The model must outlive it. */
int qattn_model_plan_create(qattn_model* model, int32_t max_tokens, int32_t max_seqs,
                            qattn_model_plan** out);
void qattn_model_plan_destroy(qattn_model_plan* plan);

/* One batch (Qwen3ExecutionPlan.run, model.ts:113-139, over a packed varlen batch): host token
 * ids [cu_seqlens[nseq]] (each in [0, vocab)) and host cu_seqlens (nseq+1 offsets, as in
 * qattn_run_desc).  Embedding lookup and the initial norm, then per layer: QKV projection,
 * QK-norm + RoPE (positions restart at 0 per sequence), attention, output projection, residual +
 * norm, gate/up projection, SwiGLU, down projection, residual + next norm (the next layer's
 * attn_norm, output_norm after the last); then the last-token pool + L2 normalisation into
 * out[i*out_row_stride + c], f32, c < 1024, a device pointer (16-byte aligned, stride a multiple
 * of 4).  The ids are copied to the device before the call returns; the rest is enqueued on
 * `stream` (the plan's buffers are reused by the next call, which must come after this one on the
 * same stream or after a synchronisation). */
int qattn_model_plan_run(qattn_model_plan* plan, const int32_t* ids, const int32_t* cu_seqlens,
                         int32_t nseq, float* out, int64_t out_row_stride, qattn_stream_t stream);

/* The stages of one run, as the reference's profile() names them (model.ts:157-168). */
enum qattn_model_stage {
  QATTN_STAGE_EMBEDDING_NORM = 0,
  QATTN_STAGE_QKV = 1,
  QATTN_STAGE_ROPE_ATTENTION = 2,
  QATTN_STAGE_ATTENTION_OUTPUT = 3,
  QATTN_STAGE_POST_ATTENTION_NORM = 4,
  QATTN_STAGE_FFN_UP_GATE = 5,
  QATTN_STAGE_SWIGLU = 6,
  QATTN_STAGE_FFN_DOWN = 7,
  QATTN_STAGE_POST_FFN_NORM = 8,
  QATTN_STAGE_POOL = 9,
  QATTN_STAGE_COUNT = 10
};
/* qattn_model_plan_run with a HIP event pair around every stage of every layer, then a wait for
 * the stream: stage_ms[s] receives stage s's total over all layers in milliseconds
 * (Qwen3ExecutionPlan.profile, model.ts:141-182). */
int qattn_model_plan_profile(qattn_model_plan* plan, const int32_t* ids, const int32_t* cu_seqlens,
                             int32_t nseq, float* out, int64_t out_row_stride, qattn_stream_t stream,
                             float stage_ms[QATTN_STAGE_COUNT]);

/* ---- synthetic inputs ---------------------------------------------------------------------- */
/* Element (r, c), r < rows, c < row_elems, at dst[r*row_stride + c] receives
 * f16((float)N(0,1)) where the normal has index e = r*row_elems + c: Box-Muller over the pair
 * e>>1 of the SplitMix64(seed) stream (outputs e&~1 and e|1), cos for even e, sin for odd e. */
int qattn_fill_normal(qattn_ctx* ctx, void* dst, int64_t rows, int64_t row_elems,
                      int64_t row_stride, uint64_t seed, qattn_stream_t stream);
/* Row r (r < rows) of dst receives row_elems fp16 N(0,1) draws keyed by the token id ids[r]
 * (device int32 array): draw c comes from the SplitMix64 stream seeded with
 * seed + (uint32)ids[r] * 0xD1B54A32D192ED03, paired as in qattn_fill_normal.  A stand-in for
 * the projections that produce Q/K/V from token embeddings (outside this library), so that an
 * engine driving the attention path sees outputs that depend on its token ids. */
int qattn_fill_token_rows(qattn_ctx* ctx, void* dst, const int32_t* ids, int64_t rows,
                          int64_t row_elems, int64_t row_stride, uint64_t seed,
                          qattn_stream_t stream);
/* Seeded Q/K/V of one (config, layer): raw N(0,1) fp16 Q [T,16,128], K [T,8,128],
 * V [T,8,128] (seeds 0x51574E33_00000000 | config<<16 | layer<<8 | tensor), then
 * qattn_qk_norm_rope on Q and K (unit gain, eps 1e-6, theta 1e6). */
int qattn_gen_qkv(qattn_ctx* ctx, uint32_t config, uint32_t layer, const int32_t* cu_seqlens,
                  int32_t nseq, void* q, int64_t q_row_stride, void* k, int64_t k_row_stride,
                  void* v, int64_t v_row_stride, qattn_stream_t stream);

/* ---- timing (hosts without a HIP runtime: Node, ctypes) ------------------------------------ */
int qattn_event_create(qattn_ctx* ctx, qattn_event_t* ev);
int qattn_event_record(qattn_event_t ev, qattn_stream_t stream);
int qattn_event_elapsed_ms(qattn_event_t start, qattn_event_t stop, float* ms);
/* Blocks until the work recorded before `ev` has finished (the reference's per-submit
 * readback, model.ts:133-135): a host that keeps several batches in
 * flight on one stream waits for each batch's own event, not for the stream. */
int qattn_event_synchronize(qattn_event_t ev);
int qattn_event_destroy(qattn_event_t ev);

#ifdef __cplusplus
}
#endif
#endif
