'use strict';
// EmbeddingRuntime plugin (reference interface: src/webgpu/embedding-engine.ts:7-13) that runs the
// attention path of Qwen3-Embedding-0.6B on an MI355X through libqattn.so.
//
// What a plan's run(ids, lengths) computes, per micro-batch (packed varlen, no padding):
//   for each of `layers` layers:
//     qkvRaw [T, 4096] <- stand-in projection: seeded N(0,1) rows keyed by each token id
//       (qattn_fill_token_rows; the Q4_0 projection that really produces qkvRaw from hidden
//       states, src/webgpu/quant-matmul.ts and model.ts:69, is outside this path)
//     Q [T,16,128], K [T,8,128] <- per-head RMSNorm + RoPE (theta 1e6) of qkvRaw's Q and K
//       blocks at per-sequence positions, one launch (QKNormRopeKernel, ops.ts:104-166)
//     O <- causal GQA attention, 176-prefix + 432-local mask (ops.ts:168-241), V read in place
//       from qkvRaw (value stride 4096, offset 3072, as the reference binds it)
//   result i = L2-normalised last-token row of request i's last-layer attention output, f32
//     (the row the reference's pool reads, ops.ts:357), length 2048.
// So the engine, the packer, the N-API boundary and the kernels are the real ones, while the
// returned vectors are attention-path outputs, not model embeddings.
//
// Host work per batch: one token-id upload, one re-plan of the plan's attention run (created
// once, at the plan's capacity), then 3 launches per layer and the pool -- no allocation, no
// per-layer planning.  plan.timing reports the host enqueue time and the wall time of the last
// run.

const { DeviceContext, CausalAttentionKernel } = require('./ops');
const { cuSeqlensOf } = require('./embedding-engine');

const HALF_TO_FLOAT = (() => {
  // binary16 -> f32 for all 65,536 patterns (IEEE: subnormals, Inf, NaN).
  const table = new Float32Array(65536);
  for (let h = 0; h < 65536; h += 1) {
    const sign = h & 0x8000 ? -1 : 1;
    const exponent = (h >> 10) & 0x1f;
    const fraction = h & 0x3ff;
    if (exponent === 0) table[h] = sign * fraction * Math.pow(2, -24);
    else if (exponent === 31) table[h] = fraction ? NaN : sign * Infinity;
    else table[h] = sign * (1 + fraction / 1024) * Math.pow(2, exponent - 15);
  }
  return table;
})();

function halvesToFloat32(bits) {
  const out = new Float32Array(bits.length);
  for (let i = 0; i < bits.length; i += 1) out[i] = HALF_TO_FLOAT[bits[i]];
  return out;
}

function l2Normalize(x) {
  let sum = 0;
  for (let i = 0; i < x.length; i += 1) sum += x[i] * x[i];
  const inv = sum > 0 ? 1 / Math.sqrt(sum) : 0;
  for (let i = 0; i < x.length; i += 1) x[i] *= inv;
  return x;
}

class HipAttentionPlan {
  constructor(runtime, batch, sequence) {
    this.runtime = runtime;
    this.batch = batch;
    this.sequence = sequence;
    this.capacity = batch * sequence;  // tokens: the longest request times the batch
    const ctx = runtime.context;
    this.ids = ctx.alloc(this.capacity * 4);
    this.qkv = ctx.alloc(this.capacity * 4096 * 2);
    this.q = ctx.alloc(this.capacity * 2048 * 2);
    this.k = ctx.alloc(this.capacity * 1024 * 2);
    this.o = ctx.alloc(this.capacity * 2048 * 2);
    this.last = ctx.alloc(batch * 2048 * 2);
    this.embeddings = ctx.alloc(batch * 2048 * 4);
    this.poolRows = Int32Array.from({ length: batch + 1 }, (_, i) => i);
    // The attention run, planned once for `batch` requests of `sequence` tokens and re-planned
    // for each batch's lengths (updateRun) in the same device work-list buffer.
    const full = new Int32Array(batch + 1);
    for (let i = 0; i < batch; i += 1) full[i + 1] = full[i] + sequence;
    this.attentionRun = runtime.attention.createVarlenRun(this.q, this.k, this.qkv, this.o, full, {
      mask: runtime.mask, prefix: runtime.prefix, window: runtime.window, lastRows: this.last,
      valueStride: 4096, valueOffset: 3072, batchInvariant: runtime.batchInvariant,
    });
    this.timing = null;
  }

  async run(ids, lengths) {
    if (lengths.length !== this.batch) throw new Error('lengths do not match execution plan');
    let total = 0;
    for (let i = 0; i < lengths.length; i += 1) {
      if (lengths[i] < 1) throw new Error('every request needs at least one token');
      total += lengths[i];
    }
    if (ids.length !== total || total > this.capacity) throw new Error('token buffer does not match execution plan');
    const start = process.hrtime.bigint();
    const rt = this.runtime;
    const ctx = rt.context;
    const addon = ctx.addon;
    const cu = cuSeqlensOf(lengths);
    // Token ids are < 2^31, so a Uint32Array's bytes are the Int32 ids the generator reads.
    this.ids.write(ids instanceof Uint32Array || ids instanceof Int32Array ? ids : Int32Array.from(ids));
    rt.attention.updateRun(this.attentionRun, cu);
    for (let layer = 0; layer < rt.layers; layer += 1) {
      addon.fillTokenRows(ctx.handle, this.qkv.handle, this.ids.handle, total, 4096, 4096, 0x51574e33,
        rt.seed + layer * 16);
      addon.qkNormRopeQkv(ctx.handle, this.qkv.handle, 4096, this.q.handle, 2048, this.k.handle, 1024, cu, 1e-6, 1e6);
      rt.attention.encode(this.attentionRun);
    }
    // Last-token pool + L2 norm on the device (LastTokenPoolKernel, ops.ts:347-379) over the
    // o_last rows, one per request.
    addon.poolLastL2(ctx.handle, this.last.handle, 2048, 2048, this.poolRows, this.embeddings.handle);
    const enqueued = process.hrtime.bigint();
    await ctx.synchronizeAsync();
    const done = process.hrtime.bigint();
    this.timing = { hostMs: Number(enqueued - start) / 1e6, totalMs: Number(done - start) / 1e6, tokens: total };
    const flat = this.embeddings.read(new Float32Array(this.batch * 2048));
    const out = [];
    for (let i = 0; i < this.batch; i += 1) out.push(flat.subarray(i * 2048, (i + 1) * 2048));
    return out;
  }

  destroy() {
    if (this.attentionRun) this.runtime.attention.destroyRun(this.attentionRun);
    this.attentionRun = null;
    for (const b of [this.ids, this.qkv, this.q, this.k, this.o, this.last, this.embeddings]) b.destroy();
  }
}

class HipAttentionRuntime {
  constructor(options = {}) {
    this.context = options.context || new DeviceContext(options.device || 0);
    this.attention = new CausalAttentionKernel(this.context);
    this.layers = options.layers === undefined ? 28 : options.layers;
    this.mask = options.mask || 'prefix-local';
    this.prefix = options.prefix === undefined ? 176 : options.prefix;
    this.window = options.window === undefined ? 432 : options.window;
    this.seed = options.seed === undefined ? 0 : options.seed;
    // Like the reference, a request's embedding does not depend on what it was batched with
    // (bitwise); batchInvariant: false lets the planner split long items across workgroups.
    this.batchInvariant = options.batchInvariant === undefined ? true : !!options.batchInvariant;
    this.packing = 'varlen';
    this.plans = [];
  }

  createPlan(batch, sequence) {
    const plan = new HipAttentionPlan(this, batch, sequence);
    this.plans.push(plan);
    return plan;
  }

  destroy() {
    for (const plan of this.plans) plan.destroy();
    this.plans = [];
    this.context.destroy();
  }
}

module.exports = { HipAttentionRuntime, HipAttentionPlan, halvesToFloat32, l2Normalize };
