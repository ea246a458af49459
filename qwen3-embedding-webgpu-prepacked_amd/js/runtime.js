'use strict';
// EmbeddingRuntime plugin (reference interface: src/webgpu/embedding-engine.ts:7-13) that runs the
// attention path of Qwen3-Embedding-0.6B on an MI355X through libqattn.so.
//
// What a plan's run(ids, lengths) computes, per micro-batch (packed varlen, no padding):
//   for each of `layers` layers:
//     Q [T,16,128], K [T,8,128], V [T,8,128] <- stand-in projections: seeded N(0,1) rows keyed by
//       each token id (qattn_fill_token_rows; the Q4_0 projections that really produce them from
//       hidden states, src/webgpu/quant-matmul.ts, are outside this library)
//     Q, K <- per-head RMSNorm + RoPE (theta 1e6) at per-sequence positions (ops.ts:104-150)
//     O    <- causal GQA attention, 176-prefix + 432-local mask (ops.ts:168-241), on the GPU
//   result i = L2-normalised last-token row of request i's last-layer attention output, f32
//     (the row the reference's pool reads, ops.ts:357), length 2048.
// So the engine, the packer, the N-API boundary and the attention kernels are the real ones,
// while the returned vectors are attention-path outputs, not model embeddings.

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
    this.q = ctx.alloc(this.capacity * 2048 * 2);
    this.k = ctx.alloc(this.capacity * 1024 * 2);
    this.v = ctx.alloc(this.capacity * 1024 * 2);
    this.o = ctx.alloc(this.capacity * 2048 * 2);
    this.last = ctx.alloc(batch * 2048 * 2);
    this.embeddings = ctx.alloc(batch * 2048 * 4);
  }

  async run(ids, lengths) {
    if (lengths.length !== this.batch) throw new Error('lengths do not match execution plan');
    const total = lengths.reduce((sum, l) => sum + l, 0);
    if (ids.length !== total || total > this.capacity) throw new Error('token buffer does not match execution plan');
    if (Array.prototype.some.call(lengths, (l) => l < 1)) throw new Error('every request needs at least one token');
    const rt = this.runtime;
    const ctx = rt.context;
    const addon = ctx.addon;
    const cu = cuSeqlensOf(lengths);
    this.ids.write(Int32Array.from(ids));
    const run = rt.attention.createVarlenRun(this.q, this.k, this.v, this.o, cu, {
      mask: rt.mask, prefix: rt.prefix, window: rt.window, lastRows: this.last,
      batchInvariant: rt.batchInvariant,
    });
    try {
      for (let layer = 0; layer < rt.layers; layer += 1) {
        const base = rt.seed + layer * 16;
        addon.fillTokenRows(ctx.handle, this.q.handle, this.ids.handle, total, 2048, 2048, 0x51574e33, base);
        addon.fillTokenRows(ctx.handle, this.k.handle, this.ids.handle, total, 1024, 1024, 0x51574e33, base + 1);
        addon.fillTokenRows(ctx.handle, this.v.handle, this.ids.handle, total, 1024, 1024, 0x51574e33, base + 2);
        addon.qkNormRope(ctx.handle, this.q.handle, 2048, 0, 16, cu, 1e-6, 1e6);
        addon.qkNormRope(ctx.handle, this.k.handle, 1024, 0, 8, cu, 1e-6, 1e6);
        rt.attention.encode(run);
      }
      // Last-token pool + L2 norm on the device (LastTokenPoolKernel, ops.ts:347-379) over the
      // o_last rows, one per request.
      addon.poolLastL2(ctx.handle, this.last.handle, 2048, 2048, Int32Array.from({ length: this.batch + 1 }, (_, i) => i),
        this.embeddings.handle);
      await ctx.synchronizeAsync();
    } finally {
      rt.attention.destroyRun(run);
    }
    const flat = this.embeddings.read(new Float32Array(this.batch * 2048));
    const out = [];
    for (let i = 0; i < this.batch; i += 1) out.push(flat.slice(i * 2048, (i + 1) * 2048));
    return out;
  }

  destroy() {
    for (const b of [this.ids, this.q, this.k, this.v, this.o, this.last, this.embeddings]) b.destroy();
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
