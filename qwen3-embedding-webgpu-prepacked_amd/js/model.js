'use strict';
// The Qwen3-Embedding-0.6B model on an MI355X: the reference's Qwen3WebGPUModel and
// Qwen3ExecutionPlan (src/webgpu/model.ts:49-255) over libqattn.so's qattn_model /
// qattn_model_plan, plus an EmbeddingRuntime (embedding-engine.ts:11-13) for the engine.
//
//   new HipQwen3Model(context, prepacked)   uploads a parsed .wgpack's tensors (parsePrepackedModel)
//                                           and checks names, types and shapes (model.ts:211-224)
//   model.createPlan(batch, sequence)       an execution plan for up to `batch` requests of up to
//                                           `sequence` tokens each (model.ts:273)
//   plan.run(ids, lengths)                  packed token ids -> one L2-normalised 1024-float
//                                           embedding per request (model.ts:113-139)
//   plan.enqueue(ids, lengths) -> ticket    the same run, submitted; plan.complete(ticket) resolves
//                                           to its embeddings (two submits of a plan in flight)
//   plan.profile(ids, lengths)              stage totals in ms (model.ts:141-182)
//   new HipQwen3Runtime({ model | prepacked, context })   EmbeddingRuntime for Qwen3EmbeddingEngine
//
// The forward is the reference's stage sequence: Q6_K embedding lookup and the first RMSNorm, then
// per layer the fused QKV Q4_0 projection, QK-norm + RoPE, attention (176-prefix + 432-window
// mask), output projection, residual + RMSNorm, gate/up projection, SwiGLU, down projection,
// residual + next RMSNorm; last-token pool + L2.  Batches are packed varlen (no padding rows);
// positions restart at 0 per request.

const { DeviceContext } = require('./ops');
const { GGML_TYPE, STORAGE_COMPACT, STORAGE_RAW } = require('./prepacked');
const { cuSeqlensOf } = require('./embedding-engine');

const HIDDEN = 1024;
const INTERMEDIATE = 3072;
const MAX_LAYERS = 28;
const GGML_Q6_K = GGML_TYPE.Q6_K;
const MASK = { causal: 0, 'prefix-local': 1 };
const STAGES = ['embedding_norm', 'qkv', 'rope_attention', 'attention_output', 'post_attention_norm',
  'ffn_up_gate', 'swiglu', 'ffn_down', 'post_ffn_norm', 'pool'];

// Expected tensors: [name, storage, type, dimensions] (dimensions GGUF order: [K, N] / [width]).
function layerTensors(layer) {
  const p = `blk.${layer}`;
  return [
    [`${p}.attn_norm.weight`, STORAGE_RAW, GGML_TYPE.F32, [HIDDEN]],
    [`${p}.attn_qkv.weight`, STORAGE_COMPACT, GGML_TYPE.Q4_0, [HIDDEN, 2048 + 2 * 1024]],
    [`${p}.attn_q_norm.weight`, STORAGE_RAW, GGML_TYPE.F32, [128]],
    [`${p}.attn_k_norm.weight`, STORAGE_RAW, GGML_TYPE.F32, [128]],
    [`${p}.attn_output.weight`, STORAGE_COMPACT, GGML_TYPE.Q4_0, [2048, HIDDEN]],
    [`${p}.ffn_norm.weight`, STORAGE_RAW, GGML_TYPE.F32, [HIDDEN]],
    [`${p}.ffn_gate_up.weight`, STORAGE_COMPACT, GGML_TYPE.Q4_0, [HIDDEN, 2 * INTERMEDIATE]],
    [`${p}.ffn_down.weight`, STORAGE_COMPACT, GGML_TYPE.Q4_0, [INTERMEDIATE, HIDDEN]],
  ];
}
const FIELDS = ['attnNorm', 'attnQkv', 'attnQNorm', 'attnKNorm', 'attnOutput', 'ffnNorm', 'ffnGateUp', 'ffnDown'];

function checkTensor(model, name, storage, type, dims) {
  const t = model.tensors.get(name);
  if (!t) throw new Error(`prepacked model has no tensor ${name}`);
  const sameDims = t.dimensions.length === dims.length && t.dimensions.every((d, i) => d === dims[i]);
  if (t.storage !== storage || t.type !== type || !sameDims) {
    throw new Error(`${name}: ${t.storage} type ${t.type} [${t.dimensions}], expected ${storage} type ${type} [${dims}]`);
  }
  return t;
}

class HipQwen3Model {
  constructor(context, prepacked, options = {}) {
    this.context = context;
    let layers = 0;
    while (prepacked.tensors.has(`blk.${layers}.attn_qkv.weight`)) layers += 1;
    if (layers < 1 || layers > MAX_LAYERS) throw new Error(`prepacked model has ${layers} layers; expected 1..${MAX_LAYERS}`);
    this.layers = layers;
    this.buffers = [];
    const upload = (t) => {
      const b = context.alloc(t.byteLength);
      b.write(new Uint8Array(prepacked.buffer, t.byteOffset, t.byteLength));
      this.buffers.push(b);
      return b.handle;
    };
    const embd = prepacked.tensors.get('token_embd.weight');
    if (!embd || embd.type !== GGML_Q6_K || embd.storage !== STORAGE_RAW || embd.dimensions[0] !== HIDDEN) {
      throw new Error('token_embd.weight must be a raw Q6_K [1024, vocab] tensor');
    }
    this.vocab = embd.dimensions[1];
    const desc = {
      tokenEmbd: upload(embd),
      outputNorm: upload(checkTensor(prepacked, 'output_norm.weight', STORAGE_RAW, GGML_TYPE.F32, [HIDDEN])),
      layers: [],
      eps: 1e-6,
      ropeTheta: 1e6,
      mask: MASK[options.mask || 'prefix-local'],
      prefix: options.prefix === undefined ? 176 : options.prefix,
      window: options.window === undefined ? 432 : options.window,
      // a request's embedding is bitwise independent of its batch unless this is false
      batchInvariant: options.batchInvariant === undefined ? true : !!options.batchInvariant,
    };
    if (desc.mask === undefined) throw new Error(`unknown mask ${options.mask}`);
    for (let layer = 0; layer < layers; layer += 1) {
      const entry = {};
      layerTensors(layer).forEach(([name, storage, type, dims], i) => {
        entry[FIELDS[i]] = upload(checkTensor(prepacked, name, storage, type, dims));
      });
      desc.layers.push(entry);
    }
    this.handle = context.addon.createModel(context.handle, desc);
  }

  createPlan(batch, sequence) {
    return new HipQwen3Plan(this, batch, sequence);
  }

  destroy() {
    if (this.handle) this.context.addon.destroyModel(this.handle);
    this.handle = null;
    for (const b of this.buffers) b.destroy();
    this.buffers = [];
  }
}

class HipQwen3Plan {
  constructor(model, batch, sequence) {
    this.model = model;
    this.batch = batch;
    this.sequence = sequence;
    const ctx = model.context;
    this.handle = ctx.addon.createModelPlan(model.handle, batch * sequence, batch);
    // Two output buffers, each with the event that ends its submit, so a second batch can be
    // enqueued while the first runs (the reference's readback buffer, model.ts:90-95, 133-135).
    this.slots = [0, 1].map(() => ({ out: ctx.alloc(batch * HIDDEN * 4), event: ctx.addon.createEvent(ctx.handle), busy: false }));
    this.next = 0;
    this.timing = null;
  }

  // ids: the requests' token ids packed back to back (Uint32Array / Int32Array), lengths[i] tokens
  // for request i; resolves to one Float32Array(1024) per request.
  async run(ids, lengths) {
    return this.complete(this.enqueue(ids, lengths));
  }

  // Submits one batch on the context stream and returns at once; at most two per plan may be in
  // flight (complete() frees a slot).  Batches run in submission order.
  enqueue(ids, lengths) {
    const cu = this.check(ids, lengths);
    const slot = this.slots[this.next];
    if (slot.busy) throw new Error('two batches of this plan are already in flight');
    const start = process.hrtime.bigint();
    const addon = this.model.context.addon;
    addon.runModelPlan(this.handle, ids, cu, slot.out.handle);
    addon.recordEvent(slot.event);
    slot.busy = true;
    this.next ^= 1;
    return { slot, n: lengths.length, tokens: cu[cu.length - 1], start, enqueued: process.hrtime.bigint() };
  }

  // Resolves to the embeddings of an enqueued batch once its own work is done (a later batch is
  // not waited for).
  async complete(ticket) {
    const flat = new Float32Array(ticket.n * HIDDEN);
    try {
      await this.model.context.addon.readAfterAsync(ticket.slot.out.handle, ticket.slot.event, flat);
    } finally {
      ticket.slot.busy = false;
    }
    const done = process.hrtime.bigint();
    this.timing = {
      hostMs: Number(ticket.enqueued - ticket.start) / 1e6,
      totalMs: Number(done - ticket.start) / 1e6,
      tokens: ticket.tokens,
    };
    const out = [];
    for (let i = 0; i < ticket.n; i += 1) out.push(flat.subarray(i * HIDDEN, (i + 1) * HIDDEN));
    return out;
  }

  // One run with every stage timed: { stage name: ms over all layers } (model.ts:141-182 names).
  profile(ids, lengths) {
    if (this.slots.some((slot) => slot.busy)) throw new Error('profile() while batches of this plan are in flight');
    const cu = this.check(ids, lengths);
    return this.model.context.addon.profileModelPlan(this.handle, ids, cu, this.slots[0].out.handle);
  }

  check(ids, lengths) {
    if (lengths.length < 1 || lengths.length > this.batch) throw new Error('lengths do not match execution plan');
    const cu = cuSeqlensOf(lengths);
    const total = cu[cu.length - 1];
    if (ids.length !== total || total > this.batch * this.sequence) throw new Error('token buffer does not match execution plan');
    for (let i = 0; i < lengths.length; i += 1) if (lengths[i] < 1) throw new Error('every request needs at least one token');
    return cu;
  }

  destroy() {
    if (this.slots.some((slot) => slot.busy)) throw new Error('destroy() while batches of this plan are in flight');
    const addon = this.model.context.addon;
    if (this.handle) addon.destroyModelPlan(this.handle);
    this.handle = null;
    for (const slot of this.slots) {
      addon.destroyEvent(slot.event);
      slot.out.destroy();
    }
    this.slots = [];
  }
}

// EmbeddingRuntime (embedding-engine.ts:11-13) over the model: options.prepacked (a parsed .wgpack)
// or options.model (a HipQwen3Model), options.context (else a new DeviceContext on options.device).
class HipQwen3Runtime {
  constructor(options = {}) {
    this.ownsContext = !options.context && !options.model;
    this.context = options.model ? options.model.context : options.context || new DeviceContext(options.device || 0);
    this.model = options.model || new HipQwen3Model(this.context, options.prepacked, options);
    this.ownsModel = !options.model;
    this.packing = 'varlen';
    this.plans = [];
  }

  createPlan(batch, sequence) {
    const plan = this.model.createPlan(batch, sequence);
    this.plans.push(plan);
    return plan;
  }

  destroy() {
    for (const plan of this.plans) plan.destroy();
    this.plans = [];
    if (this.ownsModel) this.model.destroy();
    if (this.ownsContext) this.context.destroy();
  }
}

module.exports = { HipQwen3Model, HipQwen3Plan, HipQwen3Runtime, STAGES, GGML_Q6_K };
