'use strict';
// Micro-batching embedding engine: the reference's Qwen3EmbeddingEngine
// (src/webgpu/embedding-engine.ts:22-88) with the same public surface --
//   new Qwen3EmbeddingEngine(runtime, tokenizer, maxBatchSize = 16, batchWindowMs = 0, eosToken = 151643)
//   engine.embed(text) -> Promise<Float32Array>
// and the same plugin seam (EmbeddingRuntime.createPlan(batch, sequence) -> EmbeddingPlan,
// EmbeddingPlan.run(ids, lengths) -> Promise<Float32Array[]>, ee:7-13).
//
// Packing.  The reference pads every request of a micro-batch to the longest one with the EOS id
// (ee:62-69) and its plan runs over batch x sequence rows.  A runtime that declares
// `packing = 'varlen'` instead receives the requests packed back to back with no padding:
// ids.length === sum(lengths), in request order, so attention (and everything else) costs nothing
// for padding.  Runtimes without that property get exactly the reference's padded layout.
// Plans are cached per `${batch}:${sequence}` (ee:70-75) in both modes, sequence being the
// longest request.
//
// Pipelining.  The reference awaits each micro-batch's run before packing the next (ee:76-78).
// A plan that also offers enqueue(ids, lengths) -> ticket and complete(ticket) -> Promise of the
// embeddings (HipQwen3Plan) gets up to MAX_IN_FLIGHT batches submitted at once: while one runs on
// the GPU, the next is packed and enqueued.  Batches still resolve in order, one batch's failure
// rejects only its requests, and plans with run() alone are run as in the reference.

const MAX_BATCH = 16;
const MAX_IN_FLIGHT = 2;

function packPadded(tokenLists, eosToken) {
  const sequence = Math.max.apply(null, tokenLists.map((t) => t.length));
  const ids = new Uint32Array(tokenLists.length * sequence);
  ids.fill(eosToken);
  const lengths = new Uint32Array(tokenLists.length);
  for (let i = 0; i < tokenLists.length; i += 1) {
    ids.set(tokenLists[i], i * sequence);
    lengths[i] = tokenLists[i].length;
  }
  return { ids, lengths, sequence };
}

function packVarlen(tokenLists) {
  const sequence = Math.max.apply(null, tokenLists.map((t) => t.length));
  const total = tokenLists.reduce((sum, t) => sum + t.length, 0);
  const ids = new Uint32Array(total);
  const lengths = new Uint32Array(tokenLists.length);
  let offset = 0;
  for (let i = 0; i < tokenLists.length; i += 1) {
    ids.set(tokenLists[i], offset);
    lengths[i] = tokenLists[i].length;
    offset += tokenLists[i].length;
  }
  return { ids, lengths, sequence };
}

// Cumulative offsets (n+1 entries, starting at 0) of packed sequences of the given lengths.
function cuSeqlensOf(lengths) {
  const cu = new Int32Array(lengths.length + 1);
  for (let i = 0; i < lengths.length; i += 1) cu[i + 1] = cu[i] + lengths[i];
  return cu;
}

class Qwen3EmbeddingEngine {
  constructor(runtime, tokenizer, maxBatchSize = MAX_BATCH, batchWindowMs = 0, eosToken = 151643) {
    if (maxBatchSize < 1 || maxBatchSize > MAX_BATCH) throw new Error('maxBatchSize must be between 1 and 16');
    this.runtime = runtime;
    this.tokenizer = tokenizer;
    this.maxBatchSize = maxBatchSize;
    this.batchWindowMs = batchWindowMs;
    this.eosToken = eosToken;
    this.pending = [];
    this.plans = new Map();
    this.scheduled = false;
    this.flushing = false;
  }

  embed(text) {
    const tokens = this.tokenizer(text).input_ids.tolist()[0].map(Number);
    if (tokens[tokens.length - 1] !== this.eosToken) tokens.push(this.eosToken);
    return new Promise((resolve, reject) => {
      this.pending.push({ tokens, resolve, reject });
      this.schedule();
    });
  }

  schedule() {
    if (this.scheduled || this.flushing) return;
    this.scheduled = true;
    setTimeout(() => {
      this.scheduled = false;
      this.flush();
    }, this.batchWindowMs);
  }

  async flush() {
    if (this.flushing) return;
    this.flushing = true;
    const inFlight = [];
    // A failed batch rejects every request in it (ee:79-81); later batches still run.
    const finish = async ({ requests, plan, ticket }) => {
      try {
        const embeddings = await plan.complete(ticket);
        requests.forEach((request, index) => request.resolve(embeddings[index]));
      } catch (error) {
        requests.forEach((request) => request.reject(error));
      }
    };
    try {
      while (this.pending.length > 0 || inFlight.length > 0) {
        if (this.pending.length === 0 || inFlight.length >= MAX_IN_FLIGHT) {
          await finish(inFlight.shift());
          continue;
        }
        const requests = this.pending.splice(0, this.maxBatchSize);
        const tokenLists = requests.map((request) => request.tokens);
        const packed = this.runtime.packing === 'varlen' ? packVarlen(tokenLists) : packPadded(tokenLists, this.eosToken);
        const key = `${requests.length}:${packed.sequence}`;
        let plan = this.plans.get(key);
        try {
          if (!plan) {
            plan = this.runtime.createPlan(requests.length, packed.sequence);
            this.plans.set(key, plan);
          }
          if (typeof plan.enqueue === 'function' && typeof plan.complete === 'function') {
            // submitted; the next batch is packed while this one runs
            inFlight.push({ requests, plan, ticket: plan.enqueue(packed.ids, packed.lengths) });
            continue;
          }
          while (inFlight.length > 0) await finish(inFlight.shift());
          const embeddings = await plan.run(packed.ids, packed.lengths);
          requests.forEach((request, index) => request.resolve(embeddings[index]));
        } catch (error) {
          requests.forEach((request) => request.reject(error));
        }
      }
    } finally {
      this.flushing = false;
      if (this.pending.length > 0) this.schedule();
    }
  }
}

module.exports = { Qwen3EmbeddingEngine, packPadded, packVarlen, cuSeqlensOf, MAX_BATCH, MAX_IN_FLIGHT };
