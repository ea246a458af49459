'use strict';
// End-to-end timing of the Node engine on the GPU: Qwen3EmbeddingEngine.embed() (the reference's
// micro-batching engine, src/webgpu/embedding-engine.ts:38-87) over HipQwen3Runtime (the 28-layer
// forward in libqattn.so) for concurrent requests -- the reference README's measurement
// (16 concurrent 500-token requests, one 5,000-token request).  There is no model file in this
// image, so the model is synthetic, of the real shapes, and goes through the package's own
// .wgpack writer and parser: random q4_0-tile32-compact records (f16 scale ~0.005, nibbles 1..15
// so the weights are zero-mean) and a random Q6_K token table of 151,669 rows.  The tokenizer is
// a stand-in that returns fixed pseudo-random ids; time spent in a real tokenizer is not counted.
//
//   node js/bench-engine.js [layers = 28] [batches = 5]
//
// prints one JSON line per workload: median wall time per round (embed() of every request through
// the resolved promises), requests/s and tokens/s, and the plan's host enqueue time.  The 64 x 500
// round is four micro-batches: the engine submits the next while one runs (two in flight); the
// line counts the batches enqueued while an earlier one was still running and how long before
// that batch's completion they were enqueued.
const { Qwen3EmbeddingEngine, HipQwen3Runtime, prepacked: fmt } = require('./index');

const HIDDEN = 1024;
const INTER = 3072;
const VOCAB = 151669;
const EOS = 151643;

// xorshift32: deterministic bytes without a dependency
function generator(seed) {
  let s = seed >>> 0 || 1;
  return () => {
    s ^= s << 13;
    s >>>= 0;
    s ^= s >>> 17;
    s ^= s << 5;
    s >>>= 0;
    return s;
  };
}

// IEEE binary16 bits of a positive normal float (round to nearest).
function halfBits(x) {
  const e = Math.floor(Math.log2(x));
  const m = Math.round((x / Math.pow(2, e) - 1) * 1024);
  return m === 1024 ? ((e + 16) << 10) : ((e + 15) << 10) | m;
}

function compact(name, K, N, next) {
  const records = (N / 32) * (K / 32) * 32;
  const bytes = new Uint8Array(records * 20);
  const scales = [];
  for (let i = 0; i < 16; i += 1) scales.push(halfBits(0.005 * (0.5 + i / 16)));
  for (let r = 0; r < records; r += 1) {
    const o = r * 20;
    const sc = scales[next() & 15];
    bytes[o] = sc & 255;
    bytes[o + 1] = sc >> 8;
    for (let j = 4; j < 20; j += 4) {
      const v = next();
      for (let b = 0; b < 4; b += 1) {
        const byte = (v >>> (8 * b)) & 255;
        bytes[o + j + b] = ((byte & 15) % 15 + 1) | (((byte >> 4) % 15 + 1) << 4);  // nibbles 1..15
      }
    }
  }
  return { name, dimensions: [K, N], type: fmt.GGML_TYPE.Q4_0, storage: fmt.STORAGE_COMPACT, bytes };
}

function q6kTable(next) {
  const bytes = new Uint8Array(VOCAB * 4 * 210);
  const d = halfBits(0.006);
  for (let blk = 0; blk < VOCAB * 4; blk += 1) {
    const o = blk * 210;
    for (let j = 0; j < 192; j += 4) {
      const v = next();
      bytes[o + j] = v & 255;
      bytes[o + j + 1] = (v >>> 8) & 255;
      bytes[o + j + 2] = (v >>> 16) & 255;
      bytes[o + j + 3] = v >>> 24;
    }
    for (let j = 0; j < 16; j += 1) {
      const v = next();
      const mag = (v & 15) % 15 + 1;
      bytes[o + 192 + j] = (v & 16 ? -mag : mag) & 255;  // int8 scale, +-(1..15)
    }
    bytes[o + 208] = d & 255;
    bytes[o + 209] = d >> 8;
  }
  return fmt.rawTensor('token_embd.weight', [HIDDEN, VOCAB], fmt.GGML_TYPE.Q6_K, bytes);
}

function gains(name, n, next) {
  const g = new Float32Array(n);
  for (let i = 0; i < n; i += 1) g[i] = 1 + 0.1 * ((next() / 4294967296) * 2 - 1);
  return fmt.rawTensor(name, [n], fmt.GGML_TYPE.F32, new Uint8Array(g.buffer));
}

function syntheticModel(layers, seed) {
  const next = generator(seed);
  const tensors = [q6kTable(next), gains('output_norm.weight', HIDDEN, next)];
  for (let l = 0; l < layers; l += 1) {
    const p = `blk.${l}`;
    tensors.push(gains(`${p}.attn_norm.weight`, HIDDEN, next), compact(`${p}.attn_qkv.weight`, HIDDEN, 4096, next),
      gains(`${p}.attn_q_norm.weight`, 128, next), gains(`${p}.attn_k_norm.weight`, 128, next),
      compact(`${p}.attn_output.weight`, 2048, HIDDEN, next), gains(`${p}.ffn_norm.weight`, HIDDEN, next),
      compact(`${p}.ffn_gate_up.weight`, HIDDEN, 2 * INTER, next), compact(`${p}.ffn_down.weight`, INTER, HIDDEN, next));
  }
  const file = fmt.buildPrepackedFile('0'.repeat(64), 0, { 'qwen3.block_count': layers }, tensors);
  return fmt.parsePrepackedModel(file.buffer.slice(file.byteOffset, file.byteOffset + file.byteLength));
}

// "<length>:<request>:<batch>" -> length - 1 pseudo-random ids below EOS (the engine appends EOS)
function tokenizer(text) {
  const [len, req, batch] = text.split(':').map(Number);
  const next = generator(1 + req * 7919 + batch * 104729);
  const ids = [];
  for (let i = 0; i < len - 1; i += 1) ids.push(next() % EOS);
  return { input_ids: { tolist: () => [ids] } };
}

// Wraps every plan the runtime creates so that each submit and completion is logged with the
// number of batches in flight at the time.
function instrument(runtime) {
  const log = [];
  let inFlight = 0;
  const create = runtime.createPlan.bind(runtime);
  runtime.createPlan = (batch, sequence) => {
    const plan = create(batch, sequence);
    const enqueue = plan.enqueue.bind(plan);
    const complete = plan.complete.bind(plan);
    plan.enqueue = (ids, lengths) => {
      const ticket = enqueue(ids, lengths);
      log.push({ kind: 'enqueue', at: process.hrtime.bigint(), before: inFlight });
      inFlight += 1;
      return ticket;
    };
    plan.complete = async (ticket) => {
      const out = await complete(ticket);
      inFlight -= 1;
      log.push({ kind: 'complete', at: process.hrtime.bigint() });
      return out;
    };
    return plan;
  };
  return log;
}

// Of the round's batches after the first: how many were enqueued while an earlier batch was still
// running, and by how much (median ms) their enqueue preceded that earlier batch's completion.
function overlap(log) {
  const enq = log.filter((e) => e.kind === 'enqueue');
  const done = log.filter((e) => e.kind === 'complete');
  const leads = [];
  let overlapped = 0;
  for (let k = 1; k < enq.length; k += 1) {
    if (enq[k].before > 0) overlapped += 1;
    if (done[k - 1]) leads.push(Number(done[k - 1].at - enq[k].at) / 1e6);
  }
  leads.sort((a, b) => a - b);
  return { micro_batches: enq.length, enqueued_while_previous_running: overlapped,
    enqueue_ahead_of_previous_completion_ms: leads.length ? +leads[leads.length >> 1].toFixed(3) : null };
}

async function workload(engine, runtime, log, name, requests, length, batches, layers) {
  const run = (b) => Promise.all(Array.from({ length: requests }, (_, i) => engine.embed(`${length}:${i}:${b}`)));
  await run(-1);  // warm-up: plan creation, first launches
  const ms = [];
  let last = null;
  let ov = null;
  for (let b = 0; b < batches; b += 1) {
    log.length = 0;
    const t0 = process.hrtime.bigint();
    last = await run(b);
    ms.push(Number(process.hrtime.bigint() - t0) / 1e6);
    ov = overlap(log);
  }
  ms.sort((a, b) => a - b);
  const median = ms[ms.length >> 1];
  const plan = runtime.plans[runtime.plans.length - 1];
  const norms = last.map((e) => Math.sqrt(e.reduce((s, v) => s + v * v, 0)));
  return {
    path: 'Qwen3EmbeddingEngine.embed -> HipQwen3Runtime',
    workload: name,
    layers,
    requests,
    tokens_per_request: length,
    batches,
    ms_per_round_median: +median.toFixed(3),
    ms_per_round_min: +ms[0].toFixed(3),
    requests_per_s: +(requests / (median / 1000)).toFixed(1),
    tokens_per_s: Math.round((requests * length) / (median / 1000)),
    plan_host_enqueue_ms: plan && plan.timing ? +plan.timing.hostMs.toFixed(3) : null,
    plan_total_ms: plan && plan.timing ? +plan.timing.totalMs.toFixed(3) : null,
    ...ov,
    embeddings_unit_norm: norms.every((n) => Math.abs(n - 1) < 1e-3),
    node: process.version,
  };
}

async function main() {
  const layers = Number(process.argv[2] || 28);
  const batches = Number(process.argv[3] || 5);
  const t0 = Date.now();
  const model = syntheticModel(layers, 7);
  const runtime = new HipQwen3Runtime({ prepacked: model });
  const log = instrument(runtime);
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 16, 0, EOS);
  console.error(`# synthetic ${layers}-layer model built and uploaded in ${Date.now() - t0} ms`);
  console.log(JSON.stringify(await workload(engine, runtime, log, '16x500', 16, 500, batches, layers)));
  console.log(JSON.stringify(await workload(engine, runtime, log, '64x500', 64, 500, batches, layers)));
  console.log(JSON.stringify(await workload(engine, runtime, log, '1x5000', 1, 5000, batches, layers)));
  runtime.destroy();
}

main().catch((e) => {
  console.error(e);
  process.exit(1);
});
