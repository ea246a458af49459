'use strict';
// CPU tests of the Node engine and the host side of the N-API boundary (no GPU needed).
// The first three cases run the packer vectors of tests/golden/reference_vectors.json: the
// reference's own engine tests (tests/embedding-engine.test.ts:5-23 and :25-36), with a fake
// runtime and tokenizer, and this build's varlen packing of the same requests.
const assert = require('assert');
const path = require('path');
const pkg = require(path.join(__dirname, '..', '..', 'qwen3-embedding-webgpu-prepacked_amd', 'js'));
const { Qwen3EmbeddingEngine, packVarlen, cuSeqlensOf, loadAddon } = pkg;
const vectors = require(path.join(__dirname, '..', 'golden', 'reference_vectors.json'));

const cases = [];
function test(name, fn) { cases.push({ name, fn }); }

test('coalesces up to 16 simultaneous requests and preserves result order', async () => {
  const calls = [];
  const runtime = {
    createPlan(batch, sequence) {
      return {
        async run(ids, lengths) {
          calls.push({ batch, sequence, ids: Array.from(ids), lengths: Array.from(lengths) });
          return Array.from({ length: batch }, (_, index) => new Float32Array([ids[index * sequence]]));
        },
      };
    },
  };
  const v = vectors.engine_coalesce;
  const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, v.max_batch);
  assert.strictEqual(engine.eosToken, v.eos);
  const results = await Promise.all(v.requests.map((r) => engine.embed(r.join(','))));
  assert.strictEqual(calls.length, v.expect_calls.length);
  calls.forEach((c, i) => {
    assert.strictEqual(c.batch, v.expect_calls[i].batch);
    assert.strictEqual(c.sequence, v.expect_calls[i].sequence);
    assert.deepStrictEqual(c.lengths, v.expect_calls[i].lengths);
  });
  assert.deepStrictEqual(results.map((value) => value[0]), v.expect_first_ids);
});

test('pads mixed-length requests after their final token', async () => {
  let recorded = [];
  const runtime = {
    createPlan(batch) {
      return { async run(ids) { recorded = Array.from(ids); return Array.from({ length: batch }, () => new Float32Array(1)); } };
    },
  };
  const v = vectors.engine_pad;
  const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, v.max_batch, 0, v.eos);
  await Promise.all(v.requests.map((r) => engine.embed(r.join(','))));
  assert.deepStrictEqual(recorded, v.expect_padded_ids);
});

test('a varlen runtime receives requests packed back to back, without padding', async () => {
  for (const c of vectors.varlen_pack.cases) {
    const seen = [];
    const runtime = {
      packing: 'varlen',
      createPlan(batch, sequence) {
        return { async run(ids, lengths) { seen.push({ batch, sequence, ids: Array.from(ids), lengths: Array.from(lengths) });
          return Array.from({ length: batch }, (_, i) => new Float32Array([lengths[i]])); } };
      },
    };
    const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });
    const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 16, 0, vectors.varlen_pack.eos);
    const out = await Promise.all(c.requests.map((r) => engine.embed(r.join(','))));
    assert.deepStrictEqual(seen, [{ batch: c.requests.length, sequence: c.sequence, ids: c.ids, lengths: c.lengths }]);
    assert.deepStrictEqual(Array.from(cuSeqlensOf(seen[0].lengths)), c.cu_seqlens);
    assert.deepStrictEqual(out.map((x) => x[0]), c.lengths);
  }
});

test('more than maxBatchSize requests split into batches in arrival order; plans are cached per batch:sequence', async () => {
  const created = [];
  const batches = [];
  const runtime = {
    createPlan(batch, sequence) {
      created.push(`${batch}:${sequence}`);
      return { async run(ids, lengths) { batches.push(Array.from(ids)); return Array.from(lengths, (_, i) => new Float32Array([ids[i * sequence]])); } };
    },
  };
  const tokenizer = (text) => ({ input_ids: { tolist: () => [[Number(text)]] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 4, 0, 0);
  const first = await Promise.all(Array.from({ length: 10 }, (_, i) => engine.embed(String(i + 1))));
  assert.deepStrictEqual(first.map((x) => x[0]), [1, 2, 3, 4, 5, 6, 7, 8, 9, 10]);
  assert.deepStrictEqual(created, ['4:2', '2:2']);
  assert.strictEqual(batches.length, 3);
  await Promise.all(Array.from({ length: 4 }, (_, i) => engine.embed(String(i + 20))));
  assert.deepStrictEqual(created, ['4:2', '2:2'], 'the 4:2 plan is reused');
});

test('a failing run rejects every request of its batch and later batches still run', async () => {
  let calls = 0;
  const runtime = {
    createPlan(batch) {
      return { async run() { calls += 1; if (calls === 1) throw new Error('device lost'); return Array.from({ length: batch }, () => new Float32Array([7])); } };
    },
  };
  const tokenizer = () => ({ input_ids: { tolist: () => [[5]] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 2, 0, 0);
  const settled = await Promise.all([1, 2, 3].map(() => engine.embed('x').then((v) => v[0], (e) => e.message)));
  assert.deepStrictEqual(settled, ['device lost', 'device lost', 7]);
});

test('a failing createPlan rejects its batch instead of leaving it pending', async () => {
  const runtime = { createPlan() { throw new Error('out of memory'); } };
  const tokenizer = () => ({ input_ids: { tolist: () => [[5]] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer);
  await assert.rejects(engine.embed('x'), /out of memory/);
});

test('a plan with enqueue/complete gets the next batch submitted while one runs; batches resolve in order', async () => {
  const events = [];
  let inFlight = 0;
  let maxInFlight = 0;
  const runtime = {
    packing: 'varlen',
    createPlan(batch) {
      return {
        enqueue(ids, lengths) {
          inFlight += 1;
          maxInFlight = Math.max(maxInFlight, inFlight);
          events.push(`enqueue ${ids[0]}`);
          return { first: ids[0], n: lengths.length };
        },
        async complete(ticket) {
          await new Promise((r) => setTimeout(r, 5));
          inFlight -= 1;
          events.push(`complete ${ticket.first}`);
          if (ticket.first === 9) throw new Error('device lost');
          return Array.from({ length: ticket.n }, (_, i) => new Float32Array([ticket.first + i]));
        },
        async run() { throw new Error('run() must not be used when enqueue/complete exist'); },
      };
    },
  };
  const tokenizer = (text) => ({ input_ids: { tolist: () => [[Number(text)]] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 4, 0, 0);
  // 14 requests: batches [1..4] [5..8] [9..12] [13, 14]; the third batch fails
  const settled = await Promise.allSettled(Array.from({ length: 14 }, (_, i) => engine.embed(String(i + 1))));
  assert.strictEqual(maxInFlight, 2);
  assert.deepStrictEqual(events, ['enqueue 1', 'enqueue 5', 'complete 1', 'enqueue 9', 'complete 5', 'enqueue 13',
    'complete 9', 'complete 13']);
  settled.forEach((r, i) => {
    if (i >= 8 && i < 12) assert.strictEqual(r.status, 'rejected');
    else assert.strictEqual(r.value[0], i + 1);
  });
});

test('maxBatchSize outside 1..16 throws (reference ee:35)', () => {
  assert.throws(() => new Qwen3EmbeddingEngine({}, () => null, 0), /between 1 and 16/);
  assert.throws(() => new Qwen3EmbeddingEngine({}, () => null, 17), /between 1 and 16/);
});

test('appends EOS only when missing', async () => {
  const seen = [];
  const runtime = { packing: 'varlen', createPlan(batch) { return { async run(ids, lengths) { seen.push(Array.from(ids)); return Array.from({ length: batch }, () => new Float32Array(1)); } }; } };
  const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 16, 0, 9);
  await Promise.all([engine.embed('1,9'), engine.embed('3')]);
  assert.deepStrictEqual(seen, [[1, 9, 3, 9]]);
});

test('packVarlen / cuSeqlensOf offsets', () => {
  const p = packVarlen([[1, 2, 3], [4], [5, 6]]);
  assert.deepStrictEqual(Array.from(p.ids), [1, 2, 3, 4, 5, 6]);
  assert.deepStrictEqual(Array.from(p.lengths), [3, 1, 2]);
  assert.strictEqual(p.sequence, 3);
  assert.deepStrictEqual(Array.from(cuSeqlensOf(p.lengths)), [0, 3, 4, 6]);
});

test('N-API addon loads; host-side planning and validation work without a GPU', () => {
  const addon = loadAddon();
  assert.strictEqual(addon.abiVersion(), 9);
  const plan = addon.planDescribe({ q: 1, k: 1, v: 1, o: 1, cuSeqlens: new Int32Array([0, 50, 550]) });
  assert.strictEqual(plan.info.tokens, 550);
  assert.strictEqual(plan.info.pairs, 1275 + 125250);
  assert.strictEqual(plan.info.workItems, 8 * (1 + 8));
  assert.strictEqual(plan.info.slots, 8 * 9);  // 9 items per KV head on 9 slots
  // Splitting the 8-tile items would not pay for the merge kernel here: whole items.
  assert.ok(plan.items.length === plan.info.workItems * 8 && plan.info.splitItems === 0);
  // One 5,000-token sequence (79 items per KV head on 64 slots): long items are split.
  const long = addon.planDescribe({ q: 1, k: 1, v: 1, o: 1, cuSeqlens: new Int32Array([0, 5000]) });
  assert.strictEqual(long.info.slots, 512);
  assert.ok(long.items.length > long.info.workItems * 8 && long.info.splitItems > 0);
  const inv = addon.planDescribe({ q: 1, k: 1, v: 1, o: 1, cuSeqlens: new Int32Array([0, 5000]), flags: 1 });
  assert.strictEqual(inv.items.length, inv.info.workItems * 8);  // batch-invariant: whole items
  assert.strictEqual(inv.info.splitItems, 0);
  assert.throws(() => addon.planDescribe({ q: 1, k: 1, v: 1, o: 1, cuSeqlens: new Int32Array([0, 5, 3]) }), /non-decreasing/);
  assert.throws(() => addon.planDescribe({ q: 1, k: 1, v: 1, o: 1, cuSeqlens: new Int32Array([0, 5]), mask: 1, prefix: 0, window: 0 }), /both 0/);
});

test('kernel key iteration (host build) equals the reference mask predicate', () => {
  const addon = loadAddon();
  for (const L of [1, 63, 64, 65, 607, 608, 609, 700]) {
    const bits = addon.planMask(L, 1, 176, 432);
    const words = (L + 31) >> 5;
    for (let q = 0; q < L; q += 1) {
      for (let k = 0; k < L; k += 1) {
        const want = k <= q && (k < 176 || q - k < 432);
        const got = ((bits[q * words + (k >> 5)] >>> (k & 31)) & 1) === 1;
        if (want !== got) throw new Error(`L=${L} q=${q} k=${k}: kernel ${got}, reference ${want}`);
      }
    }
  }
});

test('creating a device context without a GPU fails with the C ABI error', () => {
  if (process.env.QATTN_EXPECT_GPU === '1') return;
  const addon = loadAddon();
  assert.throws(() => addon.createContext(0), /qattn error -4/);
});

(async () => {
  let failed = 0;
  for (const c of cases) {
    try {
      await c.fn();
      console.log(`ok - ${c.name}`);
    } catch (error) {
      failed += 1;
      console.log(`not ok - ${c.name}\n  ${error && error.stack}`);
    }
  }
  console.log(`${cases.length - failed}/${cases.length} passed`);
  process.exit(failed ? 1 : 0);
})();
