'use strict';
// GPU tests of the Node path: engine -> HipAttentionRuntime -> N-API -> libqattn.so on gfx950.
// Usage: node gpu.test.js <workdir>   (workdir holds the inputs written by tests/test_gpu_js.py)
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const pkg = require(path.join(__dirname, '..', '..', 'qwen3-embedding-webgpu-prepacked_amd', 'js'));
const { Qwen3EmbeddingEngine, HipAttentionRuntime, DeviceContext, CausalAttentionKernel } = pkg;
const { halvesToFloat32, l2Normalize } = require(path.join(__dirname, '..', '..', 'qwen3-embedding-webgpu-prepacked_amd', 'js', 'runtime.js'));

const work = process.argv[2];
const cases = [];
function test(name, fn) { cases.push({ name, fn }); }
function readU16(file) { const b = fs.readFileSync(file); return new Uint16Array(b.buffer, b.byteOffset, b.length / 2); }
function readI32(file) { const b = fs.readFileSync(file); return new Int32Array(b.buffer, b.byteOffset, b.length / 4); }

let ctx;

test('device is gfx950', () => {
  ctx = new DeviceContext(0);
  const info = ctx.info();
  console.log('  device', info.name, info.computeUnits);
  assert.ok(info.name.startsWith('gfx950'));
});

test('varlen operator through N-API on oracle inputs (output checked in Python)', async () => {
  const q = readU16(path.join(work, 'q.bin')), k = readU16(path.join(work, 'k.bin')), v = readU16(path.join(work, 'v.bin'));
  const cu = readI32(path.join(work, 'cu.bin'));
  const T = cu[cu.length - 1];
  const bq = ctx.alloc(q.byteLength), bk = ctx.alloc(k.byteLength), bv = ctx.alloc(v.byteLength), bo = ctx.alloc(T * 4096), bl = ctx.alloc((cu.length - 1) * 4096);
  bq.write(q); bk.write(k); bv.write(v);
  const attention = new CausalAttentionKernel(ctx);
  const run = attention.createVarlenRun(bq, bk, bv, bo, cu, { lastRows: bl });
  assert.strictEqual(run.info.tokens, T);
  attention.encode(run);
  await ctx.synchronizeAsync();
  const o = bo.read(new Uint16Array(T * 2048));
  fs.writeFileSync(path.join(work, 'o.bin'), Buffer.from(o.buffer));
  const last = bl.read(new Uint16Array((cu.length - 1) * 2048));
  for (let s = 0; s < cu.length - 1; s += 1) {
    const row = cu[s + 1] - 1;
    for (let d = 0; d < 2048; d += 1) assert.strictEqual(last[s * 2048 + d], o[row * 2048 + d]);
  }
  attention.destroyRun(run);
  for (const b of [bq, bk, bv, bo, bl]) b.destroy();
});

test('padded createRun (reference layout) equals the varlen run on valid rows', async () => {
  const q = readU16(path.join(work, 'q.bin')), k = readU16(path.join(work, 'k.bin')), v = readU16(path.join(work, 'v.bin'));
  const cu = readI32(path.join(work, 'cu.bin'));
  const o = readU16(path.join(work, 'o.bin'));
  const batch = cu.length - 1;
  let S = 0;
  for (let s = 0; s < batch; s += 1) S = Math.max(S, cu[s + 1] - cu[s]);
  const qp = new Uint16Array(batch * S * 2048), kp = new Uint16Array(batch * S * 1024), vp = new Uint16Array(batch * S * 1024);
  for (let s = 0; s < batch; s += 1) {
    qp.set(q.subarray(cu[s] * 2048, cu[s + 1] * 2048), s * S * 2048);
    kp.set(k.subarray(cu[s] * 1024, cu[s + 1] * 1024), s * S * 1024);
    vp.set(v.subarray(cu[s] * 1024, cu[s + 1] * 1024), s * S * 1024);
  }
  const bq = ctx.alloc(qp.byteLength), bk = ctx.alloc(kp.byteLength), bv = ctx.alloc(vp.byteLength), bo = ctx.alloc(batch * S * 4096);
  bq.write(qp); bk.write(kp); bv.write(vp);
  const attention = new CausalAttentionKernel(ctx);
  const run = attention.createRun(bq, bk, bv, bo, batch, S);
  attention.encode(run);
  await ctx.synchronizeAsync();
  const op = bo.read(new Uint16Array(batch * S * 2048));
  for (let s = 0; s < batch; s += 1) {
    const n = (cu[s + 1] - cu[s]) * 2048;
    assert.deepStrictEqual(op.subarray(s * S * 2048, s * S * 2048 + n), o.subarray(cu[s] * 2048, cu[s] * 2048 + n));
  }
  attention.destroyRun(run);
  for (const b of [bq, bk, bv, bo]) b.destroy();
});

test('device mask check through N-API equals the host evaluation', () => {
  for (const L of [50, 609, 1500]) {
    const dev = ctx.addon.debugMask(ctx.handle, L, 1, 176, 432);
    const host = ctx.addon.planMask(L, 1, 176, 432);
    assert.deepStrictEqual(dev, host);
  }
});

test('engine.embed() end to end: unit vectors; a request alone equals the same request in a batch of 16', async () => {
  const runtime = new HipAttentionRuntime({ context: ctx, layers: 3 });
  const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(' ').map((w) => w.length * 131 + w.charCodeAt(0))] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer);
  const texts = Array.from({ length: 16 }, (_, i) => Array.from({ length: 5 + 37 * i }, (_, j) => `w${(i * 7 + j * 13) % 97}x`).join(' '));
  const batch = await Promise.all(texts.map((t) => engine.embed(t)));
  for (const e of batch) {
    assert.strictEqual(e.length, 2048);
    let norm = 0;
    for (const x of e) { assert.ok(Number.isFinite(x)); norm += x * x; }
    assert.ok(Math.abs(Math.sqrt(norm) - 1) < 1e-5);
  }
  for (const i of [0, 7, 15]) {
    const alone = await engine.embed(texts[i]);
    let dot = 0;
    for (let d = 0; d < 2048; d += 1) dot += alone[d] * batch[i][d];
    assert.ok(dot > 0.99999, `batch-vs-single cosine ${dot}`);
    assert.deepStrictEqual(Array.from(alone), Array.from(batch[i]));
  }
  const a = await engine.embed('alpha beta gamma'), b = await engine.embed('alpha beta delta');
  let dot = 0;
  for (let d = 0; d < 2048; d += 1) dot += a[d] * b[d];
  assert.ok(dot < 0.999, 'different token ids give different outputs');
  for (const p of runtime.plans) p.destroy();
  runtime.plans = [];
});

test('device pool (poolLastL2) equals the host L2 normalisation of the o_last rows', async () => {
  const runtime = new HipAttentionRuntime({ context: ctx, layers: 2 });
  const plan = runtime.createPlan(3, 40);
  const lengths = [40, 1, 17];
  const ids = Array.from({ length: 58 }, (_, i) => (i * 7919) % 151000);
  const got = await plan.run(ids, lengths);
  const bits = plan.last.read(new Uint16Array(3 * 2048));
  for (let i = 0; i < 3; i += 1) {
    const want = l2Normalize(halvesToFloat32(bits.subarray(i * 2048, (i + 1) * 2048)));
    for (let d = 0; d < 2048; d += 1) {
      assert.ok(Math.abs(got[i][d] - want[d]) <= 3e-6 * Math.abs(want[d]) + 1e-12, `row ${i} dim ${d}: ${got[i][d]} vs ${want[d]}`);
    }
  }
  for (const p of runtime.plans) p.destroy();
  runtime.plans = [];
});

test('.wgpack compact Q4_0 tensor -> device -> CompactQ4Matmul equals the host product exactly', () => {
  const fmt = pkg.prepacked;
  // K = 64, N = 40 (two tiles, the second partial), scale 2^-5, x in {-2..2}: every product and
  // partial sum is a multiple of 2^-5 below 64, exact in fp32 and fp16, so the result is exact.
  const k = 64, n = 40, rows = 9;
  const raw = new Uint8Array(n * 2 * 18);
  let seed = 12345;
  const rnd = () => { seed = (seed * 1103515245 + 12345) & 0x7fffffff; return seed >> 8; };
  for (let b = 0; b < n * 2; b += 1) {
    raw[b * 18] = 0x00; raw[b * 18 + 1] = 0x28;  // f16 0x2800 = 2^-5
    for (let j = 2; j < 18; j += 1) raw[b * 18 + j] = rnd() & 255;
  }
  const packed = fmt.packQ40Tile32('blk.0.attn_qkv.weight', [{ name: 'w', k, n, bytes: raw }]);
  const file = fmt.buildPrepackedFile('0', 0, {}, [packed]);
  const model = fmt.parsePrepackedModel(file.buffer);
  const mm = new pkg.CompactQ4Matmul(ctx);
  const weight = mm.upload(model, 'blk.0.attn_qkv.weight');
  const xs = Array.from({ length: rows * k }, () => (rnd() % 5) - 2);
  const halves = { '-2': 0xc000, '-1': 0xbc00, '0': 0x0000, '1': 0x3c00, '2': 0x4000 };
  const x = ctx.alloc(rows * k * 2);
  x.write(Uint16Array.from(xs, (v) => halves[String(v)]));
  const ldy = 40;
  const y = ctx.alloc(rows * ldy * 2);
  mm.run(x, rows, weight, y);
  ctx.synchronize();
  const got = y.read(new Uint16Array(rows * ldy));
  const f16 = (h) => { const e = (h >> 10) & 31, m = h & 1023, sgn = h & 0x8000 ? -1 : 1;
    return e === 0 ? sgn * m * 2 ** -24 : sgn * (1 + m / 1024) * 2 ** (e - 15); };
  for (let r = 0; r < rows; r += 1) for (let c = 0; c < n; c += 1) {
    let want = 0;
    for (let kk = 0; kk < k; kk += 1) {
      const block = (c * 2 + (kk >> 5)) * 18, j = kk & 31;
      const byte = raw[block + 2 + (j & 15)];
      const q = j < 16 ? byte & 15 : byte >> 4;
      want += xs[r * k + kk] * (q - 8) * 2 ** -5;
    }
    assert.strictEqual(f16(got[r * ldy + c]), want, `row ${r} col ${c}`);
  }
  for (const b of [x, y, weight.buffer]) b.destroy();
});

test('a plan re-plans its one attention run per batch: same results as a fresh plan, any lengths', async () => {
  const runtime = new HipAttentionRuntime({ context: ctx, layers: 2 });
  const plan = runtime.createPlan(4, 300);
  const handle = plan.attentionRun.handle;
  const batches = [[300, 300, 300, 300], [1, 2, 3, 4], [299, 17, 300, 64], [5, 300, 1, 250]];
  for (const lengths of batches) {
    const total = lengths.reduce((a, b) => a + b, 0);
    const ids = Uint32Array.from({ length: total }, (_, i) => (i * 7919 + lengths[0]) % 151000);
    const got = await plan.run(ids, lengths);
    assert.strictEqual(plan.attentionRun.handle, handle);
    assert.strictEqual(plan.attentionRun.info.tokens, total);
    const fresh = runtime.createPlan(4, Math.max.apply(null, lengths));
    const want = await fresh.run(ids, lengths);
    for (let i = 0; i < 4; i += 1) assert.deepStrictEqual(Array.from(got[i]), Array.from(want[i]), `${lengths} request ${i}`);
    fresh.destroy();
    runtime.plans.pop();
  }
  assert.throws(() => runtime.attention.updateRun(plan.attentionRun, [0, 1201]), RangeError);
  plan.destroy();
  runtime.plans = [];
});

test('host enqueue time of one 16 x 500 batch, 28 layers (reported)', async () => {
  const runtime = new HipAttentionRuntime({ context: ctx, layers: 28 });
  const plan = runtime.createPlan(16, 500);
  const lengths = new Uint32Array(16).fill(500);
  const ids = Uint32Array.from({ length: 8000 }, (_, i) => (i * 104729) % 151000);
  await plan.run(ids, lengths);  // warm
  const runs = [];
  for (let r = 0; r < 5; r += 1) {
    await plan.run(ids, lengths);
    runs.push(plan.timing);
  }
  const med = (key) => runs.map((t) => t[key]).sort((a, b) => a - b)[2];
  console.log(`# embed host timing: ${JSON.stringify({ batch: '16x500', layers: 28, launches: 28 * 3 + 1,
    host_enqueue_ms: +med('hostMs').toFixed(3), wall_ms: +med('totalMs').toFixed(3),
    host_us_per_launch: +(1000 * med('hostMs') / (28 * 3 + 1)).toFixed(2) })}`);
  assert.ok(med('hostMs') < med('totalMs'));
  plan.destroy();
  runtime.plans = [];
});

test('a run whose bound buffer was freed refuses to encode or re-plan', () => {
  const attention = new CausalAttentionKernel(ctx);
  const T = 64;
  const bufs = [ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048), ctx.alloc(T * 4096)];
  const run = attention.createVarlenRun(bufs[0], bufs[1], bufs[2], bufs[3], [0, T], { mask: 'causal' });
  attention.encode(run);
  ctx.synchronize();
  bufs[2].destroy();
  assert.throws(() => attention.encode(run), /freed/);
  assert.throws(() => attention.updateRun(run, [0, 32]), /freed/);
  attention.destroyRun(run);
  for (const b of bufs) b.destroy();
});

test('plan.run rejects malformed input before launching', async () => {
  const runtime = new HipAttentionRuntime({ context: ctx, layers: 1 });
  const plan = runtime.createPlan(2, 4);
  await assert.rejects(plan.run(new Uint32Array(9), new Uint32Array([4, 5])), /does not match/);
  await assert.rejects(plan.run(new Uint32Array(3), new Uint32Array([3])), /lengths do not match/);
  plan.destroy();
});

test('createRun / genQkv reject descriptors that reach past their buffers (RangeError) before any launch', () => {
  const addon = ctx.addon;
  const T = 100;
  const bq = ctx.alloc(T * 4096), bk = ctx.alloc(T * 2048), bv = ctx.alloc(T * 2048), bo = ctx.alloc(T * 4096);
  const qkv = ctx.alloc(T * 8192), qkvShort = ctx.alloc(T * 8192 - 16), short4 = ctx.alloc(T * 4096 - 16), short2 = ctx.alloc(T * 2048 - 16);
  const cuSeqlens = new Int32Array([0, 40, T]);
  const base = { q: bq.handle, k: bk.handle, v: bv.handle, o: bo.handle, cuSeqlens, mask: 0 };
  const run = addon.createRun(ctx.handle, base);  // exact sizes are accepted
  addon.destroyRun(run);
  const bad = [
    Object.assign({}, base, { q: short4.handle }),
    Object.assign({}, base, { k: short2.handle }),
    Object.assign({}, base, { v: short2.handle }),
    Object.assign({}, base, { o: short4.handle }),
    Object.assign({}, base, { qOffsetBytes: 16 }),
    Object.assign({}, base, { qOffsetBytes: T * 4096 }),
    Object.assign({}, base, { kOffsetBytes: 8 }),
    Object.assign({}, base, { oLast: short2.handle, oLastOffsetBytes: T * 2048 - 32 }),
    // the reference's qkvRaw layout (V in place: stride 4096, offset 3072) one row short
    Object.assign({}, base, { v: qkvShort.handle, vRowStride: 4096, vOffset: 3072 }),
    Object.assign({}, base, { q: qkvShort.handle, qRowStride: 4096, k: qkvShort.handle, kRowStride: 4096, kOffsetBytes: 4096, v: qkvShort.handle, vRowStride: 4096, vOffset: 3072 }),
  ];
  for (const d of bad) assert.throws(() => addon.createRun(ctx.handle, d), RangeError);
  const inPlace = addon.createRun(ctx.handle, Object.assign({}, base, {
    q: qkv.handle, qRowStride: 4096, k: qkv.handle, kRowStride: 4096, kOffsetBytes: 4096, v: qkv.handle, vRowStride: 4096, vOffset: 3072 }));
  addon.destroyRun(inPlace);
  assert.throws(() => addon.genQkv(ctx.handle, 1, 0, cuSeqlens, short4.handle, bk.handle, bv.handle), RangeError);
  assert.throws(() => addon.genQkv(ctx.handle, 1, 0, cuSeqlens, bq.handle, bk.handle, short2.handle), RangeError);
  const other = new DeviceContext(0);
  const foreign = other.alloc(T * 4096);
  assert.throws(() => addon.createRun(ctx.handle, Object.assign({}, base, { q: foreign.handle })), /another context/);
  other.destroy();
  for (const b of [bq, bk, bv, bo, qkv, qkvShort, short4, short2]) b.destroy();
});

test('destroying a context before its buffers and runs: they throw afterwards, nothing is used after free', () => {
  const c2 = new DeviceContext(0);
  const attention = new CausalAttentionKernel(c2);
  const T = 70;
  const bufs = [c2.alloc(T * 4096), c2.alloc(T * 2048), c2.alloc(T * 2048), c2.alloc(T * 4096)];
  const run = attention.createVarlenRun(bufs[0], bufs[1], bufs[2], bufs[3], [0, T], { mask: 'causal' });
  c2.destroy();
  assert.throws(() => attention.encode(run), /destroyed/);
  assert.throws(() => c2.addon.runInfo(run.handle), /destroyed/);
  assert.throws(() => bufs[0].read(new Uint16Array(8)), /freed/);
  attention.destroyRun(run);  // no-ops once the context is gone
  for (const b of bufs) b.destroy();
});

test('handles dropped without destroy() are finalized in any order without faults', async () => {
  for (let round = 0; round < 3; round += 1) {
    (() => {
      const c2 = new DeviceContext(0);
      const attention = new CausalAttentionKernel(c2);
      const bufs = [c2.alloc(64 * 4096), c2.alloc(64 * 2048), c2.alloc(64 * 2048), c2.alloc(64 * 4096)];
      attention.createVarlenRun(bufs[0], bufs[1], bufs[2], bufs[3], [0, 64], { mask: 'causal' });
    })();
    if (global.gc) global.gc();
    await new Promise((r) => setImmediate(r));
  }
  ctx.synchronize();
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
  if (ctx) ctx.destroy();
  console.log(`${cases.length - failed}/${cases.length} passed`);
  process.exit(failed ? 1 : 0);
})();
