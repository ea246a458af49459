'use strict';
// CPU tests of js/model.js's loader: the tensors a .wgpack must hold (names, storages, types and
// shapes of the reference's prepacked model, model.ts:86-106, 211-224) and how they reach the
// addon.  A stand-in device context records uploads and the model description instead of a GPU.
const assert = require('assert');
const path = require('path');
const js = path.join(__dirname, '..', '..', 'qwen3-embedding-webgpu-prepacked_amd', 'js');
const fmt = require(path.join(js, 'prepacked.js'));
const { HipQwen3Model } = require(path.join(js, 'model.js'));

const cases = [];
function test(name, fn) { cases.push({ name, fn }); }

function fakeContext() {
  const ctx = { uploads: [], desc: null, handle: 'ctx' };
  ctx.alloc = (bytes) => {
    const b = { bytes, handle: { id: ctx.uploads.length, bytes }, write(data) { ctx.uploads.push(data.byteLength); }, destroy() {} };
    return b;
  };
  ctx.addon = {
    createModel: (handle, desc) => { ctx.desc = desc; return 'model'; },
    destroyModel: () => {},
  };
  return ctx;
}

function modelFile(layers, mutate = () => {}) {
  const raw = (name, dims, type, bytes) => fmt.rawTensor(name, dims, type, new Uint8Array(bytes));
  const compact = (name, k, n) => ({ name, dimensions: [k, n], type: fmt.GGML_TYPE.Q4_0, storage: fmt.STORAGE_COMPACT,
    bytes: new Uint8Array((n / 32) * (k / 32) * 32 * 20) });
  const tensors = [raw('token_embd.weight', [1024, 10], fmt.GGML_TYPE.Q6_K, 10 * 840),
    raw('output_norm.weight', [1024], fmt.GGML_TYPE.F32, 4096)];
  for (let l = 0; l < layers; l += 1) {
    const p = `blk.${l}`;
    tensors.push(raw(`${p}.attn_norm.weight`, [1024], fmt.GGML_TYPE.F32, 4096), compact(`${p}.attn_qkv.weight`, 1024, 4096),
      raw(`${p}.attn_q_norm.weight`, [128], fmt.GGML_TYPE.F32, 512), raw(`${p}.attn_k_norm.weight`, [128], fmt.GGML_TYPE.F32, 512),
      compact(`${p}.attn_output.weight`, 2048, 1024), raw(`${p}.ffn_norm.weight`, [1024], fmt.GGML_TYPE.F32, 4096),
      compact(`${p}.ffn_gate_up.weight`, 1024, 6144), compact(`${p}.ffn_down.weight`, 3072, 1024));
  }
  mutate(tensors);
  return fmt.parsePrepackedModel(fmt.buildPrepackedFile('0', 0, {}, tensors).buffer);
}

test('a well-formed file: every tensor uploaded once, the description maps them by layer', () => {
  const ctx = fakeContext();
  const m = new HipQwen3Model(ctx, modelFile(2));
  assert.strictEqual(m.layers, 2);
  assert.strictEqual(m.vocab, 10);
  assert.strictEqual(ctx.uploads.length, 2 + 2 * 8);
  assert.strictEqual(ctx.desc.layers.length, 2);
  assert.deepStrictEqual(Object.keys(ctx.desc.layers[0]),
    ['attnNorm', 'attnQkv', 'attnQNorm', 'attnKNorm', 'attnOutput', 'ffnNorm', 'ffnGateUp', 'ffnDown']);
  assert.strictEqual(ctx.desc.layers[1].attnQkv.bytes, 4096 / 32 * 1024 / 32 * 32 * 20);
  assert.deepStrictEqual([ctx.desc.mask, ctx.desc.prefix, ctx.desc.window, ctx.desc.batchInvariant], [1, 176, 432, true]);
  assert.strictEqual(ctx.desc.eps, 1e-6);
  assert.strictEqual(ctx.desc.ropeTheta, 1e6);
});

test('missing, mistyped or misshapen tensors are rejected before the device sees a description', () => {
  const drop = (name) => (ts) => ts.splice(ts.findIndex((t) => t.name === name), 1);
  const retype = (name, type) => (ts) => { ts.find((t) => t.name === name).type = type; };
  const reshape = (name, dims) => (ts) => { ts.find((t) => t.name === name).dimensions = dims; };
  const bad = [
    [drop('blk.0.ffn_down.weight'), /no tensor blk.0.ffn_down.weight/],
    [drop('output_norm.weight'), /no tensor output_norm.weight/],
    [retype('token_embd.weight', fmt.GGML_TYPE.F16), /Q6_K/],
    [retype('blk.1.attn_q_norm.weight', fmt.GGML_TYPE.F16), /attn_q_norm/],
    [reshape('blk.0.attn_output.weight', [1024, 2048]), /attn_output/],
  ];
  for (const [mutate, message] of bad) {
    const ctx = fakeContext();
    assert.throws(() => new HipQwen3Model(ctx, modelFile(2, mutate)), message);
    assert.strictEqual(ctx.desc, null);
  }
  assert.throws(() => new HipQwen3Model(fakeContext(), modelFile(0)), /0 layers/);
});

let failed = 0;
for (const c of cases) {
  try {
    c.fn();
    console.log(`ok - ${c.name}`);
  } catch (e) {
    failed += 1;
    console.log(`not ok - ${c.name}\n  ${e.stack}`);
  }
}
process.exit(failed ? 1 : 0);
