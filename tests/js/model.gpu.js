'use strict';
// GPU check of the Node model path, run by tests/test_gpu_js.py: a .wgpack (written by the test)
// -> parsePrepackedModel -> HipQwen3Runtime -> Qwen3EmbeddingEngine.embed() for every request at
// once (one micro-batch) -> emb.bin for the Python side to compare with the forward oracle.  Also
// checks here: a request embedded alone gives bitwise what it gave inside the batch, and a
// plan's profile() names the reference's stages.
const fs = require('fs');
const path = require('path');
const assert = require('assert');
const { Qwen3EmbeddingEngine, HipQwen3Runtime, prepacked } = require('../../qwen3-embedding-webgpu-prepacked_amd/js');
const { STAGES } = require('../../qwen3-embedding-webgpu-prepacked_amd/js/model');

async function main() {
  const dir = process.argv[2];
  const file = fs.readFileSync(path.join(dir, 'model.wgpack'));
  const model = prepacked.parsePrepackedModel(file.buffer.slice(file.byteOffset, file.byteOffset + file.byteLength));
  const { eos, lists } = JSON.parse(fs.readFileSync(path.join(dir, 'requests.json'), 'utf8'));
  const runtime = new HipQwen3Runtime({ prepacked: model });
  assert.strictEqual(runtime.model.layers, 2);
  // text "3,17,5" -> token ids [3, 17, 5], the shape transformers.js returns (main.ts:191-199)
  const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });
  const engine = new Qwen3EmbeddingEngine(runtime, tokenizer, 16, 0, eos);
  const outs = await Promise.all(lists.map((ids) => engine.embed(ids.join(','))));
  const flat = new Float32Array(outs.length * 1024);
  outs.forEach((o, i) => flat.set(o, i * 1024));
  fs.writeFileSync(path.join(dir, 'emb.bin'), Buffer.from(flat.buffer));

  const alone = await engine.embed(lists[1].join(','));
  assert.ok(alone.every((x, i) => x === outs[1][i]), 'a request alone differs from the same request in a batch');

  // 40 requests at once: micro-batches of 16, 16 and 8 with two submitted at a time (the next one
  // packed and enqueued while the previous runs); each embedding equals the request's own
  // single-request embedding bit for bit, so batches in flight do not disturb one another.
  const many = Array.from({ length: 40 }, (_, r) => lists[r % lists.length].slice(0, 2 + ((r * 37) % (lists[r % lists.length].length - 1))));
  many.forEach((ids) => { ids[ids.length - 1] = eos; });
  const manyOut = await Promise.all(many.map((ids) => engine.embed(ids.join(','))));
  for (let r = 0; r < many.length; r += 1) {
    const single = await engine.embed(many[r].join(','));
    assert.ok(single.every((x, i) => x === manyOut[r][i]), `request ${r}: pipelined batch differs from the request alone`);
  }

  const plan = runtime.model.createPlan(2, 256);
  const ids = Uint32Array.from(lists[0].concat(lists[1]));
  const stages = plan.profile(ids, [lists[0].length, lists[1].length]);
  assert.deepStrictEqual(Object.keys(stages), STAGES);
  // the gate/up projection and SwiGLU are one launch, timed as ffn_up_gate; swiglu stays empty
  assert.ok(Object.entries(stages).every(([k, ms]) => (k === 'swiglu' ? ms >= 0 : ms > 0)));
  assert.throws(() => plan.profile(Uint32Array.from([0, 1]), [3]), /token buffer/);
  const [e0] = await plan.run(Uint32Array.from(lists[1]), [lists[1].length]);
  assert.ok(e0.every((x, i) => x === outs[1][i]), 'plan.run differs from the engine');
  plan.destroy();

  // A plan or context with a readback in flight refuses to be destroyed until it settles.
  const small = runtime.model.createPlan(1, 16);
  const ticket = small.enqueue(Uint32Array.from([1, 2, eos]), [3]);
  const pending = small.complete(ticket);
  assert.throws(() => small.destroy(), /in flight/);
  assert.throws(() => runtime.context.addon.destroyContext(runtime.context.handle), /in flight/);
  // nor does the buffer being read back, freed directly through the addon
  assert.throws(() => runtime.context.addon.free(small.slots[0].out.handle), /in flight/);
  const [tiny] = await pending;
  assert.ok(Math.abs(Math.hypot(...tiny) - 1) < 1e-3);
  small.destroy();
  runtime.destroy();
  console.log(JSON.stringify({ ok: true, requests: outs.length, stages }));
}

main().catch((e) => {
  console.error(e);
  process.exit(1);
});
