'use strict';
// CPU tests of the `.wgpack` container (js/prepacked.js).  The first case is the reference's own
// format test (tests/prepacked-format.test.ts:13-33): same inputs, same expected bytes and fields.
const assert = require('assert');
const path = require('path');
const fmt = require(path.join(__dirname, '..', '..', 'qwen3-embedding-webgpu-prepacked_amd', 'js', 'prepacked.js'));

const cases = [];
function test(name, fn) { cases.push({ name, fn }); }

function q40Block(scaleBits, quants) {
  const block = new Uint8Array(18);
  block.set(scaleBits, 0);
  for (let i = 0; i < 16; i += 1) block[i + 2] = quants[i] | (quants[i + 16] << 4);
  return block;
}

test('reference vector: compact tile-major Q4_0 and raw tensors round-trip', () => {
  const first = q40Block([0x00, 0x3c], Array.from({ length: 32 }, (_, i) => i & 15));
  const second = q40Block([0x00, 0x40], Array.from({ length: 32 }, (_, i) => 15 - (i & 15)));
  const packed = fmt.packQ40Tile32('fused', [
    { name: 'first', k: 32, n: 1, bytes: first },
    { name: 'second', k: 32, n: 1, bytes: second },
  ]);
  assert.deepStrictEqual(packed.dimensions, [32, 2]);
  assert.strictEqual(packed.bytes.byteLength, 32 * 20);
  assert.deepStrictEqual(Array.from(packed.bytes.slice(0, 8)), [0x00, 0x3c, 0x00, 0x00, 0x00, 0x11, 0x22, 0x33]);
  assert.deepStrictEqual(Array.from(packed.bytes.slice(20, 28)), [0x00, 0x40, 0x00, 0x00, 0xff, 0xee, 0xdd, 0xcc]);
  const raw = fmt.rawTensor('norm', [1], fmt.GGML_TYPE.F32, new Uint8Array([1, 2, 3, 4]));
  const file = fmt.buildPrepackedFile('abc123', 42, { 'general.name': 'test' }, [raw, packed]);
  const parsed = fmt.parsePrepackedModel(file.buffer);
  assert.strictEqual(parsed.header.sourceSha256, 'abc123');
  assert.strictEqual(parsed.header.sourceBytes, 42);
  assert.strictEqual(parsed.header.metadata['general.name'], 'test');
  const norm = parsed.tensors.get('norm');
  assert.deepStrictEqual([norm.dimensions, norm.type, norm.storage, norm.byteLength], [[1], fmt.GGML_TYPE.F32, 'raw', 4]);
  const fused = parsed.tensors.get('fused');
  assert.deepStrictEqual([fused.dimensions, fused.type, fused.storage, fused.byteLength],
    [[32, 2], fmt.GGML_TYPE.Q4_0, 'q4_0-tile32-compact', 640]);
  // data placement: 256-byte aligned, bytes intact
  assert.strictEqual(parsed.dataOffset % 256, 0);
  assert.strictEqual(fused.byteOffset % 256, 0);
  assert.deepStrictEqual(Array.from(fmt.tensorBytes(parsed, 'fused')), Array.from(packed.bytes));
  assert.deepStrictEqual(Array.from(fmt.tensorBytes(parsed, 'norm')), [1, 2, 3, 4]);
});

test('tile order over several tiles and K blocks', () => {
  // 40 rows x 64 columns: row r, block kb gets scale byte r, first quant byte 16 * kb + (r & 15).
  const k = 64, n = 40;
  const bytes = new Uint8Array(n * 2 * 18);
  for (let r = 0; r < n; r += 1) for (let kb = 0; kb < 2; kb += 1) {
    const o = (r * 2 + kb) * 18;
    bytes[o] = r; bytes[o + 1] = 0x3c; bytes[o + 2] = 16 * kb + (r & 15);
  }
  const packed = fmt.packQ40Tile32('w', [{ name: 'w', k, n, bytes }]);
  assert.strictEqual(packed.bytes.byteLength, 2 * 2 * 32 * 20);
  for (const r of [0, 31, 32, 39]) for (let kb = 0; kb < 2; kb += 1) {
    const rec = (((r >> 5) * 2 + kb) * 32 + (r & 31)) * 20;
    assert.deepStrictEqual(Array.from(packed.bytes.slice(rec, rec + 5)), [r, 0x3c, 0, 0, 16 * kb + (r & 15)]);
  }
  const pad = (((40 >> 5) * 2 + 1) * 32 + 8) * 20;  // row 40 of the last tile: zero
  assert.ok(packed.bytes.slice(pad, pad + 20).every((b) => b === 0));
});

// The reference rejects these inputs (src/prepacked/format.ts); each rejection here is a
// PrepackedFormatError naming the rule that failed.
test('packing and parsing reject what the reference rejects', () => {
  const code = (c) => (e) => e instanceof fmt.PrepackedFormatError && e.code === c;
  assert.throws(() => fmt.packQ40Tile32('x', []), code('NO_PARTS'));
  assert.throws(() => fmt.packQ40Tile32('x', [{ name: 'a', k: 48, n: 1, bytes: new Uint8Array(27) }]), code('K_NOT_BLOCKS'));
  assert.throws(() => fmt.packQ40Tile32('x', [{ name: 'a', k: 32, n: 1, bytes: new Uint8Array(18) },
    { name: 'b', k: 64, n: 1, bytes: new Uint8Array(36) }]), code('K_MISMATCH'));
  assert.throws(() => fmt.packQ40Tile32('x', [{ name: 'a', k: 32, n: 2, bytes: new Uint8Array(18) }]), code('PART_SIZE'));
  const good = fmt.buildPrepackedFile('s', 1, {}, [fmt.rawTensor('t', [4], 0, new Uint8Array(16))]);
  assert.throws(() => fmt.parsePrepackedModel(new ArrayBuffer(4)), code('TRUNCATED_PRELUDE'));
  const badMagic = good.slice(); badMagic[0] = 0x58;
  assert.throws(() => fmt.parsePrepackedModel(badMagic.buffer), code('BAD_MAGIC'));
  const longHeader = good.slice(); new DataView(longHeader.buffer).setUint32(8, 1 << 30, true);
  assert.throws(() => fmt.parsePrepackedModel(longHeader.buffer), code('TRUNCATED_HEADER'));
  assert.throws(() => fmt.parsePrepackedModel(good.slice(0, good.byteLength - 1).buffer), code('TENSOR_OUT_OF_BOUNDS'));
  const rebuild = (mutate) => {
    const p = fmt.parsePrepackedModel(good.slice().buffer);
    const header = JSON.parse(JSON.stringify(p.header));
    mutate(header);
    const json = new TextEncoder().encode(JSON.stringify(header));
    const dataOffset = Math.ceil((12 + json.byteLength) / 256) * 256;
    const out = new Uint8Array(dataOffset + 64);
    out.set(new TextEncoder().encode('WGPACK02'), 0);
    new DataView(out.buffer).setUint32(8, json.byteLength, true);
    out.set(json, 12);
    return out.buffer;
  };
  for (const field of ['version', 'layout', 'tileRows', 'blockValues', 'blockBytes']) {
    assert.throws(() => fmt.parsePrepackedModel(rebuild((h) => { h[field] = 'other'; })), code('BAD_LAYOUT'), field);
  }
  assert.throws(() => fmt.parsePrepackedModel(rebuild((h) => { h.tensors.push(Object.assign({}, h.tensors[0])); })), code('DUPLICATE_TENSOR'));
  assert.throws(() => fmt.parsePrepackedModel(rebuild((h) => { h.tensors[0].storage = 'q4_0-tile32-compact'; })), code('BAD_COMPACT_TENSOR'));
  assert.throws(() => fmt.parsePrepackedModel(rebuild((h) => { h.tensors[0].storage = 'zip'; })), code('BAD_STORAGE'));
  // what it accepts: a compact 2-D Q4_0 entry, and an unchanged header
  fmt.parsePrepackedModel(rebuild((h) => { Object.assign(h.tensors[0], { storage: 'q4_0-tile32-compact', type: 2, dimensions: [32, 1] }); }));
  fmt.parsePrepackedModel(rebuild(() => {}));
});

test('the file layout: prelude, header length, aligned data start and tensor offsets', () => {
  const a = fmt.rawTensor('a', [3], 0, new Uint8Array([1, 2, 3]));
  const b = fmt.rawTensor('b', [300], 0, new Uint8Array(300).fill(7));
  const c = fmt.rawTensor('c', [1], 0, new Uint8Array([9]));
  const file = fmt.buildPrepackedFile('sha', 5, { k: 'v' }, [a, b, c]);
  assert.strictEqual(Buffer.from(file.subarray(0, 8)).toString('latin1'), 'WGPACK02');
  const n = new DataView(file.buffer).getUint32(8, true);
  const header = JSON.parse(Buffer.from(file.subarray(12, 12 + n)).toString('utf8'));
  assert.deepStrictEqual(header.tensors.map((t) => [t.offset, t.byteLength]), [[0, 3], [256, 300], [768, 1]]);
  const start = Math.ceil((12 + n) / 256) * 256;
  assert.strictEqual(file.byteLength, start + 769);
  assert.deepStrictEqual(Array.from(file.subarray(start, start + 3)), [1, 2, 3]);
  assert.strictEqual(file[start + 768], 9);
  const parsed = fmt.parsePrepackedModel(file.buffer);
  assert.strictEqual(parsed.dataOffset, start);
  assert.strictEqual(parsed.tensors.get('b').byteOffset, start + 256);
});

(async () => {
  let failed = 0;
  for (const c of cases) {
    try { await c.fn(); console.log(`ok   ${c.name}`); } catch (e) { failed += 1; console.log(`FAIL ${c.name}\n${e.stack}`); }
  }
  console.log(`${cases.length - failed}/${cases.length} passed`);
  process.exit(failed ? 1 : 0);
})();
