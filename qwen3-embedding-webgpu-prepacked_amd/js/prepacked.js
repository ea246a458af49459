'use strict';
// The `.wgpack` container (the reference's src/prepacked/format.ts): an 8-byte magic
// "WGPACK02", the JSON header's byte length (u32, little endian), the JSON header, then the
// tensors, each at a 256-byte aligned offset from the data start (itself 256-byte aligned).
// Q4_0 weight matrices are stored "q4_0-tile32-compact": 20-byte records (f16 scale, 2 zero
// bytes, the 16 quant bytes of GGML's Q4_0 block) ordered tile-major, tile = 32 output rows:
// record ((n >> 5) * (K / 32) + k_block) * 32 + (n & 31).  qattn_q4_matmul reads that layout
// from device memory as is.  Written for this package; the byte format is the reference's, so
// files move between the two.

const MAGIC = 'WGPACK02';
const PRELUDE_BYTES = 12;
const DATA_ALIGNMENT = 256;
const LAYOUT = 'q4_0-tile32-compact-v2';
const TILE_ROWS = 32;
const BLOCK_VALUES = 32;
const BLOCK_BYTES = 20;
const Q40_BLOCK_BYTES = 18;  // GGML Q4_0: f16 scale + 16 quant bytes
const STORAGE_COMPACT = 'q4_0-tile32-compact';
const STORAGE_RAW = 'raw';
// GGML tensor type ids used here (the reference's src/gguf/types.ts enum).
const GGML_TYPE = { F32: 0, F16: 1, Q4_0: 2 };

function roundUp(value, alignment) {
  return Math.ceil(value / alignment) * alignment;
}

// Stacks the rows of `parts` ({ name, k, n, bytes }: GGML Q4_0 rows of one K) into one compact
// tensor of dimensions [K, N] (format.ts:64-96).  Rows past N in the last tile stay zero.
function packQ40Tile32(name, parts) {
  if (!parts || parts.length === 0) throw new Error(`cannot pack ${name} without tensor parts`);
  const k = parts[0].k;
  if (k % BLOCK_VALUES !== 0) throw new Error(`${name} K=${k} is not divisible by 32`);
  const rows = [];
  for (const part of parts) {
    if (part.k !== k) throw new Error(`${name} has mismatched K dimensions`);
    const want = part.n * (k / BLOCK_VALUES) * Q40_BLOCK_BYTES;
    if (part.bytes.byteLength !== want) throw new Error(`${part.name} has ${part.bytes.byteLength} bytes; expected ${want}`);
    for (let r = 0; r < part.n; r += 1) rows.push({ bytes: part.bytes, row: r });
  }
  const n = rows.length;
  const kBlocks = k / BLOCK_VALUES;
  const tiles = Math.ceil(n / TILE_ROWS);
  const out = new Uint8Array(tiles * kBlocks * TILE_ROWS * BLOCK_BYTES);
  rows.forEach(({ bytes, row }, outRow) => {
    const tile = Math.floor(outRow / TILE_ROWS);
    const local = outRow % TILE_ROWS;
    for (let kb = 0; kb < kBlocks; kb += 1) {
      const src = (row * kBlocks + kb) * Q40_BLOCK_BYTES;
      const dst = ((tile * kBlocks + kb) * TILE_ROWS + local) * BLOCK_BYTES;
      out[dst] = bytes[src];
      out[dst + 1] = bytes[src + 1];
      out.set(bytes.subarray(src + 2, src + Q40_BLOCK_BYTES), dst + 4);
    }
  });
  return { name, dimensions: [k, n], type: GGML_TYPE.Q4_0, storage: STORAGE_COMPACT, bytes: out };
}

function rawTensor(name, dimensions, type, bytes) {
  return { name, dimensions: Array.from(dimensions), type, storage: STORAGE_RAW, bytes };
}

// The whole file as bytes (format.ts:103-137).
function buildPrepackedFile(sourceSha256, sourceBytes, metadata, tensors) {
  let cursor = 0;
  const entries = tensors.map((t) => {
    cursor = roundUp(cursor, DATA_ALIGNMENT);
    const entry = { name: t.name, dimensions: Array.from(t.dimensions), type: t.type, storage: t.storage,
      offset: cursor, byteLength: t.bytes.byteLength };
    cursor += t.bytes.byteLength;
    return entry;
  });
  const header = { version: 2, sourceSha256, sourceBytes, layout: LAYOUT, tileRows: TILE_ROWS,
    blockValues: BLOCK_VALUES, blockBytes: BLOCK_BYTES, metadata, tensors: entries };
  const json = new TextEncoder().encode(JSON.stringify(header));
  const dataOffset = roundUp(PRELUDE_BYTES + json.byteLength, DATA_ALIGNMENT);
  const out = new Uint8Array(dataOffset + cursor);
  out.set(new TextEncoder().encode(MAGIC), 0);
  new DataView(out.buffer).setUint32(8, json.byteLength, true);
  out.set(json, PRELUDE_BYTES);
  tensors.forEach((t, i) => out.set(t.bytes, dataOffset + entries[i].offset));
  return out;
}

// Validates and indexes a file (format.ts:139-169): returns { header, tensors (Map of name ->
// header entry plus its absolute byteOffset), buffer, dataOffset }.  Throws on a bad magic, a
// header past the end, an unsupported layout, a tensor past the end, a duplicate name, compact
// storage that is not a 2-D Q4_0 matrix, or an unknown storage.
function parsePrepackedModel(buffer) {
  if (buffer.byteLength < PRELUDE_BYTES) throw new Error('prepacked model is shorter than its prelude');
  const magic = new TextDecoder().decode(new Uint8Array(buffer, 0, 8));
  if (magic !== MAGIC) throw new Error(`invalid prepacked model magic ${JSON.stringify(magic)}`);
  const headerLength = new DataView(buffer).getUint32(8, true);
  if (PRELUDE_BYTES + headerLength > buffer.byteLength) throw new Error('prepacked model header extends past end of file');
  const header = JSON.parse(new TextDecoder().decode(new Uint8Array(buffer, PRELUDE_BYTES, headerLength)));
  if (header.version !== 2 || header.layout !== LAYOUT || header.tileRows !== TILE_ROWS
      || header.blockValues !== BLOCK_VALUES || header.blockBytes !== BLOCK_BYTES) {
    throw new Error(`unsupported prepacked layout ${header.layout}`);
  }
  const dataOffset = roundUp(PRELUDE_BYTES + headerLength, DATA_ALIGNMENT);
  const tensors = new Map();
  for (const t of header.tensors) {
    const byteOffset = dataOffset + t.offset;
    if (byteOffset + t.byteLength > buffer.byteLength) throw new Error(`${t.name} extends past end of prepacked file`);
    if (tensors.has(t.name)) throw new Error(`duplicate prepacked tensor ${t.name}`);
    if (t.storage === STORAGE_COMPACT && (t.type !== GGML_TYPE.Q4_0 || t.dimensions.length !== 2)) {
      throw new Error(`${t.name} has invalid compact Q4_0 metadata`);
    }
    if (t.storage !== STORAGE_COMPACT && t.storage !== STORAGE_RAW) throw new Error(`${t.name} has unsupported storage ${t.storage}`);
    tensors.set(t.name, Object.assign({}, t, { byteOffset }));
  }
  return { header, tensors, buffer, dataOffset };
}

// The bytes of one tensor of a parsed file (a view, no copy).
function tensorBytes(model, name) {
  const t = model.tensors.get(name);
  if (!t) throw new Error(`prepacked model has no tensor ${name}`);
  return new Uint8Array(model.buffer, t.byteOffset, t.byteLength);
}

module.exports = {
  MAGIC, LAYOUT, TILE_ROWS, BLOCK_VALUES, BLOCK_BYTES, STORAGE_COMPACT, STORAGE_RAW, GGML_TYPE,
  packQ40Tile32, rawTensor, buildPrepackedFile, parsePrepackedModel, tensorBytes,
};
