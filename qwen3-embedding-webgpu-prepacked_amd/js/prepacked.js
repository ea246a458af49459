'use strict';
// `.wgpack` files: the container the reference's converter writes (src/prepacked/format.ts) and
// this package reads, byte for byte the same format.
//
//   bytes 0..7     "WGPACK02"
//   bytes 8..11    n = byte length of the JSON header (u32, little endian)
//   bytes 12..     the JSON header
//   data           starts at the first 256-byte boundary after the header; every tensor's `offset`
//                  (relative to the data start) is a multiple of 256
//
// Q4_0 weight matrices use storage "q4_0-tile32-compact": 20-byte records (the f16 scale, two
// zero bytes, the 16 quant bytes of a GGML Q4_0 block) grouped by tiles of 32 output rows --
// record index ((row / 32) * (K / 32) + block) * 32 + row % 32 -- the layout qattn_q4_matmul
// reads from device memory.  Other tensors are stored "raw".
//
// Every rejection throws a PrepackedFormatError whose `code` names the rule that failed.

const FORMAT = Object.freeze({
  magic: 'WGPACK02',
  preludeBytes: 12,      // magic + header length
  alignment: 256,        // of the data start and of every tensor
  header: Object.freeze({ version: 2, layout: 'q4_0-tile32-compact-v2', tileRows: 32, blockValues: 32, blockBytes: 20 }),
});
const MAGIC = FORMAT.magic;
const LAYOUT = FORMAT.header.layout;
const TILE_ROWS = FORMAT.header.tileRows;
const BLOCK_VALUES = FORMAT.header.blockValues;
const BLOCK_BYTES = FORMAT.header.blockBytes;
const GGML_Q40_BYTES = 18;  // one GGML Q4_0 block: f16 scale + 16 quant bytes
const STORAGE_COMPACT = 'q4_0-tile32-compact';
const STORAGE_RAW = 'raw';
// GGML tensor type ids used here (the reference's src/gguf/types.ts enum).
const GGML_TYPE = Object.freeze({ F32: 0, F16: 1, Q4_0: 2, Q6_K: 14 });

class PrepackedFormatError extends Error {
  constructor(code, message) {
    super(`.wgpack: ${message}`);
    this.name = 'PrepackedFormatError';
    this.code = code;
  }
}
function reject(code, message) { throw new PrepackedFormatError(code, message); }

const align = (x) => Math.ceil(x / FORMAT.alignment) * FORMAT.alignment;

// ---- writing --------------------------------------------------------------------------------

// One compact [K, N] Q4_0 tensor from GGML Q4_0 row blocks: `parts` ({ name, k, n, bytes }, all
// of one K) are stacked in order into N = sum of their n rows (the reference fuses its Q, K and V
// projections this way).  Rows past N in the last tile stay zero.
function packQ40Tile32(name, parts) {
  if (!Array.isArray(parts) || parts.length === 0) reject('NO_PARTS', `${name}: nothing to pack`);
  const k = parts[0].k;
  if (!(k > 0) || k % BLOCK_VALUES) reject('K_NOT_BLOCKS', `${name}: K = ${k} is not a whole number of 32-value blocks`);
  const blocks = k / BLOCK_VALUES;
  // source of every output row: (bytes of its part, row index inside the part)
  const sources = [];
  for (const part of parts) {
    if (part.k !== k) reject('K_MISMATCH', `${name}: part ${part.name} has K = ${part.k}, the first part K = ${k}`);
    const need = part.n * blocks * GGML_Q40_BYTES;
    if (part.bytes.byteLength !== need) {
      reject('PART_SIZE', `${name}: part ${part.name} holds ${part.bytes.byteLength} bytes, ${part.n} rows of K = ${k} need ${need}`);
    }
    for (let r = 0; r < part.n; r += 1) sources.push([part.bytes, r * blocks * GGML_Q40_BYTES]);
  }
  const n = sources.length;
  const tiles = Math.ceil(n / TILE_ROWS);
  const out = new Uint8Array(tiles * blocks * TILE_ROWS * BLOCK_BYTES);
  // Walk the output in storage order: tile, block, row of the tile.
  let record = 0;
  for (let tile = 0; tile < tiles; tile += 1) {
    for (let b = 0; b < blocks; b += 1) {
      for (let local = 0; local < TILE_ROWS; local += 1, record += 1) {
        const row = tile * TILE_ROWS + local;
        if (row >= n) continue;
        const [bytes, rowStart] = sources[row];
        const src = rowStart + b * GGML_Q40_BYTES;
        const dst = record * BLOCK_BYTES;
        out[dst] = bytes[src];          // f16 scale, then two zero bytes
        out[dst + 1] = bytes[src + 1];
        out.set(bytes.subarray(src + 2, src + GGML_Q40_BYTES), dst + 4);
      }
    }
  }
  return { name, dimensions: [k, n], type: GGML_TYPE.Q4_0, storage: STORAGE_COMPACT, bytes: out };
}

function rawTensor(name, dimensions, type, bytes) {
  return { name, dimensions: Array.from(dimensions), type, storage: STORAGE_RAW, bytes };
}

// The file for `tensors` (from packQ40Tile32 / rawTensor), in order.
function buildPrepackedFile(sourceSha256, sourceBytes, metadata, tensors) {
  const table = [];
  let dataBytes = 0;
  for (const t of tensors) {
    const offset = align(dataBytes);
    table.push({ name: t.name, dimensions: Array.from(t.dimensions), type: t.type, storage: t.storage,
      offset, byteLength: t.bytes.byteLength });
    dataBytes = offset + t.bytes.byteLength;
  }
  const header = Object.assign({}, { version: FORMAT.header.version, sourceSha256, sourceBytes },
    { layout: LAYOUT, tileRows: TILE_ROWS, blockValues: BLOCK_VALUES, blockBytes: BLOCK_BYTES },
    { metadata, tensors: table });
  const json = Buffer.from(JSON.stringify(header), 'utf8');
  const dataStart = align(FORMAT.preludeBytes + json.length);
  const file = new Uint8Array(dataStart + dataBytes);
  Buffer.from(file.buffer).write(MAGIC, 0, 'latin1');
  new DataView(file.buffer).setUint32(8, json.length, true);
  file.set(json, FORMAT.preludeBytes);
  tensors.forEach((t, i) => file.set(t.bytes, dataStart + table[i].offset));
  return file;
}

// ---- reading --------------------------------------------------------------------------------

// Rules every tensor entry must meet, in order: [code, passes(entry, context), message(entry)].
const TENSOR_RULES = [
  ['TENSOR_OUT_OF_BOUNDS', (t, c) => c.dataStart + t.offset + t.byteLength <= c.fileBytes,
    (t) => `tensor ${t.name} reaches past the end of the file`],
  ['DUPLICATE_TENSOR', (t, c) => !c.seen.has(t.name), (t) => `tensor name ${t.name} appears twice`],
  ['BAD_COMPACT_TENSOR', (t) => t.storage !== STORAGE_COMPACT || (t.type === GGML_TYPE.Q4_0 && t.dimensions.length === 2),
    (t) => `compact tensor ${t.name} must be a 2-D Q4_0 matrix`],
  ['BAD_STORAGE', (t) => t.storage === STORAGE_COMPACT || t.storage === STORAGE_RAW,
    (t) => `tensor ${t.name} has storage ${JSON.stringify(t.storage)}; known: ${STORAGE_COMPACT}, ${STORAGE_RAW}`],
];

// Checks a file and indexes its tensors: { header, tensors (Map name -> header entry + absolute
// byteOffset), buffer, dataOffset }.  No tensor data is copied.
function parsePrepackedModel(buffer) {
  const fileBytes = buffer.byteLength;
  if (fileBytes < FORMAT.preludeBytes) reject('TRUNCATED_PRELUDE', `${fileBytes} bytes cannot hold the 12-byte prelude`);
  const magic = Buffer.from(buffer, 0, 8).toString('latin1');
  if (magic !== MAGIC) reject('BAD_MAGIC', `magic ${JSON.stringify(magic)} is not ${MAGIC}`);
  const jsonBytes = new DataView(buffer).getUint32(8, true);
  if (FORMAT.preludeBytes + jsonBytes > fileBytes) {
    reject('TRUNCATED_HEADER', `the ${jsonBytes}-byte header does not fit in a ${fileBytes}-byte file`);
  }
  const header = JSON.parse(Buffer.from(buffer, FORMAT.preludeBytes, jsonBytes).toString('utf8'));
  for (const [field, want] of Object.entries(FORMAT.header)) {
    if (header[field] !== want) {
      reject('BAD_LAYOUT', `header ${field} is ${JSON.stringify(header[field])}, this reader knows ${JSON.stringify(want)} (layout ${LAYOUT})`);
    }
  }
  const context = { dataStart: align(FORMAT.preludeBytes + jsonBytes), fileBytes, seen: new Set() };
  const tensors = new Map();
  for (const entry of header.tensors) {
    for (const [code, passes, message] of TENSOR_RULES) if (!passes(entry, context)) reject(code, message(entry));
    context.seen.add(entry.name);
    tensors.set(entry.name, Object.assign({ byteOffset: context.dataStart + entry.offset }, entry));
  }
  return { header, tensors, buffer, dataOffset: context.dataStart };
}

// The bytes of one tensor of a parsed file (a view, no copy).
function tensorBytes(model, name) {
  const t = model.tensors.get(name);
  if (!t) reject('NO_TENSOR', `the file has no tensor ${name}`);
  return new Uint8Array(model.buffer, t.byteOffset, t.byteLength);
}

module.exports = {
  MAGIC, LAYOUT, TILE_ROWS, BLOCK_VALUES, BLOCK_BYTES, STORAGE_COMPACT, STORAGE_RAW, GGML_TYPE,
  PrepackedFormatError, packQ40Tile32, rawTensor, buildPrepackedFile, parsePrepackedModel, tensorBytes,
};
