'use strict';
// CPU restatement, in ES2019 JavaScript for Node, of the reference's tiled flash-attention
// shader (src/webgpu/ops.ts:168-241): one (sequence, query head, 16-query tile) workgroup at a
// time, 16-key tiles, the 176-prefix / 432-window skip and predicate (ops.ts:205-209, 219-220),
// update_stats (ops.ts:186-193) and the f16 accumulation (ops.ts:229-239).  It is the Node CPU
// baseline bench.py times (the reference itself runs this math only inside a browser's WebGPU
// stack).  Test and measurement infrastructure: nothing in the product path loads it.
//
// Rounding points follow the WGSL types, as oracle/oracle.c tiled16_group does:
//   * each 4-wide dot(vec4<f16>, vec4<f16>) is evaluated in f16 (product and sum rounded per
//     step), added to an f32 score, scaled in f32 by f32(0.08838834764831845);
//   * the block max and denominator sum are f32; weights, alpha, beta, the running denominator
//     and the accumulator tile are f16; exp is f32(exp(x)) of the f32 argument;
//   * O = f16(total / denominator).
// Every f16 rounding is round-to-nearest-even of the exact double value.
//
// Usage (all inputs little-endian files written by bench.py / tests):
//   node tiled16.js run <dir>            -> <dir>/o.bin: all groups of <dir>/meta.json (or only
//                                           its `sample` groups; other rows stay 0)
//   node tiled16.js time <dir> <threads> -> one JSON line: the sampled groups of meta.json timed
//                                           on `threads` worker threads (1 = this thread)
// meta.json: {cu: [...], kind, prefix, window, sample: [[seq, tile, head], ...]}
// q.bin [T,16,128] f16, k.bin / v.bin [T,8,128] f16.

const fs = require('fs');
const path = require('path');
const os = require('os');

const HQ = 16;
const HKV = 8;
const HD = 128;
const NEG = Math.fround(-3.402823e38);
const SCALE = Math.fround(0.08838834764831845);

// ---- f16 <-> double ------------------------------------------------------------------------
const F16 = new Float64Array(65536);
for (let h = 0; h < 65536; h += 1) {
  const s = h & 0x8000 ? -1 : 1;
  const e = (h >> 10) & 31;
  const m = h & 1023;
  if (e === 0) F16[h] = s * m * 2 ** -24;
  else if (e === 31) F16[h] = m ? NaN : s * Infinity;
  else F16[h] = s * (1 + m / 1024) * 2 ** (e - 15);
}

const f64 = new Float64Array(1);
const u32 = new Uint32Array(f64.buffer);
const BIG = 2 ** 52;
// Round a double to the nearest f16 value (ties to even), returned as a double.
function r16(x) {
  if (x !== x || x === 0) return x;
  const a = Math.abs(x);
  if (a >= 65520) return x > 0 ? Infinity : -Infinity;
  f64[0] = a;
  let e = ((u32[1] >>> 20) & 0x7ff) - 1023;
  if (e < -14) e = -14;
  const q = 2 ** (e - 10);  // spacing of f16 values in [2^e, 2^(e+1)) (subnormal spacing below)
  const c = BIG * q;
  const r = (a + c) - c;  // one double rounding at spacing q: ties to even
  return x > 0 ? r : -r;
}
// Bits of a double that is an f16 value.
function f16Bits(x) {
  if (x !== x) return 0x7e00;
  const s = x < 0 || Object.is(x, -0) ? 0x8000 : 0;
  const a = Math.abs(x);
  if (a === Infinity) return s | 0x7c00;
  if (a < 2 ** -14) return s | Math.round(a * 2 ** 24);
  f64[0] = a;
  const e = ((u32[1] >>> 20) & 0x7ff) - 1023;
  const m = Math.round((a / 2 ** e - 1) * 1024);
  return s | ((e + 15) << 10) | m;
}
const f32 = Math.fround;
const expf = (x) => f32(Math.exp(x));

// ---- one workgroup: ops.ts:194-240 ------------------------------------------------------------
function tileGroup(a, seq, qHead, gx, out) {
  const t0 = a.cu[seq];
  const S = a.cu[seq + 1] - t0;
  const kvHead = (qHead / (HQ / HKV)) | 0;
  const query = a.qt, key = a.kt, value = a.vt, total = a.tt;
  const scores = a.scores, weights = a.weights;
  const maxima = a.maxima, den = a.den, alphas = a.alphas, betas = a.betas;
  for (let row = 0; row < 16; row += 1) {
    const position = gx * 16 + row;
    const src = ((t0 + position) * HQ + qHead) * HD;
    for (let d = 0; d < HD; d += 1) {
      query[row * HD + d] = position < S ? F16[a.q[src + d]] : 0;
      total[row * HD + d] = 0;
    }
    maxima[row] = NEG;
    den[row] = 0;
  }
  const keyLimit = Math.min(S, (gx + 1) * 16);
  const prefixSize = Math.min(S, a.prefix);
  const localWindow = Math.min(S, a.window);
  const qStart = gx * 16;
  const localStart = qStart + 1 > localWindow ? qStart + 1 - localWindow : 0;
  const sparse = a.kind === 1;
  for (let keyBase = 0; keyBase < keyLimit; keyBase += 16) {
    if (sparse && keyBase >= prefixSize && keyBase + 15 < localStart) continue;
    for (let row = 0; row < 16; row += 1) {
      const kPos = keyBase + row;
      const ks = ((t0 + kPos) * HKV + kvHead) * HD;
      for (let d = 0; d < HD; d += 1) {
        key[row * HD + d] = kPos < S ? F16[a.k[ks + d]] : 0;
        value[row * HD + d] = kPos < S ? F16[a.v[ks + d]] : 0;
      }
    }
    // ops.ts:219-225
    for (let y = 0; y < 16; y += 1) {
      const qPos = gx * 16 + y;
      for (let x = 0; x < 16; x += 1) {
        const kPos = keyBase + x;
        let score = NEG;
        if (qPos < S && kPos <= qPos && kPos < S && (!sparse || kPos < prefixSize || kPos + localWindow > qPos)) {
          score = 0;
          const qo = y * HD, ko = x * HD;
          for (let d = 0; d < HD; d += 4) {
            let dt = r16(query[qo + d] * key[ko + d]);
            dt = r16(dt + r16(query[qo + d + 1] * key[ko + d + 1]));
            dt = r16(dt + r16(query[qo + d + 2] * key[ko + d + 2]));
            dt = r16(dt + r16(query[qo + d + 3] * key[ko + d + 3]));
            score = f32(score + dt);
          }
          score = f32(score * SCALE);
        }
        scores[y * 16 + x] = score;
      }
    }
    // update_stats, ops.ts:186-193
    for (let row = 0; row < 16; row += 1) {
      let blockMax = NEG;
      for (let c = 0; c < 16; c += 1) blockMax = Math.max(blockMax, scores[row * 16 + c]);
      let blockDen = 0;
      for (let c = 0; c < 16; c += 1) {
        const w = expf(f32(scores[row * 16 + c] - blockMax));
        weights[row * 16 + c] = r16(w);
        blockDen = f32(blockDen + w);
      }
      const nextMax = Math.max(maxima[row], blockMax);
      const alpha = expf(f32(maxima[row] - nextMax));
      const beta = expf(f32(blockMax - nextMax));
      alphas[row] = r16(alpha);
      betas[row] = r16(beta);
      den[row] = r16(r16(den[row] * alphas[row]) + r16(f32(beta * blockDen)));
      maxima[row] = nextMax;
    }
    // ops.ts:229-233
    for (let row = 0; row < 16; row += 1) {
      const al = alphas[row], be = betas[row];
      for (let d = 0; d < HD; d += 1) {
        let av = 0;
        for (let c = 0; c < 16; c += 1) av = r16(av + r16(weights[row * 16 + c] * value[c * HD + d]));
        total[row * HD + d] = r16(r16(total[row * HD + d] * al) + r16(be * av));
      }
    }
  }
  // ops.ts:236-239
  if (!out) return;
  for (let row = 0; row < 16; row += 1) {
    const position = gx * 16 + row;
    if (position >= S) continue;
    const dst = ((t0 + position) * HQ + qHead) * HD;
    for (let d = 0; d < HD; d += 1) out[dst + d] = f16Bits(r16(total[row * HD + d] / den[row]));
  }
}

function state(meta, q, k, v) {
  return {
    cu: meta.cu, kind: meta.kind, prefix: meta.prefix, window: meta.window, q, k, v,
    qt: new Float64Array(16 * HD), kt: new Float64Array(16 * HD), vt: new Float64Array(16 * HD),
    tt: new Float64Array(16 * HD), scores: new Float32Array(256), weights: new Float64Array(256),
    maxima: new Float32Array(16), den: new Float64Array(16), alphas: new Float64Array(16),
    betas: new Float64Array(16),
  };
}

// Inputs as Uint16Arrays over SharedArrayBuffers, so worker threads read them without copies.
function loadShared(dir, name) {
  const b = fs.readFileSync(path.join(dir, name));
  const sab = new SharedArrayBuffer(b.length);
  new Uint8Array(sab).set(b);
  return new Uint16Array(sab);
}

function allGroups(cu) {
  const groups = [];
  for (let s = 0; s + 1 < cu.length; s += 1) {
    const tiles = Math.ceil((cu[s + 1] - cu[s]) / 16);
    for (let t = 0; t < tiles; t += 1) for (let h = 0; h < HQ; h += 1) groups.push([s, t, h]);
  }
  return groups;
}

function main() {
  const [mode, dir, threadArg] = process.argv.slice(2);
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const q = loadShared(dir, 'q.bin'), k = loadShared(dir, 'k.bin'), v = loadShared(dir, 'v.bin');
  if (mode === 'run') {
    const T = meta.cu[meta.cu.length - 1];
    const out = new Uint16Array(T * HQ * HD);
    const a = state(meta, q, k, v);
    for (const [s, t, h] of meta.sample || allGroups(meta.cu)) tileGroup(a, s, h, t, out);
    fs.writeFileSync(path.join(dir, 'o.bin'), Buffer.from(out.buffer));
    return;
  }
  if (mode !== 'time') throw new Error(`unknown mode ${mode}`);
  const threads = Math.max(1, parseInt(threadArg || '1', 10));
  const groups = meta.sample;
  const report = (seconds) => {
    process.stdout.write(JSON.stringify({ threads, groups: groups.length, seconds, node: process.version,
      cpus: os.cpus().length }) + '\n');
  };
  if (threads === 1) {
    const a = state(meta, q, k, v);
    const t0 = process.hrtime.bigint();
    for (const [s, t, h] of groups) tileGroup(a, s, h, t, null);
    report(Number(process.hrtime.bigint() - t0) / 1e9);
    return;
  }
  const { Worker } = require('worker_threads');
  const shares = Array.from({ length: threads }, () => []);
  groups.forEach((g, i) => shares[i % threads].push(g));
  let ready = 0, done = 0;
  let t0 = 0n;
  const workers = shares.map((share) => new Worker(__filename, { workerData: { meta, q, k, v, share } }));
  for (const w of workers) {
    w.on('message', (m) => {
      if (m === 'ready') {
        ready += 1;
        if (ready === threads) {
          t0 = process.hrtime.bigint();
          for (const x of workers) x.postMessage('go');
        }
      } else if (m === 'done') {
        done += 1;
        if (done === threads) {
          report(Number(process.hrtime.bigint() - t0) / 1e9);
          for (const x of workers) x.terminate();
        }
      }
    });
    w.on('error', (e) => { throw e; });
  }
}

function worker() {
  const { parentPort, workerData } = require('worker_threads');
  const { meta, q, k, v, share } = workerData;
  const a = state(meta, q, k, v);
  parentPort.on('message', () => {
    for (const [s, t, h] of share) tileGroup(a, s, h, t, null);
    parentPort.postMessage('done');
  });
  parentPort.postMessage('ready');
}

if (require.main === module) {
  if (require('worker_threads').isMainThread) main();
  else worker();
}

module.exports = { r16, f16Bits, tileGroup };
