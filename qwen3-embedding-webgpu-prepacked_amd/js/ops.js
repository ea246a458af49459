'use strict';
// Attention operator over libqattn.so, mirroring the reference's CausalAttentionKernel
// (src/webgpu/ops.ts:318-345):
//   createRun(q, k, v, output, batch, sequence, qHeads = 16, kvHeads = 8, valueStride = 1024,
//             valueOffset = 0) -> AttentionRun      (padded [batch, sequence] layout, ops.ts:327)
//   encode(run)                                     (ops.ts:344; the stream is the context's)
//   destroyRun(run)                                 (the run's owned buffers, model.ts:108-111)
// plus createVarlenRun(q, k, v, output, cuSeqlens, options) for packed sequences and
// updateRun(run, cuSeqlens) to re-plan a run for the next batch of the same tensors.
// Buffers are device buffers from DeviceContext.alloc().  The mask is the reference's
// always-on 176-token prefix + 432-token local window (ops.ts:206) unless options say otherwise.

const { loadAddon } = require('./addon');

const MASK = { causal: 0, 'prefix-local': 1 };

function maskCode(name) {
  if (!(name in MASK)) throw new Error(`unknown mask ${name}; expected 'causal' or 'prefix-local'`);
  return MASK[name];
}

class DeviceBuffer {
  constructor(context, bytes) {
    this.context = context;
    this.bytes = bytes;
    this.handle = context.addon.alloc(context.handle, bytes);
  }
  write(typedArray, byteOffset = 0) { this.context.addon.write(this.handle, typedArray, byteOffset); }
  read(typedArray, byteOffset = 0) { this.context.addon.read(this.handle, typedArray, byteOffset); return typedArray; }
  destroy() {
    if (this.handle) this.context.addon.free(this.handle);
    this.handle = null;
  }
}

// One device (reference: requestWebGPUDevice, src/webgpu/device.ts:6-24).
class DeviceContext {
  constructor(device = 0) {
    this.addon = loadAddon();
    this.handle = this.addon.createContext(device);
  }
  info() { return this.addon.deviceName(this.handle); }
  alloc(bytes) { return new DeviceBuffer(this, bytes); }
  synchronize() { this.addon.synchronize(this.handle); }
  synchronizeAsync() { return this.addon.synchronizeAsync(this.handle); }
  destroy() {
    if (this.handle) this.addon.destroyContext(this.handle);
    this.handle = null;
  }
}

class CausalAttentionKernel {
  constructor(context) {
    this.context = context;
  }

  // Padded layout exactly as the reference plans it: batch sequences of `sequence` rows each.
  createRun(q, k, v, output, batch, sequence, qHeads = 16, kvHeads = 8, valueStride = 1024, valueOffset = 0, options = {}) {
    if (qHeads !== 16 || kvHeads !== 8) throw new Error('only 16 query heads over 8 KV heads (Qwen3-Embedding-0.6B) are supported');
    const cuSeqlens = new Int32Array(batch + 1);
    for (let b = 0; b < batch; b += 1) cuSeqlens[b + 1] = cuSeqlens[b] + sequence;
    return this.createVarlenRun(q, k, v, output, cuSeqlens, Object.assign({ valueStride, valueOffset }, options));
  }

  // Packed varlen layout: sequence i is rows cuSeqlens[i]..cuSeqlens[i+1]-1.
  createVarlenRun(q, k, v, output, cuSeqlens, options = {}) {
    const desc = {
      q: q.handle, k: k.handle, v: v.handle, o: output.handle,
      qRowStride: options.queryStride || 2048,
      kRowStride: options.keyStride || 1024,
      vRowStride: options.valueStride || 1024,
      oRowStride: options.outputStride || 2048,
      vOffset: options.valueOffset || 0,
      cuSeqlens: Int32Array.from(cuSeqlens),
      mask: maskCode(options.mask || 'prefix-local'),
      prefix: options.prefix === undefined ? 176 : options.prefix,
      window: options.window === undefined ? 432 : options.window,
      flags: options.batchInvariant ? 1 : 0,
    };
    if (options.lastRows) desc.oLast = options.lastRows.handle;
    const addon = this.context.addon;
    const handle = addon.createRun(this.context.handle, desc);
    return { handle, info: addon.runInfo(handle), cuSeqlens: desc.cuSeqlens };
  }

  // A new batch for a run's tensors: re-plans the work list in place (qattn_run_update), so one
  // run created at a plan's capacity serves every batch of that plan.
  updateRun(run, cuSeqlens) {
    const cu = Int32Array.from(cuSeqlens);
    this.context.addon.updateRun(run.handle, cu);
    run.cuSeqlens = cu;
    run.info = this.context.addon.runInfo(run.handle);
  }

  encode(run) { this.context.addon.encode(run.handle); }

  destroyRun(run) {
    if (run.handle) this.context.addon.destroyRun(run.handle);
    run.handle = null;
  }
}

// The projection over a `.wgpack` Q4_0 tensor (the reference's compact batch matmul,
// src/webgpu/quant-matmul.ts:267-307, and its `matmul(input, name, rows, output)` helper):
// upload(model, name) places a parsed file's q4_0-tile32-compact tensor [K, N] on the device as
// it is stored; run(x, rows, y) computes y = x W^T for fp16 rows x [rows, K] into y [rows, N].
class CompactQ4Matmul {
  constructor(context) {
    this.context = context;
  }

  upload(model, name) {
    const t = model.tensors.get(name);
    if (!t) throw new Error(`prepacked model has no tensor ${name}`);
    if (t.storage !== 'q4_0-tile32-compact') throw new Error(`${name} is not a compact Q4_0 tensor`);
    const [k, n] = t.dimensions;
    const buffer = this.context.alloc(t.byteLength);
    buffer.write(new Uint8Array(model.buffer, t.byteOffset, t.byteLength));
    return { name, k, n, buffer };
  }

  run(x, rows, weight, y, options = {}) {
    const ldx = options.inputStride === undefined ? weight.k : options.inputStride;
    const ldy = options.outputStride === undefined ? weight.n : options.outputStride;
    this.context.addon.q4Matmul(this.context.handle, x.handle, ldx, rows, weight.k, weight.buffer.handle,
      weight.buffer.bytes, weight.n, y.handle, ldy);
  }
}

module.exports = { DeviceContext, DeviceBuffer, CausalAttentionKernel, CompactQ4Matmul, MASK };
