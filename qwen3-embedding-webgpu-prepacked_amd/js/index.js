'use strict';
// Node entry point of the MI355X attention path (the reference's src/webgpu engine surface).
const { Qwen3EmbeddingEngine, packPadded, packVarlen, cuSeqlensOf } = require('./embedding-engine');
const { DeviceContext, DeviceBuffer, CausalAttentionKernel, CompactQ4Matmul, MASK } = require('./ops');
const { HipAttentionRuntime, HipAttentionPlan } = require('./runtime');
const { loadAddon } = require('./addon');
const prepacked = require('./prepacked');

module.exports = {
  Qwen3EmbeddingEngine,
  HipAttentionRuntime,
  HipAttentionPlan,
  CausalAttentionKernel,
  CompactQ4Matmul,
  DeviceContext,
  DeviceBuffer,
  MASK,
  packPadded,
  packVarlen,
  cuSeqlensOf,
  loadAddon,
  prepacked,
};
