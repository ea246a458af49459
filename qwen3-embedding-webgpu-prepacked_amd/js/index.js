'use strict';
// Node entry point of the MI355X attention path (the reference's src/webgpu engine surface).
const { Qwen3EmbeddingEngine, packPadded, packVarlen, cuSeqlensOf } = require('./embedding-engine');
const { DeviceContext, DeviceBuffer, CausalAttentionKernel, MASK } = require('./ops');
const { HipAttentionRuntime, HipAttentionPlan } = require('./runtime');
const { loadAddon } = require('./addon');

module.exports = {
  Qwen3EmbeddingEngine,
  HipAttentionRuntime,
  HipAttentionPlan,
  CausalAttentionKernel,
  DeviceContext,
  DeviceBuffer,
  MASK,
  packPadded,
  packVarlen,
  cuSeqlensOf,
  loadAddon,
};
