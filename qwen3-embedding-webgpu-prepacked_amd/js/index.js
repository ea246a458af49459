'use strict';
// Node entry point of the MI355X attention path and model forward (the reference's src/webgpu
// engine surface).
const { Qwen3EmbeddingEngine, packPadded, packVarlen, cuSeqlensOf } = require('./embedding-engine');
const { DeviceContext, DeviceBuffer, CausalAttentionKernel, CompactQ4Matmul, MASK } = require('./ops');
const { HipAttentionRuntime, HipAttentionPlan } = require('./runtime');
const { HipQwen3Model, HipQwen3Plan, HipQwen3Runtime } = require('./model');
const { loadAddon } = require('./addon');
const prepacked = require('./prepacked');

module.exports = {
  Qwen3EmbeddingEngine,
  HipAttentionRuntime,
  HipAttentionPlan,
  HipQwen3Model,
  HipQwen3Plan,
  HipQwen3Runtime,
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
