// Type declarations of the Node attention-path package (js/index.js).  The engine and plugin
// interfaces match src/webgpu/embedding-engine.ts:1-13 of the reference.

export interface TokenizerResult {
  input_ids: { tolist(): number[][] };
}
export type TokenizerLike = (text: string) => TokenizerResult;

export interface EmbeddingPlan {
  run(ids: Uint32Array, lengths: Uint32Array): Promise<Float32Array[]>;
  /** Optional split of run(): a plan that has both gets up to two batches in flight from the
   *  engine (the next is packed and enqueued while one runs); results still resolve in order. */
  enqueue?(ids: Uint32Array, lengths: Uint32Array): unknown;
  complete?(ticket: unknown): Promise<Float32Array[]>;
}
export interface EmbeddingRuntime {
  /** 'varlen': the engine packs requests back to back (ids.length === sum(lengths)). */
  packing?: 'padded' | 'varlen';
  createPlan(batch: number, sequence: number): EmbeddingPlan;
}

export class Qwen3EmbeddingEngine {
  constructor(runtime: EmbeddingRuntime, tokenizer: TokenizerLike, maxBatchSize?: number,
              batchWindowMs?: number, eosToken?: number);
  readonly maxBatchSize: number;
  readonly batchWindowMs: number;
  readonly eosToken: number;
  embed(text: string): Promise<Float32Array>;
}

export function packPadded(tokenLists: number[][], eosToken: number): { ids: Uint32Array; lengths: Uint32Array; sequence: number };
export function packVarlen(tokenLists: number[][]): { ids: Uint32Array; lengths: Uint32Array; sequence: number };
export function cuSeqlensOf(lengths: ArrayLike<number>): Int32Array;

export type MaskName = 'causal' | 'prefix-local';

export class DeviceBuffer {
  readonly bytes: number;
  write(data: ArrayBufferView, byteOffset?: number): void;
  read<T extends ArrayBufferView>(data: T, byteOffset?: number): T;
  destroy(): void;
}

export class DeviceContext {
  constructor(device?: number);
  info(): { name: string; computeUnits: number };
  alloc(bytes: number): DeviceBuffer;
  synchronize(): void;
  synchronizeAsync(): Promise<void>;
  destroy(): void;
}

export interface RunInfo {
  tokens: number; pairs: number; flops: number; bytes: number;
  workItems: number; blockQueries: number; tilePairs: number; slots: number; splitItems: number;
}
export interface AttentionRun { handle: unknown; info: RunInfo; cuSeqlens: Int32Array }
export interface VarlenOptions {
  queryStride?: number; keyStride?: number; valueStride?: number; outputStride?: number;
  valueOffset?: number; mask?: MaskName; prefix?: number; window?: number; lastRows?: DeviceBuffer;
  /** Never split an item across workgroups: results independent of batch composition. */
  batchInvariant?: boolean;
}

export class CausalAttentionKernel {
  constructor(context: DeviceContext);
  createRun(q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, output: DeviceBuffer, batch: number,
            sequence: number, qHeads?: number, kvHeads?: number, valueStride?: number,
            valueOffset?: number, options?: VarlenOptions): AttentionRun;
  createVarlenRun(q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, output: DeviceBuffer,
                  cuSeqlens: ArrayLike<number>, options?: VarlenOptions): AttentionRun;
  /** Re-plans a run for the next batch of the same tensors (same options, new lengths). */
  updateRun(run: AttentionRun, cuSeqlens: ArrayLike<number>): void;
  encode(run: AttentionRun): void;
  destroyRun(run: AttentionRun): void;
}

export interface HipRuntimeOptions {
  device?: number; context?: DeviceContext; layers?: number; mask?: MaskName;
  prefix?: number; window?: number; seed?: number;
  /** Default true: embeddings are bitwise independent of batching (no split-K). */
  batchInvariant?: boolean;
}
export interface HipAttentionPlan extends EmbeddingPlan {
  /** Host enqueue time and wall time (ms) of the last run, and its token count. */
  readonly timing: { hostMs: number; totalMs: number; tokens: number } | null;
  destroy(): void;
}
export class HipAttentionRuntime implements EmbeddingRuntime {
  constructor(options?: HipRuntimeOptions);
  readonly packing: 'varlen';
  createPlan(batch: number, sequence: number): HipAttentionPlan;
  destroy(): void;
}

// ---- the `.wgpack` container (the reference's src/prepacked/format.ts) and the Q4_0 projection.
export interface PackedTensorBytes {
  name: string; dimensions: number[]; type: number;
  storage: 'q4_0-tile32-compact' | 'raw'; bytes: Uint8Array;
}
export interface PrepackedTensorHeader {
  name: string; dimensions: number[]; type: number; storage: 'q4_0-tile32-compact' | 'raw';
  offset: number; byteLength: number;
}
export interface PrepackedModel {
  header: {
    version: 2; sourceSha256: string; sourceBytes: number; layout: 'q4_0-tile32-compact-v2';
    tileRows: 32; blockValues: 32; blockBytes: 20;
    metadata: Record<string, string | number | boolean | Array<string | number | boolean>>;
    tensors: PrepackedTensorHeader[];
  };
  tensors: Map<string, PrepackedTensorHeader & { byteOffset: number }>;
  buffer: ArrayBuffer;
  dataOffset: number;
}
/** Every rejection of the container code; `code` names the rule (e.g. 'BAD_MAGIC', 'TENSOR_OUT_OF_BOUNDS'). */
export class PrepackedFormatError extends Error {
  readonly code: 'NO_PARTS' | 'K_NOT_BLOCKS' | 'K_MISMATCH' | 'PART_SIZE' | 'TRUNCATED_PRELUDE' | 'BAD_MAGIC'
    | 'TRUNCATED_HEADER' | 'BAD_LAYOUT' | 'TENSOR_OUT_OF_BOUNDS' | 'DUPLICATE_TENSOR' | 'BAD_COMPACT_TENSOR'
    | 'BAD_STORAGE' | 'NO_TENSOR';
}
export const prepacked: {
  PrepackedFormatError: typeof PrepackedFormatError;
  MAGIC: 'WGPACK02'; LAYOUT: 'q4_0-tile32-compact-v2'; TILE_ROWS: 32; BLOCK_VALUES: 32; BLOCK_BYTES: 20;
  STORAGE_COMPACT: 'q4_0-tile32-compact'; STORAGE_RAW: 'raw'; GGML_TYPE: { F32: 0; F16: 1; Q4_0: 2; Q6_K: 14 };
  packQ40Tile32(name: string, parts: ReadonlyArray<{ name: string; k: number; n: number; bytes: Uint8Array }>): PackedTensorBytes;
  rawTensor(name: string, dimensions: number[], type: number, bytes: Uint8Array): PackedTensorBytes;
  buildPrepackedFile(sourceSha256: string, sourceBytes: number,
                     metadata: PrepackedModel['header']['metadata'], tensors: ReadonlyArray<PackedTensorBytes>): Uint8Array;
  parsePrepackedModel(buffer: ArrayBuffer): PrepackedModel;
  tensorBytes(model: PrepackedModel, name: string): Uint8Array;
};

export interface CompactQ4Weight { name: string; k: number; n: number; buffer: DeviceBuffer }
/** y = x W^T over a compact Q4_0 tensor (the reference's compact batch matmul). */
export class CompactQ4Matmul {
  constructor(context: DeviceContext);
  upload(model: PrepackedModel, name: string): CompactQ4Weight;
  run(x: DeviceBuffer, rows: number, weight: CompactQ4Weight, y: DeviceBuffer,
      options?: { inputStride?: number; outputStride?: number }): void;
}

// ---- the whole model (the reference's Qwen3WebGPUModel / Qwen3ExecutionPlan, model.ts:49-255).
/** Stage names of a profiled run, in order (model.ts:157-168). */
export type ModelStage = 'embedding_norm' | 'qkv' | 'rope_attention' | 'attention_output' | 'post_attention_norm'
  | 'ffn_up_gate' | 'swiglu' | 'ffn_down' | 'post_ffn_norm' | 'pool';
export interface HipModelOptions {
  /** Attention mask of the forward (default 'prefix-local', 176 / 432). */
  mask?: 'causal' | 'prefix-local'; prefix?: number; window?: number;
  /** Default true: a request's embedding is bitwise the same alone or in any batch. */
  batchInvariant?: boolean;
}
/** The weights of a parsed .wgpack on the device (Q6_K token_embd, f32 norms, 4 compact Q4_0
 * projections per layer, 1..28 layers), checked by name, storage, type and shape. */
export class HipQwen3Model {
  constructor(context: DeviceContext, prepacked: PrepackedModel, options?: HipModelOptions);
  readonly layers: number;
  readonly vocab: number;
  createPlan(batch: number, sequence: number): HipQwen3Plan;
  destroy(): void;
}
export interface HipQwen3Ticket { readonly n: number; readonly tokens: number }
export class HipQwen3Plan implements EmbeddingPlan {
  /** Packed token ids (lengths[i] per request) -> one L2-normalised Float32Array(1024) per request. */
  run(ids: Uint32Array | Int32Array, lengths: Uint32Array | number[]): Promise<Float32Array[]>;
  /** Submits one batch and returns at once (at most two of this plan in flight). */
  enqueue(ids: Uint32Array | Int32Array, lengths: Uint32Array | number[]): HipQwen3Ticket;
  /** The embeddings of an enqueued batch, once its own work is done (later batches not waited for). */
  complete(ticket: HipQwen3Ticket): Promise<Float32Array[]>;
  /** One run with each stage timed: total ms per stage over all layers. */
  profile(ids: Uint32Array | Int32Array, lengths: Uint32Array | number[]): Record<ModelStage, number>;
  readonly timing: { hostMs: number; totalMs: number; tokens: number } | null;
  destroy(): void;
}
/** EmbeddingRuntime over the model: give `prepacked` (a parsed .wgpack) or a `model`. */
export class HipQwen3Runtime implements EmbeddingRuntime {
  constructor(options: HipModelOptions & { prepacked?: PrepackedModel; model?: HipQwen3Model;
                                           context?: DeviceContext; device?: number });
  readonly packing: 'varlen';
  readonly model: HipQwen3Model;
  createPlan(batch: number, sequence: number): HipQwen3Plan;
  destroy(): void;
}
