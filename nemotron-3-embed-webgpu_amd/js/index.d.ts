// Type declarations of the JavaScript host (erasable TypeScript: interfaces
// and declarations only). EmbeddingPlan, EmbeddingRuntime and TokenizerLike
// are the reference's interfaces (src/webgpu/embedding-engine.ts:1-14), so a
// NemotronHipModel can be handed to any code written against them.

export interface TokenizerResult { input_ids: { tolist(): number[][] } }
export type TokenizerLike = (text: string) => TokenizerResult;

export interface EmbeddingPlan {
  run(ids: Uint32Array, lengths: Uint32Array): Promise<Float32Array[]>;
}

export interface EmbeddingRuntime {
  readonly maxStorageBufferBindingSize?: number;
  createPlan(batch: number, sequence: number): EmbeddingPlan;
}

export interface ModelDims {
  hidden: number; qHeads: number; kvHeads: number; headDim: number; intermediate: number; layers: number;
  vocab: number; mergeAfterLayer: number; rmsEpsilon: number; ropeTheta: number; kvStrideThreshold: number;
  kvStride: number;
  /** 0: the reference code's stride rule in every layer (src/webgpu/ops.ts:258); 1: README.md:26's rule,
   *  every key before the merge. */
  kvDenseBeforeMerge: number;
}

export declare const GGMLType: { readonly F32: 0; readonly F16: 1; readonly Q4_0: 2; readonly Q4_K: 12; readonly Q6_K: 14 };
export declare function contextualMergedLength(sequence: number): number;
export declare function referenceDims(): ModelDims;
export declare function configDims(): ModelDims;

export declare class HipDevice {
  constructor(index?: number);
  readonly index: number;
  destroy(): void;
}
export declare function requestHipDevice(index?: number): HipDevice;

export interface TensorEntry { name: string; dimensions: number[]; type: number; byteOffset: number; byteLength: number; storage?: string }
export interface TensorSource { tensors: Map<string, TensorEntry>; buffer: ArrayBuffer }

export declare class NemotronHipPlan implements EmbeddingPlan {
  readonly batch: number;
  readonly inputSequence: number;
  readonly sequence: number;
  run(ids: Uint32Array, sequenceLengths: Uint32Array): Promise<Float32Array[]>;
  profile(ids: Uint32Array, sequenceLengths: Uint32Array): Promise<Record<string, number>>;
  destroy(): void;
}

export declare class NemotronHipModel implements EmbeddingRuntime {
  constructor(device: HipDevice, source: TensorSource | PrepackedModel | GGUFModel | { synthetic: number },
              options?: { dims?: Partial<ModelDims>; embeddingType?: number });
  readonly dims: ModelDims;
  readonly maxStorageBufferBindingSize?: number;
  createPlan(batch: number, sequence: number): NemotronHipPlan;
  destroy(): void;
}

export declare class NemotronEmbeddingEngine {
  constructor(runtime: EmbeddingRuntime, tokenizer: TokenizerLike, maxBatchSize?: number, batchWindowMs?: number,
              bosToken?: number, padToken?: number);
  readonly maxBatchSize: number;
  readonly batchWindowMs: number;
  readonly bosToken: number;
  readonly padToken: number;
  embed(text: string): Promise<Float32Array>;
}

export interface PackedTensorBytes { name: string; dimensions: number[]; type: number; storage: string; bytes: Uint8Array }
export interface PrepackedHeader {
  version: 2; sourceSha256: string; sourceBytes: number; layout: string; tileRows: 32; blockValues: 32;
  blockBytes: 20; metadata: Record<string, unknown>;
  tensors: Array<{ name: string; dimensions: number[]; type: number; storage: string; offset: number; byteLength: number }>;
}
export interface PrepackedModel {
  header: PrepackedHeader;
  tensors: Map<string, TensorEntry & { offset: number; storage: string }>;
  buffer: ArrayBuffer;
  dataOffset: number;
}
export declare function packQ40Tile32(name: string, parts: Array<{ name: string; k: number; n: number; bytes: Uint8Array }>): PackedTensorBytes;
export declare function rawTensor(name: string, dimensions: number[], type: number, bytes: Uint8Array): PackedTensorBytes;
export declare function buildPrepackedFile(sourceSha256: string, sourceBytes: number, metadata: Record<string, unknown>,
                                           tensors: PackedTensorBytes[]): Uint8Array;
export declare function parsePrepackedModel(buffer: ArrayBuffer): PrepackedModel;

// GGUF (src/gguf/reader.ts, src/gguf/types.ts)
export type GGUFScalar = string | number | bigint | boolean;
export type GGUFMetadataValue = GGUFScalar | GGUFScalar[];
export interface GGUFTensorInfo {
  name: string; dimensions: number[]; type: number; offset: number; byteOffset: number; byteLength: number;
  elementCount: number;
}
export interface GGUFModel {
  version: number; alignment: number; metadata: Map<string, GGUFMetadataValue>; tensors: Map<string, GGUFTensorInfo>;
  dataOffset: number; buffer: ArrayBuffer;
}
export declare class GGUFReader {
  constructor(buffer: ArrayBuffer);
  parse(options?: { metadataKeys?: ReadonlySet<string> }): GGUFModel;
}
export declare function tensorByteLength(type: number, elements: number): number;
export declare function dimsFromMetadata(model: GGUFModel, base: ModelDims): ModelDims;
export declare const NEMOTRON3_METADATA_KEYS: ReadonlySet<string>;

/** scripts/prepack-model.ts: GGUF bytes -> .wgpack bytes (Q4_0 tile32 projections, requantized on the GPU). */
export declare function prepackGGUF(source: Uint8Array, requantize?: (type: number, bytes: Uint8Array, k: number, n: number) => Uint8Array,
                                    device?: number): Uint8Array;
