/** llm/weights-q8-io.ts:14-23 */
export interface QuantWeightManifestEntry {
  name: string;
  kind: "quant";
  /** `[N, K]` */
  shape: [number, number];
  /** Offset into the codes file, in int8 elements. */
  codesOffset: number;
  /** Offset into the scales file, in f32 elements. */
  scaleOffset: number;
}
/** llm/weights-q8-io.ts:25-31 */
export interface NormWeightManifestEntry {
  name: string;
  kind: "norm";
  shape: [number];
  /** Offset into the norms file, in f32 elements. */
  offset: number;
}
export type WeightManifestEntry = QuantWeightManifestEntry | NormWeightManifestEntry;
/** llm/weights-q8-io.ts:36-47 */
export interface WeightManifestConfig {
  numLayers: number;
  hiddenSize: number;
  numHeads: number;
  numKvHeads: number;
  headDim: number;
  ffnHidden: number;
  vocabSize: number;
  ropeTheta: number;
  rmsNormEps: number;
  tieEmbeddings: boolean;
}
export interface QuantizedLinear {
  codes: Int8Array;
  scale: Float32Array;
}
export interface LlamaLayerWeightsQ8 {
  attnNorm: Float32Array;
  wq: QuantizedLinear;
  wk: QuantizedLinear;
  wv: QuantizedLinear;
  wo: QuantizedLinear;
  ffnNorm: Float32Array;
  wGate: QuantizedLinear;
  wUp: QuantizedLinear;
  wDown: QuantizedLinear;
}
export interface LlamaWeightsQ8 {
  embedTokens: QuantizedLinear;
  layers: LlamaLayerWeightsQ8[];
  finalNorm: Float32Array;
  lmHead: QuantizedLinear;
}
export declare function llamaConfigFromManifest(config: WeightManifestConfig, maxSeqLen: number): WeightManifestConfig & { maxSeqLen: number };
export declare function buildLlamaWeightsQ8(entries: readonly WeightManifestEntry[], codesBuffer: ArrayBufferLike, scalesBuffer: ArrayBufferLike, normsBuffer: ArrayBufferLike, numLayers: number): LlamaWeightsQ8;
