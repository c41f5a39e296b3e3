import type { ResidentBuffer, ResidentQ8Device } from "../harness/resident.js";
import type { LlamaWeightsQ8, QuantizedLinear } from "./weights-q8-io.js";

export interface ResidentLinear {
  /** packed u32 `[N, ceil(K/4)]`, the reference's wire format */
  weight: ResidentBuffer;
  /** f32 `[N]` */
  scale: ResidentBuffer;
  N: number;
  K: number;
}
export interface ResidentLayerWeightsQ8 {
  attnNorm: ResidentBuffer;
  wq: ResidentLinear;
  wk: ResidentLinear;
  wv: ResidentLinear;
  wo: ResidentLinear;
  ffnNorm: ResidentBuffer;
  wGate: ResidentLinear;
  wUp: ResidentLinear;
  wDown: ResidentLinear;
}
export interface ResidentWeightsQ8 {
  embedTokens: ResidentLinear;
  layers: ResidentLayerWeightsQ8[];
  finalNorm: ResidentBuffer;
  lmHead: ResidentLinear;
}
export declare function uploadQuantizedLinear(device: ResidentQ8Device, linear: QuantizedLinear): Promise<ResidentLinear>;
export declare function uploadResidentWeightsQ8(device: ResidentQ8Device, weights: LlamaWeightsQ8): Promise<ResidentWeightsQ8>;
