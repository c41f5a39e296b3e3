/** ops/dequant_transpose/reference.ts:24-33 */
export interface DequantTransposeArgs {
  /** `[outFeatures, ceil(inFeatures / 4)]` u32, row-major — `ops/matvec`'s `q8` packed wire format (`packQ8`). */
  weight: Uint32Array;
  /** `[outFeatures]`, one absmax-derived scale per row. */
  scale: Float32Array;
  outFeatures: number;
  inFeatures: number;
}

/** ops/dequant_transpose/reference.ts:40 — `[inFeatures, outFeatures]` f32, row-major. */
export declare function dequantTranspose(args: DequantTransposeArgs): Float32Array;
