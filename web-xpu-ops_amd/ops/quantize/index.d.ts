/** ops/quantize/reference.ts:13-22 */
export declare function quantize(args: { input: Float32Array; N: number; D: number }): { output: Int32Array; scales: Float32Array };
/** `packQ8(quantize(w).output, N, K)` + `quantize(w).scales`, fused. */
export declare function quantizePackQ8(args: { input: Float32Array; N: number; K: number }): { weight: Uint32Array; scale: Float32Array };
