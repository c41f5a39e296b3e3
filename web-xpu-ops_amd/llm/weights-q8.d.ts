/** llm/weights.ts / weights-q8.ts: one quantized linear layer, `codes` `[rows, D]` int8 with one scale per row. */
export interface QuantizedLinear {
  codes: Int8Array;
  scale: Float32Array;
}

/** llm/weights-q8.ts:137 — packQ8 on one-byte-per-code input. */
export declare function packInt8Rows(codes: Int8Array, N: number, K: number): Uint32Array;

/** llm/weights-q8.ts:161 — the packed weight back to f32 `[N, K]`, code * scale per element. */
export declare function dequantizePackedQ8(weight: Uint32Array, scale: Float32Array, N: number, K: number): Float32Array;

/** llm/weights-q8.ts:207 — requested rows dequantized in request order; out-of-range indices gather zeros. */
export declare function gatherDequantRows(table: QuantizedLinear, indices: number[] | Int32Array | Uint32Array, D: number): Float32Array;
