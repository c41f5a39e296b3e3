/** llm/weights-q8.ts:137 — packQ8 on one-byte-per-code input. */
export declare function packInt8Rows(codes: Int8Array, N: number, K: number): Uint32Array;
