/** ops/matvec/reference.ts:99-110 */
export interface MatVecQ8Args {
  /** `[N, ceil(K/4)]` u32, row-major, 4 codes per word, least-significant byte first. */
  weight: Uint32Array;
  /** `[N]`, one absmax-derived scale per row — `quantize`'s convention. */
  scale: Float32Array;
  /** `[K]`, shared by every row. */
  vector: Float32Array;
  /** Rows of `weight`, and the length of the output. */
  N: number;
  /** Columns before packing, and the length of `vector`. */
  K: number;
}

export interface MatVecQ8BatchedArgs {
  weight: Uint32Array;
  scale: Float32Array;
  /** `[M, K]` row-major. */
  vectors: Float32Array;
  N: number;
  K: number;
  M: number;
}

/** `y[n] = (sum_k q[n,k] * vector[k]) * scale[n]`, f32 accumulation on the GPU. */
export declare function matvecQ8(args: MatVecQ8Args): Float32Array;
export declare function matvecQ8(vector: Float32Array, weight: Uint32Array, scale: Float32Array, N: number, K: number): Float32Array;
/** `[M, N]` row-major: M independent matvecQ8 calls on one weight. */
export declare function matvecQ8Batched(args: MatVecQ8BatchedArgs): Float32Array;
/** ops/matvec/reference.ts:267 — `[N, K]` codes to `[N, ceil(K/4)]` packed words. */
export declare function packQ8(args: { codes: Int32Array | Int8Array; N: number; K: number }): Uint32Array;
