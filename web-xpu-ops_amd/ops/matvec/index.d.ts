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

/** ops/matvec/reference.ts:196-207 */
export interface MatVecQ8FfnArgs {
  /** `[N, ceil(K/4)] u32` — `matvecQ8`'s packed format, gate projection. */
  weightGate: Uint32Array;
  /** `[N]` — gate's per-row scale. */
  scaleGate: Float32Array;
  /** `[N, ceil(K/4)] u32` — up projection, same wire format as `weightGate`. */
  weightUp: Uint32Array;
  /** `[N]` — up's per-row scale. */
  scaleUp: Float32Array;
  /** `[K]`, shared by both projections. */
  vector: Float32Array;
  N: number;
  K: number;
}

/** ops/matvec/reference.ts:235-243 */
export interface MatVecQ8ResidualArgs {
  weight: Uint32Array;
  scale: Float32Array;
  vector: Float32Array;
  /** `[N]`, added to each row's matvecQ8 output after the scale. */
  residual: Float32Array;
  N: number;
  K: number;
}

/** `y[n] = (sum_k q[n,k] * vector[k]) * scale[n]`, f32 accumulation on the GPU. */
export declare function matvecQ8(args: MatVecQ8Args): Float32Array;
export declare function matvecQ8(vector: Float32Array, weight: Uint32Array, scale: Float32Array, N: number, K: number): Float32Array;
/** `[M, N]` row-major: M independent matvecQ8 calls on one weight. */
export declare function matvecQ8Batched(args: MatVecQ8BatchedArgs): Float32Array;
/** `silu(gate[n]) * up[n]`: silu in f64 rounded to f32, then one f32 product. */
export declare function matvecQ8Ffn(args: MatVecQ8FfnArgs): Float32Array;
/** `residual[n] + matvecQ8 row n`, the sum rounded once to f32. */
export declare function matvecQ8Residual(args: MatVecQ8ResidualArgs): Float32Array;
/** ops/matvec/reference.ts:267 — `[N, K]` codes to `[N, ceil(K/4)]` packed words. */
export declare function packQ8(args: { codes: Int32Array | Int8Array; N: number; K: number }): Uint32Array;
