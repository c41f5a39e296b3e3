/** ops/matmul/reference.ts:82-100 */
export interface MatmulQ8Args {
  /** `[N, K]` f32, row-major — `matmul`'s own `a`. */
  a: Float32Array;
  /** `[M, ceil(K/4)]` u32, row-major, 4 codes per word, least-significant byte first — `matvecQ8`'s own wire format. */
  weight: Uint32Array;
  /** `[M]`, one absmax-derived scale per row. */
  scale: Float32Array;
  /** Rows of `a`, and of the output. */
  N: number;
  /** Rows of `weight`/`scale`, and columns of the output. */
  M: number;
  /** Columns of `a` before packing, and the contracted dimension. */
  K: number;
}

/** ops/matmul/reference.ts:124 — `[N, M]` f32, row-major. */
export declare function matmulQ8(args: MatmulQ8Args): Float32Array;
