/** llm/kernels.ts:185-193 — note `M` is the row count here, as in the reference. */
export interface MatVecQ8Args {
  weight: Uint32Array;
  scale: Float32Array;
  vector: Float32Array;
  M: number;
  K: number;
}
export declare function runMatVecQ8(run: unknown, args: MatVecQ8Args): Promise<Float32Array>;
