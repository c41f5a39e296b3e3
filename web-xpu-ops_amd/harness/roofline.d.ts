/** What this device gives, measured now (reference: harness/roofline.ts). */
export interface Roofline {
  /** Best sustained bytes per second read from device memory. */
  bandwidth: number;
  /** Best sustained FLOP/s, counting a fused multiply-add as 2. */
  compute: number;
}
export declare function measureRoofline(runner?: unknown): Promise<Roofline>;
export declare function roofline(runner?: unknown): Promise<Roofline>;
/** The bf16 matrix cores' sustained flop/s on matmulQ8-like operands, measured now (no counterpart in the reference). */
export declare function measureMatrixRoofline(): Promise<number>;
