export interface ResidentBuffer {
  readonly ptr: bigint;
  readonly size: number;
}
export type ResidentQ8Op =
  | { kind: "matvecQ8"; weight: ResidentBuffer; scale: ResidentBuffer; vector: ResidentBuffer; output: ResidentBuffer; N: number; K: number; M?: number }
  | { kind: "matvecQ8Ffn"; weightGate: ResidentBuffer; scaleGate: ResidentBuffer; weightUp: ResidentBuffer; scaleUp: ResidentBuffer; vector: ResidentBuffer; output: ResidentBuffer; N: number; K: number }
  | { kind: "matvecQ8Residual"; weight: ResidentBuffer; scale: ResidentBuffer; vector: ResidentBuffer; residual: ResidentBuffer; output: ResidentBuffer; N: number; K: number }
  | { kind: "packInt8Rows"; codes: ResidentBuffer; N: number; K: number; packed: ResidentBuffer }
  | { kind: "quantizePackQ8"; input: ResidentBuffer; N: number; K: number; packed: ResidentBuffer; scales: ResidentBuffer }
  | { kind: "matmulQ8"; a: ResidentBuffer; weight: ResidentBuffer; scale: ResidentBuffer; output: ResidentBuffer; N: number; M: number; K: number }
  | { kind: "dequantTranspose"; weight: ResidentBuffer; scale: ResidentBuffer; outFeatures: number; inFeatures: number; output: ResidentBuffer }
  | { kind: "gatherDequantRows"; codes: ResidentBuffer; scale: ResidentBuffer; rows: number; D: number; indices: ResidentBuffer; count: number; output: ResidentBuffer }
  | { kind: "copy"; src: ResidentBuffer; srcOffset: number; dst: ResidentBuffer; dstOffset: number; size: number };
export interface ResidentQ8Readback {
  source: ResidentBuffer;
  sourceOffset: number;
  length: number;
  type: "f32" | "i32" | "u32";
}
export interface ResidentQ8Options {
  /** Run consecutive same-vector matvecQ8 ops as one launch (default true). */
  coalesce?: boolean;
}
export declare class ResidentQ8Device {
  constructor(options?: ResidentQ8Options);
  readonly stats: { buffersCreated: number; submits: number; launches: number };
  createStorageBuffer(bytes: number): ResidentBuffer;
  upload(buffer: ResidentBuffer, offset: number, data: ArrayBufferView): void;
  batch(ops: ResidentQ8Op[], readback?: ResidentQ8Readback[]): Promise<(Float32Array | Int32Array | Uint32Array)[]>;
  destroy(): void;
}
export declare function createResidentQ8Device(options?: ResidentQ8Options): Promise<ResidentQ8Device | null>;
