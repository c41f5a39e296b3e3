// Declarations of harness/resident.js: the reference's ResidentDevice
// (harness/resident.ts:28-145) for the ops this build runs, plus native op kinds.
export interface ResidentBuffer {
  /** Device address (storage buffers) or null (uniform buffers in host memory, MAP_READ staging buffers in page-locked host memory). */
  readonly ptr: bigint | null;
  readonly size: number;
  readonly usage: number;
  readonly kind: "storage" | "uniform" | "staging";
  /** GPUBuffer.destroy(): releases the memory now; later calls do nothing, later uses throw. */
  destroy(): void;
}
export declare class UnsupportedPipelineError extends Error {
  readonly name: "UnsupportedPipelineError";
}
export interface ResidentPipeline {
  /** The MI355X op the WGSL interface was recognised as. */
  readonly op: "matvecQ8" | "matvecQ8Ffn" | "matvecQ8Residual" | "matmulQ8";
  readonly entry: string;
}
export interface ResidentBindGroup {
  readonly pipeline: ResidentPipeline;
  readonly buffers: readonly ResidentBuffer[];
}
/** harness/resident.ts:28-39 ResidentOp, plus this device's native op kinds. */
export type ResidentOp =
  | { kind: "dispatch"; pipeline: ResidentPipeline; bindGroup: ResidentBindGroup; workgroups: [number] | [number, number] | [number, number, number] }
  | { kind: "copy"; src: ResidentBuffer; srcOffset: number; dst: ResidentBuffer; dstOffset: number; size: number }
  | { kind: "matvecQ8"; weight: ResidentBuffer; scale: ResidentBuffer; vector: ResidentBuffer; output: ResidentBuffer; N: number; K: number; M?: number }
  | { kind: "matvecQ8Ffn"; weightGate: ResidentBuffer; scaleGate: ResidentBuffer; weightUp: ResidentBuffer; scaleUp: ResidentBuffer; vector: ResidentBuffer; output: ResidentBuffer; N: number; K: number }
  | { kind: "matvecQ8Residual"; weight: ResidentBuffer; scale: ResidentBuffer; vector: ResidentBuffer; residual: ResidentBuffer; output: ResidentBuffer; N: number; K: number }
  | { kind: "packInt8Rows"; codes: ResidentBuffer; N: number; K: number; packed: ResidentBuffer }
  | { kind: "quantizePackQ8"; input: ResidentBuffer; N: number; K: number; packed: ResidentBuffer; scales: ResidentBuffer }
  | { kind: "matmulQ8"; a: ResidentBuffer; weight: ResidentBuffer; scale: ResidentBuffer; output: ResidentBuffer; N: number; M: number; K: number }
  | { kind: "dequantTranspose"; weight: ResidentBuffer; scale: ResidentBuffer; outFeatures: number; inFeatures: number; output: ResidentBuffer }
  | { kind: "gatherDequantRows"; codes: ResidentBuffer; scale: ResidentBuffer; rows: number; D: number; indices: ResidentBuffer; count: number; output: ResidentBuffer };
/** harness/resident.ts:41-48; the values land in `staging` (a MAP_READ buffer of this device) when given, else in pooled page-locked memory. */
export interface ResidentReadback {
  staging?: ResidentBuffer;
  source: ResidentBuffer;
  sourceOffset: number;
  length: number;
  type: "f32" | "i32" | "u32";
}
/** harness/resident.ts:75-96. */
export interface BatchProfileSink {
  submitToDoneMs: number | null;
  readbackMs: number | null;
  gpuEntries: { label: string; seconds: number }[];
}
export interface BatchProfile {
  labels?: (string | null | undefined)[];
  sink: BatchProfileSink;
}
export interface ResidentQ8Options {
  /** Run consecutive same-vector matvecQ8 ops as one launch (default true). */
  coalesce?: boolean;
  /** Capture a batch that repeats its predecessor as a HIP graph and replay it (default true). */
  graphs?: boolean;
  /**
   * Where a batch waits for the GPU: "async" (default) off the JS thread, so
   * the event loop runs and later batches can be enqueued meanwhile; "block"
   * on the JS thread, ~8-10 us less per awaited batch.
   */
  wait?: "async" | "block";
}
export declare const BufferUsage: {
  readonly MAP_READ: number; readonly MAP_WRITE: number; readonly COPY_SRC: number; readonly COPY_DST: number;
  readonly INDEX: number; readonly VERTEX: number; readonly UNIFORM: number; readonly STORAGE: number;
  readonly INDIRECT: number; readonly QUERY_RESOLVE: number;
};
export declare class ResidentQ8Device {
  constructor(options?: ResidentQ8Options);
  readonly stats: { buffersCreated: number; pipelinesCreated: number; submits: number; launches: number;
    graphsCaptured: number; graphLaunches: number };
  /** Whether repeating batches are captured and replayed (the `graphs` option). */
  graphs: boolean;
  /** Where a batch waits for the GPU (the `wait` option). */
  wait: "async" | "block";
  readonly timestampsSupported: boolean;
  createStorageBuffer(bytes: number, usage?: number): ResidentBuffer;
  createUniformBuffer(bytes: number): ResidentBuffer;
  upload(buffer: ResidentBuffer, offset: number, data: ArrayBufferView): void;
  pipelineFor(code: string, entry?: string): Promise<ResidentPipeline>;
  bindGroup(pipeline: ResidentPipeline, buffers: ResidentBuffer[]): Promise<ResidentBindGroup>;
  /**
   * Enqueues the ops and the readback copies at once and settles when the GPU
   * has run them, waiting off the JS thread; batches called while others are
   * in flight run after them, in call order.
   */
  batch(ops: ResidentOp[], readback?: ResidentReadback[], profile?: BatchProfile): Promise<(Float32Array | Int32Array | Uint32Array)[]>;
  /** Settles once every batch in flight has. */
  idle(): Promise<void>;
  destroy(): void;
}
export declare function createResidentQ8Device(options?: ResidentQ8Options): Promise<ResidentQ8Device | null>;
/** harness/resident.ts:148: the same factory under the reference's name. */
export declare const createResidentDevice: typeof createResidentQ8Device;
/** harness/wgsl.ts:12-31 Binding and Dispatch. */
export type Binding =
  | { kind: "storage"; data: Float32Array | Int32Array | Uint32Array }
  | { kind: "out"; type: "f32" | "i32" | "u32"; length: number }
  | { kind: "scratch"; length: number }
  | { kind: "uniform"; data: ArrayBuffer };
export interface Dispatch {
  code: string;
  entry?: string;
  bindings: Binding[];
  workgroups: [number] | [number, number] | [number, number, number];
}
/** harness/resident.ts:429-485: one dispatch per call on its own buffers, destroyed afterwards. */
export declare function runnerFromResident(device: ResidentQ8Device): (dispatch: Dispatch) => Promise<(Float32Array | Int32Array | Uint32Array)[]>;
/** harness/wgsl.ts:324-333 params(): a uniform's bytes, 4 per field, at least 16. */
export declare function params(fields: ["u32" | "i32" | "f32", number][]): ArrayBuffer;
