/** Raw Node-API addon surface (see web-xpu-ops_amd/napi/wxo_napi.c). */
export interface WxoAddon {
  abiVersion(): number;
  describe(): string;
  deviceCount(): number;
  init(): void;
  synchronize(): void;
  /** Best sustained HBM read bytes/s and one-wide f32 FMA flop/s of this device, measured now. */
  roofline(): { bandwidth: number; compute: number };
  matvecQ8(weight: Uint32Array, scale: Float32Array, vector: Float32Array, N: number, K: number, M?: number): Float32Array;
  /** The same call on a libuv worker thread: scale and vector are copied when it is made; the weight is read while the promise is pending. */
  matvecQ8Async(weight: Uint32Array, scale: Float32Array, vector: Float32Array, N: number, K: number, M?: number): Promise<Float32Array>;
  matvecQ8Residual(weight: Uint32Array, scale: Float32Array, vector: Float32Array, residual: Float32Array, N: number, K: number): Float32Array;
  matvecQ8Ffn(weightGate: Uint32Array, scaleGate: Float32Array, weightUp: Uint32Array, scaleUp: Float32Array, vector: Float32Array, N: number, K: number): Float32Array;
  quantize(input: Float32Array, N: number, D: number): { output: Int32Array; scales: Float32Array };
  packQ8(codes: Int32Array, N: number, K: number): Uint32Array;
  packInt8Rows(codes: Int8Array, N: number, K: number): Uint32Array;
  quantizePackQ8(input: Float32Array, N: number, K: number): { weight: Uint32Array; scale: Float32Array };
  malloc(bytes: number): bigint;
  free(ptr: bigint): void;
  upload(ptr: bigint, data: ArrayBufferView): void;
  download<T extends ArrayBufferView>(ptr: bigint, into: T): T;
  /** Page-locked host memory (a MAP_READ staging buffer's storage). */
  hostAlloc(bytes: number): ArrayBuffer;
  /** Enqueues a device-to-host copy into `into` behind the work already enqueued; the host does not wait. */
  downloadAsync(ptr: bigint, into: ArrayBufferView): void;
  /** Settles when everything enqueued before the call has run; the wait runs off the JS thread. */
  whenDone(): Promise<void>;
  /** Keeps the GPU busy for `us` microseconds on the ops stream (a test aid). */
  spin(us: number): void;
  /** Holds the ops stream until gateRelease(gate) or `maxUs` of GPU time (<= 1e6), whichever comes first. */
  gateHold(maxUs: number): number;
  /** Opens `gate` and every gate held before it. */
  gateRelease(gate: number): void;
  copy(dst: bigint, src: bigint, bytes: number): void;
  matvecQ8Device(weight: bigint, scale: bigint, vector: bigint, output: bigint, N: number, K: number, M?: number): void;
  matvecQ8MultiDevice(projections: [bigint, bigint, bigint, number][], vector: bigint, K: number): void;
  quantizePackQ8MultiDevice(matrices: [bigint, number, bigint, bigint][], K: number): void;
  matvecQ8ResidualDevice(weight: bigint, scale: bigint, vector: bigint, residual: bigint, output: bigint, N: number, K: number): void;
  matvecQ8FfnDevice(weightGate: bigint, scaleGate: bigint, weightUp: bigint, scaleUp: bigint, vector: bigint, output: bigint, N: number, K: number): void;
  quantizeDevice(input: bigint, N: number, D: number, output: bigint, scales: bigint): void;
  packQ8Device(codes: bigint, N: number, K: number, packed: bigint): void;
  packInt8RowsDevice(codes: bigint, N: number, K: number, packed: bigint): void;
  quantizePackQ8Device(input: bigint, N: number, K: number, packed: bigint, scales: bigint): void;
}
export declare const ADDON_PATH: string;
export declare function native(): WxoAddon;
export declare function describe(): string;
