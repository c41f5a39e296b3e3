// harness/resident: device-resident buffers and one-sync batches for a decode
// engine, the MI355X counterpart of the reference's ResidentDevice
// (harness/resident.ts:98-145, createResidentDevice :148, batch :231-382)
// restricted to what the matvecQ8 path needs: storage buffers, uploads,
// matvecQ8 (plain, fused FFN, fused residual) / quantize+packQ8 ops, the
// prefill-side matmulQ8 / dequantTranspose / gatherDequantRows ops and device
// copies recorded into one batch,
// one synchronisation per batch, selective readback.
//
// Buffers are HBM allocations (hipMalloc) owned by the device object and freed
// by destroy(); ops are enqueued in order on the device's stream as batch()
// walks them, so nothing is allocated inside a decode loop's steady state
// (`stats.buffersCreated` stays flat, as the reference's test checks).
import { native } from "../native/index.js";

const TYPED = { f32: Float32Array, i32: Int32Array, u32: Uint32Array };

export class ResidentQ8Device {
  constructor() {
    this.addon = native();
    this.addon.init();
    this.stats = { buffersCreated: 0, submits: 0 };
    this.buffers = new Set();
  }

  /** A device buffer of `bytes` bytes: `{ ptr: bigint, size: number }`. */
  createStorageBuffer(bytes) {
    const ptr = this.addon.malloc(bytes);
    const buffer = { ptr, size: bytes };
    this.buffers.add(buffer);
    this.stats.buffersCreated += 1;
    return buffer;
  }

  /** Host-to-device copy of `data` into `buffer` at byte `offset` (synchronous). */
  upload(buffer, offset, data) {
    if (offset < 0 || offset + data.byteLength > buffer.size) {
      throw new RangeError(`upload of ${data.byteLength} B at ${offset} overflows a ${buffer.size} B buffer`);
    }
    this.addon.upload(buffer.ptr + BigInt(offset), data);
  }

  /**
   * Enqueues every op in order, waits once, then reads back only `readback`.
   * ops: { kind: "matvecQ8", weight, scale, vector, output, N, K, M? }
   *      { kind: "matvecQ8Ffn", weightGate, scaleGate, weightUp, scaleUp, vector, output, N, K }
   *      { kind: "matvecQ8Residual", weight, scale, vector, residual, output, N, K }
   *        (output may be the residual buffer: the residual stream updated in place)
   *      { kind: "packInt8Rows", codes, N, K, packed }   (int8 codes -> packed words)
   *      { kind: "quantizePackQ8", input, N, K, packed, scales }
   *      { kind: "matmulQ8", a, weight, scale, output, N, M, K }   (prefill GEMM, output [N, M])
   *      { kind: "dequantTranspose", weight, scale, outFeatures, inFeatures, output }
   *      { kind: "gatherDequantRows", codes, scale, rows, D, indices, count, output }
   *        (indices: an int64 buffer of `count` row ids)
   *      { kind: "copy", src, srcOffset, dst, dstOffset, size }
   * readback: { source, sourceOffset, length, type: "f32" | "i32" | "u32" }
   */
  async batch(ops, readback = []) {
    const a = this.addon;
    for (const op of ops) {
      switch (op.kind) {
        case "matvecQ8": {
          const M = op.M === undefined ? 1 : op.M;
          const W = Math.ceil(op.K / 4);
          need(op.weight, op.N * W * 4, "weight");
          need(op.scale, op.N * 4, "scale");
          need(op.vector, M * op.K * 4, "vector");
          need(op.output, M * op.N * 4, "output");
          a.matvecQ8Device(op.weight.ptr, op.scale.ptr, op.vector.ptr, op.output.ptr, op.N, op.K, M);
          break;
        }
        case "matvecQ8Ffn": {
          const bytes = op.N * Math.ceil(op.K / 4) * 4;
          need(op.weightGate, bytes, "weightGate");
          need(op.scaleGate, op.N * 4, "scaleGate");
          need(op.weightUp, bytes, "weightUp");
          need(op.scaleUp, op.N * 4, "scaleUp");
          need(op.vector, op.K * 4, "vector");
          need(op.output, op.N * 4, "output");
          a.matvecQ8FfnDevice(op.weightGate.ptr, op.scaleGate.ptr, op.weightUp.ptr, op.scaleUp.ptr, op.vector.ptr,
                              op.output.ptr, op.N, op.K);
          break;
        }
        case "matvecQ8Residual": {
          need(op.weight, op.N * Math.ceil(op.K / 4) * 4, "weight");
          need(op.scale, op.N * 4, "scale");
          need(op.vector, op.K * 4, "vector");
          need(op.residual, op.N * 4, "residual");
          need(op.output, op.N * 4, "output");
          a.matvecQ8ResidualDevice(op.weight.ptr, op.scale.ptr, op.vector.ptr, op.residual.ptr, op.output.ptr, op.N,
                                   op.K);
          break;
        }
        case "packInt8Rows": {
          need(op.codes, op.N * op.K, "codes");
          need(op.packed, op.N * Math.ceil(op.K / 4) * 4, "packed");
          a.packInt8RowsDevice(op.codes.ptr, op.N, op.K, op.packed.ptr);
          break;
        }
        case "quantizePackQ8": {
          need(op.input, op.N * op.K * 4, "input");
          need(op.packed, op.N * Math.ceil(op.K / 4) * 4, "packed");
          need(op.scales, op.N * 4, "scales");
          a.quantizePackQ8Device(op.input.ptr, op.N, op.K, op.packed.ptr, op.scales.ptr);
          break;
        }
        case "matmulQ8": {
          need(op.a, op.N * op.K * 4, "a");
          need(op.weight, op.M * Math.ceil(op.K / 4) * 4, "weight");
          need(op.scale, op.M * 4, "scale");
          need(op.output, op.N * op.M * 4, "output");
          a.matmulQ8Device(op.a.ptr, op.weight.ptr, op.scale.ptr, op.output.ptr, op.N, op.M, op.K);
          break;
        }
        case "dequantTranspose": {
          need(op.weight, op.outFeatures * Math.ceil(op.inFeatures / 4) * 4, "weight");
          need(op.scale, op.outFeatures * 4, "scale");
          need(op.output, op.outFeatures * op.inFeatures * 4, "output");
          a.dequantTransposeDevice(op.weight.ptr, op.scale.ptr, op.outFeatures, op.inFeatures, op.output.ptr);
          break;
        }
        case "gatherDequantRows": {
          need(op.codes, op.rows * op.D, "codes");
          need(op.scale, op.rows * 4, "scale");
          need(op.indices, op.count * 8, "indices");
          need(op.output, op.count * op.D * 4, "output");
          a.gatherDequantRowsDevice(op.codes.ptr, op.scale.ptr, op.rows, op.D, op.indices.ptr, op.count, op.output.ptr);
          break;
        }
        case "copy": {
          if (op.srcOffset + op.size > op.src.size || op.dstOffset + op.size > op.dst.size) {
            throw new RangeError("copy range outside its buffers");
          }
          a.copy(op.dst.ptr + BigInt(op.dstOffset), op.src.ptr + BigInt(op.srcOffset), op.size);
          break;
        }
        default:
          throw new TypeError(`unknown resident op kind ${op.kind}`);
      }
    }
    a.synchronize();
    this.stats.submits += 1;
    return readback.map((r) => {
      const T = TYPED[r.type];
      if (!T) throw new TypeError(`unknown readback type ${r.type}`);
      if (r.sourceOffset + r.length * 4 > r.source.size) throw new RangeError("readback outside its buffer");
      return a.download(r.source.ptr + BigInt(r.sourceOffset), new T(r.length));
    });
  }

  /** Frees every buffer this device created. */
  destroy() {
    for (const b of this.buffers) this.addon.free(b.ptr);
    this.buffers.clear();
  }
}

function need(buffer, bytes, name) {
  if (!buffer || typeof buffer.ptr !== "bigint") throw new TypeError(`${name} must be a resident buffer`);
  if (bytes > buffer.size) throw new RangeError(`${name} buffer holds ${buffer.size} B, ${bytes} B needed`);
}

/** Resolves to null when no gfx950 device is visible (as harness/resident.ts:148 does without an adapter). */
export async function createResidentQ8Device() {
  const a = native();
  if (a.deviceCount() === 0) return null;
  return new ResidentQ8Device();
}
