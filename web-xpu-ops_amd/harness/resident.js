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
//
// Consecutive single-vector matvecQ8 ops on the same vector (the engine's
// wq/wk/wv projections, llm/engine-q8-resident.ts:1843-1845, and its lm_head
// chunks, :1869) run as one launch of matvecQ8MultiDevice when nothing in the
// run depends on another op of the run: outputs disjoint from each other, from
// the vector and from the run's weights and scales.  Consecutive
// quantizePackQ8 ops with one K run as one quantizePackQ8MultiDevice launch
// under the same condition.  The results are those of the separate ops; only
// the launch count changes (`stats.launches`).  Pass `{ coalesce: false }` to
// the constructor to issue every op on its own.
import { native } from "../native/index.js";

const TYPED = { f32: Float32Array, i32: Int32Array, u32: Uint32Array };

export class ResidentQ8Device {
  constructor(options = {}) {
    this.addon = native();
    this.addon.init();
    this.coalesce = options.coalesce !== false;
    this.stats = { buffersCreated: 0, submits: 0, launches: 0 };
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
    for (let i = 0; i < ops.length; i += 1) {
      const op = ops[i];
      this.stats.launches += 1;
      switch (op.kind) {
        case "matvecQ8": {
          const M = op.M === undefined ? 1 : op.M;
          checkMatvec(op, M);
          const run = this.coalesce && M === 1 ? sameVectorRun(ops, i) : 1;
          if (run > 1) {
            const group = ops.slice(i, i + run);
            a.matvecQ8MultiDevice(group.map((g) => [g.weight.ptr, g.scale.ptr, g.output.ptr, g.N]), op.vector.ptr,
                                  op.K);
            i += run - 1;
          } else {
            a.matvecQ8Device(op.weight.ptr, op.scale.ptr, op.vector.ptr, op.output.ptr, op.N, op.K, M);
          }
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
          checkQuantize(op);
          const run = this.coalesce ? quantizeRun(ops, i) : 1;
          if (run > 1) {
            const group = ops.slice(i, i + run);
            a.quantizePackQ8MultiDevice(group.map((g) => [g.input.ptr, g.N, g.packed.ptr, g.scales.ptr]), op.K);
            i += run - 1;
          } else {
            a.quantizePackQ8Device(op.input.ptr, op.N, op.K, op.packed.ptr, op.scales.ptr);
          }
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

function checkMatvec(op, M) {
  const W = Math.ceil(op.K / 4);
  need(op.weight, op.N * W * 4, "weight");
  need(op.scale, op.N * 4, "scale");
  need(op.vector, M * op.K * 4, "vector");
  need(op.output, M * op.N * 4, "output");
}

function checkQuantize(op) {
  need(op.input, op.N * op.K * 4, "input");
  need(op.packed, op.N * Math.ceil(op.K / 4) * 4, "packed");
  need(op.scales, op.N * 4, "scales");
}

/**
 * How many ops from `start` on (at least 1) form a run of quantizePackQ8 ops
 * with the same K, none writing what another of the run reads or writes.
 */
function quantizeRun(ops, start) {
  const K = ops[start].K;
  const ins = [];
  const outs = [];
  let n = 0;
  for (let j = start; j < ops.length; j += 1) {
    const op = ops[j];
    if (op.kind !== "quantizePackQ8") break;
    if (j > start) checkQuantize(op);
    if (op.K !== K) break;
    const input = span(op.input, op.N * op.K * 4);
    const own = [span(op.packed, op.N * Math.ceil(op.K / 4) * 4), span(op.scales, op.N * 4)];
    if (overlaps(own[0], own[1]) || own.some((o) => overlaps(o, input) || ins.some((r) => overlaps(o, r)) ||
        outs.some((w) => overlaps(o, w))) || outs.some((w) => overlaps(w, input))) {
      break;
    }
    ins.push(input);
    outs.push(...own);
    n += 1;
  }
  return Math.max(n, 1);
}

/** [start, end) byte range of `bytes` bytes at a resident buffer's address. */
function span(buffer, bytes) {
  return [buffer.ptr, buffer.ptr + BigInt(bytes)];
}

function overlaps(x, y) {
  return x[0] < y[1] && y[0] < x[1] && x[0] < x[1] && y[0] < y[1];
}

/**
 * How many ops from `start` on (at least 1) form a run of single-vector
 * matvecQ8 ops on the same vector and K with no op of the run reading what
 * another writes, so that one launch gives what the ops in order would.
 */
function sameVectorRun(ops, start) {
  const first = ops[start];
  const vec = span(first.vector, first.K * 4);
  const outs = [];
  const ins = [];
  let n = 0;
  for (let j = start; j < ops.length; j += 1) {
    const op = ops[j];
    if (op.kind !== "matvecQ8" || (op.M !== undefined && op.M !== 1)) break;
    if (j > start) checkMatvec(op, 1);
    if (op.K !== first.K || op.vector.ptr !== first.vector.ptr) break;
    const out = span(op.output, op.N * 4);
    const reads = [span(op.weight, op.N * Math.ceil(op.K / 4) * 4), span(op.scale, op.N * 4)];
    if (overlaps(out, vec) || outs.some((o) => overlaps(o, out)) ||
        reads.some((r) => outs.some((o) => overlaps(o, r))) || ins.some((r) => overlaps(r, out))) {
      break;
    }
    outs.push(out);
    ins.push(...reads);
    n += 1;
  }
  return Math.max(n, 1);
}

function need(buffer, bytes, name) {
  if (!buffer || typeof buffer.ptr !== "bigint") throw new TypeError(`${name} must be a resident buffer`);
  if (bytes > buffer.size) throw new RangeError(`${name} buffer holds ${buffer.size} B, ${bytes} B needed`);
}

/** Resolves to null when no gfx950 device is visible (as harness/resident.ts:148 does without an adapter). */
export async function createResidentQ8Device(options = {}) {
  const a = native();
  if (a.deviceCount() === 0) return null;
  return new ResidentQ8Device(options);
}
