// ops/matvec: matvecQ8, its fused decode forms and packQ8 on the MI355X, with
// the reference's op API (ops/matvec/reference.ts:99-131 matvecQ8, :196-207
// matvecQ8Ffn, :235-243 matvecQ8Residual, :267-283 packQ8, exported the same
// way as ops/matvec/index.ts:1-11).
//
// Same call shapes and data formats as the reference: the weight is
// [N, ceil(K/4)] u32 with four int8 codes per word, least-significant byte
// first; the scale is [N], applied once per row after the dot product; fresh
// typed arrays come back.  The work runs on the GPU through the Node-API
// addon; there is no CPU fallback.  One deliberate difference: arguments are
// validated (wrong typed-array type -> TypeError, too short -> RangeError)
// where the reference would read `undefined` and produce NaN.
import { native } from "../../native/index.js";

/**
 * `matvecQ8({ weight, scale, vector, N, K })` -> Float32Array [N]
 * (ops/matvec/reference.ts:117), or positionally
 * `matvecQ8(vector, weight, scale, N, K)`.
 */
export function matvecQ8(first, weight, scale, N, K) {
  if (first instanceof Float32Array) {
    return native().matvecQ8(weight, scale, first, N, K, 1);
  }
  const args = first;
  return native().matvecQ8(args.weight, args.scale, args.vector, args.N, args.K, 1);
}

/**
 * M independent matvecQ8 calls on one weight, each loaded weight word reused
 * for every vector: `vectors` is [M, K] row-major, the result [M, N].
 */
export function matvecQ8Batched({ weight, scale, vectors, N, K, M }) {
  return native().matvecQ8(weight, scale, vectors, N, K, M);
}

/**
 * `matvecQ8Ffn({ weightGate, scaleGate, weightUp, scaleUp, vector, N, K })` ->
 * Float32Array [N]: silu(gate row) * up row (ops/matvec/reference.ts:196-207),
 * both weights streamed in one pass.
 */
export function matvecQ8Ffn({ weightGate, scaleGate, weightUp, scaleUp, vector, N, K }) {
  return native().matvecQ8Ffn(weightGate, scaleGate, weightUp, scaleUp, vector, N, K);
}

/**
 * `matvecQ8Residual({ weight, scale, vector, residual, N, K })` ->
 * Float32Array [N]: residual + matvecQ8 row (ops/matvec/reference.ts:235-243).
 */
export function matvecQ8Residual({ weight, scale, vector, residual, N, K }) {
  return native().matvecQ8Residual(weight, scale, vector, residual, N, K);
}

/**
 * `packQ8({ codes, N, K })` -> Uint32Array [N * ceil(K/4)]
 * (ops/matvec/reference.ts:267).  Int32Array codes are taken `& 0xff` like the
 * reference; an Int8Array is accepted too (llm/weights-q8.ts:137-139).
 */
export function packQ8({ codes, N, K }) {
  if (codes instanceof Int8Array) return native().packInt8Rows(codes, N, K);
  return native().packQ8(codes, N, K);
}
