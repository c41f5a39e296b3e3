// llm/weights-q8: the caller-side helpers of the reference's packed-weight
// module on the GPU: packInt8Rows (llm/weights-q8.ts:137-139),
// dequantizePackedQ8 (:161-177) and gatherDequantRows (:207-222), same
// signatures and results (bit-exact).
import { native } from "../native/index.js";

/** `packInt8Rows(codes: Int8Array, N, K)` -> Uint32Array [N * ceil(K/4)]. */
export function packInt8Rows(codes, N, K) {
  return native().packInt8Rows(codes, N, K);
}

/** `dequantizePackedQ8(weight, scale, N, K)` -> Float32Array [N * K], code * scale per element. */
export function dequantizePackedQ8(weight, scale, N, K) {
  return native().dequantizePackedQ8(weight, scale, N, K);
}

/**
 * `gatherDequantRows(table: { codes: Int8Array [rows * D], scale: Float32Array [rows] }, indices, D)`
 * -> Float32Array [indices.length * D]: the requested rows dequantized, in
 * request order; indices outside [0, rows) give rows of zeros.
 */
export function gatherDequantRows(table, indices, D) {
  return native().gatherDequantRows(table.codes, table.scale, indices, D);
}
