// ops/quantize: per-row absmax int8 quantization on the MI355X, bit-exact to
// ops/quantize/reference.ts:13-38 (f64 absmax and inverse, JS Math.round ties
// toward +Infinity, clamp to [-127, 127], f32 scale = absmax / 127, scale 1 for
// an all-zero row).  Exported like ops/quantize/index.ts:1.
import { native } from "../../native/index.js";

/** `quantize({ input, N, D })` -> `{ output: Int32Array [N*D], scales: Float32Array [N] }`. */
export function quantize({ input, N, D }) {
  return native().quantize(input, N, D);
}

/**
 * `packQ8(quantize({ input, N, D: K }).output, N, K)` together with the scales,
 * in one GPU pass that never materialises the int32 codes:
 * `{ weight: Uint32Array [N*ceil(K/4)], scale: Float32Array [N] }`.
 */
export function quantizePackQ8({ input, N, K }) {
  return native().quantizePackQ8(input, N, K);
}
