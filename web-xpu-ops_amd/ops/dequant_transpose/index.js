// ops/dequant_transpose: dequantTranspose on the MI355X with the reference's op
// API (ops/dequant_transpose/reference.ts:24-59, exported as
// ops/dequant_transpose/index.ts:1): the packed [outFeatures, ceil(inFeatures/4)]
// weight and its per-row scale -> a fresh Float32Array [inFeatures, outFeatures],
// output[col * outFeatures + row] = code * scale[row], bit-exact.  The
// reference's exact-length checks (:42-47) throw the same messages.
import { native } from "../../native/index.js";

export function dequantTranspose({ weight, scale, outFeatures, inFeatures }) {
  return native().dequantTranspose(weight, scale, outFeatures, inFeatures);
}
