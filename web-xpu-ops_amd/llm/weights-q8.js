// llm/weights-q8: the caller-side packing entry of the reference
// (llm/weights-q8.ts:137-139 packInt8Rows), on the GPU.
import { native } from "../native/index.js";

/** `packInt8Rows(codes: Int8Array, N, K)` -> Uint32Array [N * ceil(K/4)]. */
export function packInt8Rows(codes, N, K) {
  return native().packInt8Rows(codes, N, K);
}
