// ops/matmul: matmulQ8, the prefill GEMM over matvecQ8's packed weight, on the
// MI355X matrix cores, with the reference's op API (ops/matmul/reference.ts:82-137,
// exported as ops/matmul/index.ts:1 does).
//
// `a` is [N, K] f32 row-major (tokens), `weight` [M, ceil(K/4)] u32 with four
// int8 codes per word, least-significant byte first, `scale` [M]; the result is
// a fresh Float32Array [N, M].  The plain f32 `matmul` of the reference is not
// part of this package (the path it serves is the quantized one).  Arguments
// are validated (TypeError / RangeError) where the reference would read
// `undefined`; there is no CPU fallback.
import { native } from "../../native/index.js";

/** `matmulQ8({ a, weight, scale, N, M, K })` -> Float32Array [N * M]. */
export function matmulQ8({ a, weight, scale, N, M, K }) {
  return native().matmulQ8(a, weight, scale, N, M, K);
}
