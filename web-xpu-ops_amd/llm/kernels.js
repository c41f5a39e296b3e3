// llm/kernels: the non-resident engine's dispatch wrapper (llm/kernels.ts:195-211
// runMatVecQ8), same signature.  The first argument is the reference's WebGPU
// `Runner["run"]`; this backend does not need it and accepts anything there, so
// a call site compiles unchanged.  No 65,535-row chunking is needed here
// (llm/kernels.ts:128-151 exists for WebGPU's workgroup limit): one call covers
// any N.  As the reference's dispatch does, the call returns at once and the
// GPU work (and the weight's trip over PCIe) is waited for off the JS thread;
// the vector is taken when the call is made.
import { native } from "../native/index.js";

/** `runMatVecQ8(run, { weight, scale, vector, M, K })` -> Promise<Float32Array [M]>, M = rows. */
export async function runMatVecQ8(_run, { weight, scale, vector, M, K }) {
  return native().matvecQ8Async(weight, scale, vector, M, K, 1);
}
