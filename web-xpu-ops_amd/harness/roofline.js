// What this device gives, measured here and now: the reference's
// harness/roofline.ts (measureRoofline :162-198, roofline :218-222) over the
// addon's wxo_roofline.  The method is the reference's: two 512 MiB buffers of
// hashed words swept once per launch with 16-byte loads (alternately, so no
// sweep is served from the 256 MB Infinity Cache), fastest of several timed
// attempts; FMAs from registers in independent chains.  Ops are reported as a
// fraction of it beside the nominal 8 TB/s.
import { native } from "../native/index.js";

/** { bandwidth: bytes/s, compute: flop/s (an FMA counts 2) }.  The runner
 * argument of the reference's signature is accepted and unused: the addon
 * measures the current device. */
export async function measureRoofline(_runner) {
  return native().roofline();
}

/** The bf16 matrix cores' sustained rate in flop/s on every CU, with operands
 * of matmulQ8's kinds (int8 codes against bf16 parts of random bits): the
 * clock sags under matrix work, so real operands do not get the nominal
 * 2.5 PFLOP/s.  No counterpart in the reference, whose roofline measures HBM
 * and FMA only; matmulQ8 (three matrix flops per useful one) is reported
 * against it. */
export async function measureMatrixRoofline() {
  return native().rooflineMatrix();
}

const CACHE = Symbol.for("web-xpu-ops-mi355x.roofline");

/** The ceiling for this session, measured once and kept on globalThis (as the
 * reference does, so every test file shares one measurement). */
export function roofline(runner) {
  if (globalThis[CACHE] === undefined) globalThis[CACHE] = measureRoofline(runner);
  return globalThis[CACHE];
}
