// Registration and agreement helpers for the Node-side suites.
import assert from "assert";
import { readFileSync } from "fs";
import { dirname, join } from "path";
import { fileURLToPath } from "url";

export { assert };

export function test(file, name, fn) {
  globalThis.__wxoTests.push({ file, name, fn, gpu: false });
}
export function gpuTest(file, name, fn) {
  globalThis.__wxoTests.push({ file, name, fn, gpu: true });
}

/** Thrown by a test that cannot run here; the runner lists it as skipped, with the reason. */
export class Skip extends Error {}

const golden = join(dirname(fileURLToPath(import.meta.url)), "..", "golden");
export const kat = JSON.parse(readFileSync(join(golden, "kat.json"), "utf8"));

/** Bit-level equality of two typed arrays (NaN == NaN). */
export function assertBitsEqual(got, want, what) {
  assert.strictEqual(got.length, want.length, `${what}: length`);
  const g = new Uint32Array(got.buffer, got.byteOffset, got.length * got.BYTES_PER_ELEMENT / 4);
  const w = new Uint32Array(want.buffer, want.byteOffset, want.length * want.BYTES_PER_ELEMENT / 4);
  if (got instanceof Float32Array) {
    for (let i = 0; i < got.length; i += 1) {
      if (Number.isNaN(want[i]) && Number.isNaN(got[i])) continue;
      if (g[i] !== w[i]) assert.fail(`${what}: index ${i} got ${got[i]} want ${want[i]}`);
    }
    return;
  }
  for (let i = 0; i < got.length; i += 1) if (got[i] !== want[i]) assert.fail(`${what}: index ${i} got ${got[i]} want ${want[i]}`);
  void g; void w;
}

/**
 * matvecQ8 tolerance: |y - y_ref| <= 1e-5 * sum_k |s q x| + 1e-7 per row, the
 * bound taken in f64 from the same packed words (any summation order of the
 * f32 kernel stays inside it).
 */
export function assertMatvecAgrees(got, want, { weight, scale, vector, N, K }, what) {
  assert.strictEqual(got.length, want.length, `${what}: length`);
  const W = Math.ceil(K / 4);
  for (let n = 0; n < N; n += 1) {
    let bound = 0;
    for (let k = 0; k < K; k += 1) {
      const byte = (weight[n * W + (k >> 2)] >>> ((k & 3) * 8)) & 0xff;
      bound += Math.abs((byte >= 128 ? byte - 256 : byte) * vector[k]);
    }
    bound *= Math.abs(scale[n]);
    if (Number.isNaN(want[n]) && Number.isNaN(got[n])) continue;
    const err = Math.abs(got[n] - want[n]);
    if (!(err <= 1e-5 * bound + 1e-7)) assert.fail(`${what}: row ${n} got ${got[n]} want ${want[n]} |err| ${err} > ${1e-5 * bound + 1e-7}`);
  }
}

function absBound({ weight, scale, vector, N, K }) {
  const W = Math.ceil(K / 4);
  const out = new Float64Array(N);
  for (let n = 0; n < N; n += 1) {
    let b = 0;
    for (let k = 0; k < K; k += 1) {
      const byte = (weight[n * W + (k >> 2)] >>> ((k & 3) * 8)) & 0xff;
      b += Math.abs((byte >= 128 ? byte - 256 : byte) * vector[k]);
    }
    out[n] = b * Math.abs(scale[n]);
  }
  return out;
}

// One f32 rounding step at |v|.
function ulp32(v) {
  const a = Math.fround(Math.abs(v));
  if (!Number.isFinite(a)) return 0;
  const bits = new Uint32Array(new Float32Array([a]).buffer)[0];
  const next = new Float32Array(new Uint32Array([bits + 1]).buffer)[0];
  return next - a;
}

/** matvecQ8Residual: the projection's bar plus one f32 rounding step of the sum. */
export function assertResidualAgrees(got, want, args, what) {
  const b = absBound(args);
  for (let n = 0; n < args.N; n += 1) {
    if (Number.isNaN(want[n]) && Number.isNaN(got[n])) continue;
    const allowed = 1e-5 * b[n] + 1e-7 + ulp32(want[n]);
    const err = Math.abs(got[n] - want[n]);
    if (!(err <= allowed)) assert.fail(`${what}: row ${n} got ${got[n]} want ${want[n]} |err| ${err} > ${allowed}`);
  }
}

/**
 * matvecQ8Ffn: each projection's bar carried through silu(g) * u (|silu'| <= 1.0999),
 * plus one f32 rounding step of silu(g) (times |u|) and one of the product.
 */
export function assertFfnAgrees(got, gate, up, silu, argsGate, argsUp, what) {
  const bg = absBound(argsGate), bu = absBound(argsUp);
  for (let n = 0; n < argsGate.N; n += 1) {
    const sg = Math.fround(silu(gate[n]));
    const want = Math.fround(sg * up[n]);
    if (Number.isNaN(want) && Number.isNaN(got[n])) continue;
    const eg = 1e-5 * bg[n] + 1e-7, eu = 1e-5 * bu[n] + 1e-7;
    const allowed = 1.0999 * eg * Math.abs(up[n]) + Math.abs(sg) * eu + 1.0999 * eg * eu +
      ulp32(sg) * Math.abs(up[n]) + ulp32(want);
    const err = Math.abs(got[n] - want);
    if (!(err <= allowed)) assert.fail(`${what}: row ${n} got ${got[n]} want ${want} |err| ${err} > ${allowed}`);
  }
}
