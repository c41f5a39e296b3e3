// The prefill-side op API of this package (ops/matmul, ops/dequant_transpose,
// llm/weights-q8's dequant and gather, the resident batch's prefill ops)
// against the ECMAScript oracle (oracle/q8_oracle.mjs).  Inputs are the
// reference tests' own generators and shapes: ops/matmul/q8.wgsl.test.ts:25-56,
// ops/matmul/q8-edges.wgsl.test.ts, ops/dequant_transpose/wgsl.test.ts:10-48,
// llm/weights-q8.test.ts:45-113.
import { test, gpuTest, assert, kat, assertBitsEqual } from "./harness.mjs";
import { matmulQ8 } from "../../web-xpu-ops_amd/ops/matmul/index.js";
import { dequantTranspose } from "../../web-xpu-ops_amd/ops/dequant_transpose/index.js";
import { dequantizePackedQ8, gatherDequantRows, packInt8Rows } from "../../web-xpu-ops_amd/llm/weights-q8.js";
import { createResidentQ8Device } from "../../web-xpu-ops_amd/harness/resident.js";
import { native } from "../../web-xpu-ops_amd/native/index.js";
import * as oracle from "../../oracle/q8_oracle.mjs";

const F = "prefill.test.mjs";
const TILE = 16;
const wave = (n, k, phase = 0) => Float32Array.from({ length: n }, (_, i) => Math.sin(i * k + phase) * 1.5);
const codeWave = (n, k, phase = 0) => Int32Array.from({ length: n }, (_, i) => Math.round(Math.sin(i * k + phase) * 100));
const scaleWave = (n) => Float32Array.from({ length: n }, (_, i) => 0.02 * (i + 1) + 0.007);

/** |y - y_ref| <= 1e-5 * sum_k |a * fround(q * s)| + 1e-7 per element (NaN == NaN, equal infinities). */
function assertMatmulAgrees(got, { a, weight, scale, N, M, K }, what) {
  const want = oracle.matmulQ8({ a, weight, scale, N, M, K });
  const b = oracle.dequantTranspose({ weight, scale, outFeatures: M, inFeatures: K });  // [K, M]
  assert.strictEqual(got.length, want.length, `${what}: length`);
  for (let n = 0; n < N; n += 1) {
    for (let m = 0; m < M; m += 1) {
      const i = n * M + m;
      if (Number.isNaN(want[i]) && Number.isNaN(got[i])) continue;
      if (got[i] === want[i]) continue;
      let bound = 0;
      for (let k = 0; k < K; k += 1) bound += Math.abs(a[n * K + k] * b[k * M + m]);
      const err = Math.abs(got[i] - want[i]);
      if (!(err <= 1e-5 * bound + 1e-7)) assert.fail(`${what}: [${n}, ${m}] got ${got[i]} want ${want[i]} |err| ${err}`);
    }
  }
}

// ------------------------------------------------------------------ no GPU needed

test(F, "exports the reference's prefill-side op names", () => {
  assert.strictEqual(typeof matmulQ8, "function");
  assert.strictEqual(typeof dequantTranspose, "function");
  assert.strictEqual(typeof dequantizePackedQ8, "function");
  assert.strictEqual(typeof gatherDequantRows, "function");
  const a = native();
  for (const name of ["matmulQ8", "dequantizePackedQ8", "dequantTranspose", "gatherDequantRows", "matmulQ8Device",
    "dequantizePackedQ8Device", "dequantTransposeDevice", "gatherDequantRowsDevice"]) {
    assert.strictEqual(typeof a[name], "function", name);
  }
});

test(F, "arguments are checked before the device is touched", () => {
  const w = new Uint32Array(2), s = new Float32Array(2), x = new Float32Array(8);
  assert.throws(() => matmulQ8({ a: new Float64Array(8), weight: w, scale: s, N: 2, M: 2, K: 4 }), TypeError);
  assert.throws(() => matmulQ8({ a: new Float32Array(7), weight: w, scale: s, N: 2, M: 2, K: 4 }), RangeError);
  assert.throws(() => matmulQ8({ a: x, weight: new Uint32Array(1), scale: s, N: 2, M: 2, K: 4 }), RangeError);
  assert.throws(() => dequantizePackedQ8(new Int32Array(2), s, 2, 4), TypeError);
  assert.throws(() => gatherDequantRows({ codes: new Int8Array(8), scale: s }, [0, 1.5], 4), TypeError);
  assert.throws(() => gatherDequantRows({ codes: new Int8Array(7), scale: s }, [0], 4), RangeError);
  // the reference's own size errors (ops/dequant_transpose/wgsl.test.ts:41-48)
  const c = kat.dequant_transpose[1];
  const weight = new Uint32Array(6);
  assert.throws(() => dequantTranspose({ weight, scale: new Float32Array(3), outFeatures: 4, inFeatures: 5 }),
    new RegExp(c.errors[0]));
  assert.throws(() => dequantTranspose({ weight, scale: new Float32Array(2), outFeatures: 3, inFeatures: 5 }),
    new RegExp(c.errors[1]));
});

// ------------------------------------------------------------------ GPU

gpuTest(F, "matmulQ8 agrees with the reference at the WGSL test's shapes (q8.wgsl.test.ts:43-56)", () => {
  for (const [N, M, K] of kat.matmul_q8[0].shapes) {
    const a = wave(N * K, 0.37);
    const weight = oracle.packQ8({ codes: codeWave(M * K, 0.19), N: M, K });
    const scale = scaleWave(M);
    assertMatmulAgrees(matmulQ8({ a, weight, scale, N, M, K }), { a, weight, scale, N, M, K }, `${N}x${M}x${K}`);
  }
});

gpuTest(F, "matmulQ8 edge cases (q8-edges.wgsl.test.ts): ragged K with sentinels, M = TILE + 1, own scales", () => {
  {
    const N = 5, M = 7, K = 19;
    const a = wave(N * K, 0.41);
    const packedRows = oracle.packQ8({ codes: codeWave(M * K, 0.23), N: M, K });
    const W = Math.ceil(K / 4);
    const weight = Uint32Array.from({ length: M * W + 64 }, (_, i) => (i < M * W ? packedRows[i] : 0x7f7f7f7f));
    const scale = scaleWave(M);
    assertMatmulAgrees(matmulQ8({ a, weight, scale, N, M, K }), { a, weight: packedRows, scale, N, M, K }, "sentinel");
  }
  {
    const N = 4, M = TILE + 1, K = 8;
    const a = wave(N * K, 0.9);
    const weight = oracle.packQ8({ codes: codeWave(M * K, 0.31), N: M, K });
    const scale = scaleWave(M);
    assertMatmulAgrees(matmulQ8({ a, weight, scale, N, M, K }), { a, weight, scale, N, M, K }, "M tail");
  }
  {
    const N = 2, M = 2, K = 12;
    const shared = codeWave(K, 0.27);
    const weight = oracle.packQ8({ codes: Int32Array.from({ length: M * K }, (_, i) => shared[i % K]), N: M, K });
    const a = wave(N * K, 0.5);
    const scale = Float32Array.from([0.03, 0.11]);
    const y = matmulQ8({ a, weight, scale, N, M, K });
    assertMatmulAgrees(y, { a, weight, scale, N, M, K }, "own scales");
    assert.notStrictEqual(y[0], y[1]);
  }
});

gpuTest(F, "dequantizePackedQ8 and gatherDequantRows KATs (llm/weights-q8.test.ts:45-113), bit-exact", () => {
  {
    const N = 4, K = 9;
    const codes = Int8Array.from({ length: N * K }, (_, i) => (i === 0 ? -128 : ((i * 37) % 255) - 127));
    const scale = Float32Array.from({ length: N }, (_, r) => 0.01 * (r + 1) + 0.003);
    const packed = packInt8Rows(codes, N, K);
    const want = new Float32Array(N * K);
    for (let row = 0; row < N; row += 1) for (let col = 0; col < K; col += 1) want[row * K + col] = codes[row * K + col] * scale[row];
    assertBitsEqual(dequantizePackedQ8(packed, scale, N, K), want, "round trip");
  }
  const c = kat.dequantize_packed_q8[1];
  const packed = packInt8Rows(Int8Array.from(c.codes), c.N, c.K);
  assert.deepStrictEqual(Array.from(dequantizePackedQ8(packed, Float32Array.from(c.scale), c.N, c.K)), c.want);
  for (const g of kat.gather_dequant_rows) {
    const table = { codes: Int8Array.from(g.codes), scale: Float32Array.from(g.scale) };
    assert.deepStrictEqual(Array.from(gatherDequantRows(table, g.indices, g.D)), g.want, g.source);
    assert.deepStrictEqual(Array.from(gatherDequantRows(table, Int32Array.from(g.indices), g.D)), g.want, g.source);
  }
});

gpuTest(F, "dequantTranspose agrees exactly at the WGSL test's shapes (ops/dequant_transpose/wgsl.test.ts:10-38)", () => {
  for (const [outFeatures, inFeatures] of kat.dequant_transpose[0].shapes) {
    const codes = Int8Array.from({ length: outFeatures * inFeatures }, (_, i) => ((i * 37) % 200) - 100);
    const scale = Float32Array.from({ length: outFeatures }, (_, i) => 0.01 + i * 1e-4);
    const weight = packInt8Rows(codes, outFeatures, inFeatures);
    assertBitsEqual(dequantTranspose({ weight, scale, outFeatures, inFeatures }),
      oracle.dequantTranspose({ weight, scale, outFeatures, inFeatures }), `${outFeatures}x${inFeatures}`);
  }
});

gpuTest(F, "resident batch: gather the prompt's rows, then matmulQ8 on resident weights, one sync", async () => {
  const dev = await createResidentQ8Device();
  try {
    const rows = 50, D = 40, M = 33, T = 6;
    const codes = Int8Array.from({ length: rows * D }, (_, i) => ((i * 29) % 251) - 125);
    const tscale = Float32Array.from({ length: rows }, (_, i) => 0.001 * (i + 1));
    const ids = [3, 49, 0, 3, 17, 60];  // 60 is out of range: a zero row
    const wcodes = codeWave(M * D, 0.13);
    const weight = oracle.packQ8({ codes: wcodes, N: M, K: D });
    const scale = scaleWave(M);
    const bCodes = dev.createStorageBuffer(codes.byteLength);
    const bTs = dev.createStorageBuffer(tscale.byteLength);
    const bIdx = dev.createStorageBuffer(T * 8);
    const bHidden = dev.createStorageBuffer(T * D * 4);
    const bW = dev.createStorageBuffer(weight.byteLength);
    const bS = dev.createStorageBuffer(scale.byteLength);
    const bOut = dev.createStorageBuffer(T * M * 4);
    dev.upload(bCodes, 0, codes);
    dev.upload(bTs, 0, tscale);
    dev.upload(bIdx, 0, BigInt64Array.from(ids.map((v) => BigInt(v))));
    dev.upload(bW, 0, weight);
    dev.upload(bS, 0, scale);
    const created = dev.stats.buffersCreated;
    const [hidden, out] = await dev.batch([
      { kind: "gatherDequantRows", codes: bCodes, scale: bTs, rows, D, indices: bIdx, count: T, output: bHidden },
      { kind: "matmulQ8", a: bHidden, weight: bW, scale: bS, output: bOut, N: T, M, K: D },
    ], [{ source: bHidden, sourceOffset: 0, length: T * D, type: "f32" },
      { source: bOut, sourceOffset: 0, length: T * M, type: "f32" }]);
    assert.strictEqual(dev.stats.buffersCreated, created);
    const wantHidden = oracle.gatherDequantRows({ codes, scale: tscale }, ids, D);
    assertBitsEqual(hidden, wantHidden, "gathered rows");
    assertMatmulAgrees(out, { a: wantHidden, weight, scale, N: T, M, K: D }, "matmulQ8 after gather");
  } finally {
    dev.destroy();
  }
});
