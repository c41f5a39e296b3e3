// cpu_baseline_ops.mjs -- times the ECMAScript oracle's restatement of each op
// the suite measures (one core, V8), for bench.py's per-row CPU baselines.
//
// TEST INFRASTRUCTURE ONLY (a reported baseline, never the product).
//
//   node oracle/cpu_baseline_ops.mjs <op> <budget_seconds>
//
// Inputs are seeded synthetic arrays of the suite's shapes (the loops' cost
// does not depend on the values).  One untimed warm-up, then runs until the
// budget is spent; prints one JSON line with the median per call and the
// sample the time covers.
import {
  quantize, packQ8, packInt8Rows, matmulQ8, dequantizePackedQ8, dequantTranspose, gatherDequantRows,
  matvecQ8Ffn,
} from "./q8_oracle.mjs";

const [op, budgetS] = process.argv.slice(2);
const budget = Number(budgetS) * 1000;

let seed = 0x9e3779b9 >>> 0;
function rand() {  // xorshift32 in [0, 1)
  seed ^= seed << 13; seed >>>= 0;
  seed ^= seed >>> 17;
  seed ^= seed << 5; seed >>>= 0;
  return seed / 4294967296;
}
const normal = (n, sd) => Float32Array.from({ length: n }, () => (rand() + rand() + rand() - 1.5) * 2 * sd);
const codesI8 = (n) => Int8Array.from({ length: n }, () => Math.floor(rand() * 255) - 127);

let run, sample;
if (op === "quantize_pack") {
  const N = 2048, K = 2048;
  const w = normal(N * K, 0.02);
  run = () => { const q = quantize({ input: w, N, D: K }); return packQ8({ codes: q.output, N, K })[0] + q.scales[0]; };
  sample = { op: "quantize then packQ8 (ops/quantize/reference.ts:13, ops/matvec/reference.ts:267)", N, K };
} else if (op === "pack_int8_rows") {
  const N = 4096, K = 4099;
  const c = codesI8(N * K);
  run = () => packInt8Rows(c, N, K)[0];
  sample = { op: "packInt8Rows (llm/weights-q8.ts:137)", N, K };
} else if (op === "matmul") {
  const T = 8, M = 2048, K = 2048;  // 8 of the prompt's tokens; the reference's cost per token is the same for all
  const a = normal(T * K, 1);
  const weight = packInt8Rows(codesI8(M * K), M, K);
  const scale = normal(M, 0.001);
  run = () => matmulQ8({ a, weight, scale, N: T, M, K })[0];
  sample = { op: "matmulQ8 (ops/matmul/reference.ts:124): per-term dequant into b, then matmul", N: T, M, K };
} else if (op === "dequantize") {
  const N = 5632, K = 2048;
  const weight = packInt8Rows(codesI8(N * K), N, K);
  const scale = normal(N, 0.001);
  run = () => dequantizePackedQ8(weight, scale, N, K)[0];
  sample = { op: "dequantizePackedQ8 (llm/weights-q8.ts:161)", N, K };
} else if (op === "dequant_transpose") {
  const N = 5632, K = 2048;
  const weight = packInt8Rows(codesI8(N * K), N, K);
  const scale = normal(N, 0.001);
  run = () => dequantTranspose({ weight, scale, outFeatures: N, inFeatures: K })[0];
  sample = { op: "dequantTranspose (ops/dequant_transpose/reference.ts:40)", N, K };
} else if (op === "gather") {
  const rows = 32000, D = 2048, T = 512;
  const table = { codes: codesI8(rows * D), scale: normal(rows, 0.001) };
  const idx = Array.from({ length: T }, () => Math.floor(rand() * rows));
  run = () => gatherDequantRows(table, idx, D)[0];
  sample = { op: "gatherDequantRows (llm/weights-q8.ts:207)", rows, D, T };
} else if (op === "ffn") {
  const N = 5632, K = 2048;
  const wg = packInt8Rows(codesI8(N * K), N, K), wu = packInt8Rows(codesI8(N * K), N, K);
  const sg = normal(N, 0.001), su = normal(N, 0.001), v = normal(K, 1);
  run = () => matvecQ8Ffn({ weightGate: wg, scaleGate: sg, weightUp: wu, scaleUp: su, vector: v, N, K })[0];
  sample = { op: "matvecQ8Ffn (ops/matvec/reference.ts:196)", N, K };
} else {
  throw new Error(`unknown op ${op}`);
}

let sink = run();  // warm-up (JIT)
const times = [];
const t0 = process.hrtime.bigint();
while (times.length < 3 || (Number(process.hrtime.bigint() - t0) / 1e6 < budget && times.length < 1000)) {
  const a = process.hrtime.bigint();
  sink += run();
  times.push(Number(process.hrtime.bigint() - a) / 1e3);
}
times.sort((x, y) => x - y);
process.stdout.write(JSON.stringify(Object.assign({}, sample, {
  runs: times.length, median_us: times[Math.floor(times.length / 2)], min_us: times[0], node: process.version,
  checksum: sink,
})) + "\n");
