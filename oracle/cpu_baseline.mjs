// cpu_baseline.mjs -- times the ECMAScript oracle's matvecQ8 (one core, V8)
// on the inputs bench.py wrote, for bench.py's cpu_baseline leg.
//
// TEST INFRASTRUCTURE ONLY (a reported baseline, never the product).
//
//   node oracle/cpu_baseline.mjs <dir> <N> <K> <budget_seconds> [rows]
//
// <dir> holds weight.bin (u32 [N*ceil(K/4)]), scale.bin (f32 [N]) and
// vector.bin (f32 [K]), little-endian.  With [rows] < N, each run covers the
// first `rows` rows (a bounded sample of the same workload).  One untimed
// warm-up, then runs until the budget is spent; prints one JSON line.
import { readFileSync } from "fs";
import { join } from "path";
import { matvecQ8 } from "./q8_oracle.mjs";

const [dir, Ns, Ks, budgetS, rowsS] = process.argv.slice(2);
const N = Number(Ns);
const K = Number(Ks);
const budget = Number(budgetS) * 1000;
const rows = rowsS ? Math.min(Number(rowsS), N) : N;
const W = Math.ceil(K / 4);

const read = (name, T) => {
  const b = readFileSync(join(dir, name));
  const copy = new Uint8Array(b.length);
  copy.set(b);
  return new T(copy.buffer, 0, b.length / T.BYTES_PER_ELEMENT);
};
const weight = read("weight.bin", Uint32Array).subarray(0, rows * W);
const scale = read("scale.bin", Float32Array).subarray(0, rows);
const vector = read("vector.bin", Float32Array);

const args = { weight, scale, vector, N: rows, K };
let sink = matvecQ8(args)[0];  // warm-up (JIT)
const times = [];
const t0 = process.hrtime.bigint();
while (times.length < 3 || (Number(process.hrtime.bigint() - t0) / 1e6 < budget && times.length < 1000)) {
  const a = process.hrtime.bigint();
  sink += matvecQ8(args)[rows - 1];
  times.push(Number(process.hrtime.bigint() - a) / 1e3);
}
times.sort((x, y) => x - y);
const median = times[Math.floor(times.length / 2)];
process.stdout.write(JSON.stringify({
  rows, N, K, runs: times.length, median_us: median, min_us: times[0],
  node: process.version, checksum: sink,
}) + "\n");
