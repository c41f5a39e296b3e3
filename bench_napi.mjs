// End-to-end timing through the Node-API addon (launch + synchronisation as a
// JavaScript caller sees them), beside the kernel-only figures bench.py takes
// with HIP events:
//   - one resident matvecQ8 per batch at N=11008, K=4096 (one launch, one
//     stream synchronisation per call), weights rotated over 12 device copies
//     so HBM, not the 256 MB last-level cache, serves them;
//   - the same batches issued without awaiting each one (in flight together);
//   - the same with the 44 KB output read back each call;
//   - the host convenience call matvecQ8({weight, scale, vector, N, K})
//     (ops/matvec/reference.ts:117), which copies the 45 MB weight in over
//     PCIe every call (the PCIe-inclusive rate), and the same call through
//     runMatVecQ8 (llm/kernels.ts:195), which does it on a worker thread: the
//     JS thread's share of one call, and calls awaited one by one;
//   - one decode step of 22 layers shaped like BASELINE cfg4 (hidden 2048,
//     FFN 5632) as the resident engine issues it (llm/engine-q8-resident.ts:
//     1843-1869): per layer wq/wk/wv on one vector, matvecQ8Residual for wo,
//     matvecQ8Ffn, matvecQ8Residual for down, with one synchronisation per step.
// Prints one JSON line: {"node": ..., "results": [...]}.
//
//   node bench_napi.mjs [calls]
import { createResidentQ8Device } from "./web-xpu-ops_amd/harness/resident.js";
import { matvecQ8 } from "./web-xpu-ops_amd/ops/matvec/index.js";
import { runMatVecQ8 } from "./web-xpu-ops_amd/llm/kernels.js";

const N = 11008, K = 4096, W = Math.ceil(K / 4), COPIES = 12;

function nowUs() {
  return Number(process.hrtime.bigint()) / 1e3;
}

function randomWords(n, seed) {
  const out = new Uint32Array(n);
  let s = seed >>> 0 || 1;
  for (let i = 0; i < n; i += 1) {
    s ^= s << 13; s >>>= 0;
    s ^= s >>> 17;
    s ^= s << 5; s >>>= 0;
    out[i] = s;
  }
  return out;
}

async function main() {
  const calls = Number(process.argv[2] || 400);
  const dev = await createResidentQ8Device();
  if (dev === null) throw new Error("no gfx950 device visible");
  const results = [];
  const words = randomWords(N * W, 7);
  const scale = new Float32Array(N).fill(0.01);
  const vector = new Float32Array(K);
  for (let k = 0; k < K; k += 1) vector[k] = Math.sin(0.37 * k);

  const weights = [];
  for (let c = 0; c < COPIES; c += 1) {
    const b = dev.createStorageBuffer(N * W * 4);
    dev.upload(b, 0, words);
    weights.push(b);
  }
  const sbuf = dev.createStorageBuffer(N * 4);
  dev.upload(sbuf, 0, scale);
  const xbuf = dev.createStorageBuffer(K * 4);
  dev.upload(xbuf, 0, vector);
  const ybuf = dev.createStorageBuffer(N * 4);
  const op = (i) => ({ kind: "matvecQ8", weight: weights[i % COPIES], scale: sbuf, vector: xbuf, output: ybuf, N, K });
  const readback = [{ source: ybuf, sourceOffset: 0, length: N, type: "f32" }];

  const timeLoop = async (n, body) => {
    for (let i = 0; i < Math.min(50, n); i += 1) await body(i);
    const t0 = nowUs();
    for (let i = 0; i < n; i += 1) await body(i);
    return (nowUs() - t0) / n;
  };
  const bytes = N * W * 4 + 4 * N + 4 * K + 4 * N;

  let us = await timeLoop(calls, (i) => dev.batch([op(i)]));
  results.push({ case: "N-API end to end: resident matvecQ8, one launch + one synchronisation per call, N=11008 K=4096",
                 us: +us.toFixed(3), "GB/s": +(bytes / us / 1e3).toFixed(1) });
  // the same batches issued without awaiting each: the host enqueues call
  // i + 1 while the GPU runs call i, and one await covers them all
  {
    for (let i = 0; i < 50; i += 1) await dev.batch([op(i)]);
    const t0 = nowUs();
    const pending = [];
    for (let i = 0; i < calls; i += 1) pending.push(dev.batch([op(i)]));
    await Promise.all(pending);
    us = (nowUs() - t0) / calls;
  }
  results.push({ case: "N-API end to end: resident matvecQ8, batches in flight together (not awaited one by one), N=11008 K=4096",
                 us: +us.toFixed(3), "GB/s": +(bytes / us / 1e3).toFixed(1) });
  us = await timeLoop(calls, (i) => dev.batch([op(i)], readback));
  results.push({ case: "N-API end to end: resident matvecQ8 + 44 KB readback per call, N=11008 K=4096",
                 us: +us.toFixed(3), "GB/s": +(bytes / us / 1e3).toFixed(1) });

  const hostCalls = Math.max(5, Math.floor(calls / 20));
  us = await timeLoop(hostCalls, () => matvecQ8({ weight: words, scale, vector, N, K }));
  results.push({ case: "N-API end to end: host convenience matvecQ8 (weight copied in over PCIe each call), N=11008 K=4096",
                 us: +us.toFixed(1), "GB/s (PCIe-inclusive)": +(bytes / us / 1e3).toFixed(2) });
  us = await timeLoop(hostCalls, () => runMatVecQ8(null, { weight: words, scale, vector, M: N, K }));
  results.push({ case: "N-API end to end: runMatVecQ8 (the same call on a worker thread), awaited one by one, N=11008 K=4096",
                 us: +us.toFixed(1), "GB/s (PCIe-inclusive)": +(bytes / us / 1e3).toFixed(2) });
  {
    let held = 0;
    for (let i = 0; i < hostCalls; i += 1) {
      const t0 = nowUs();
      const p = runMatVecQ8(null, { weight: words, scale, vector, M: N, K });
      held += nowUs() - t0;
      await p;
    }
    results.push({ case: "N-API end to end: runMatVecQ8, the JS thread's share of one call (until its promise returns), N=11008 K=4096",
                   us: +(held / hostCalls).toFixed(1) });
  }

  // One decode step, 22 layers of BASELINE cfg4's shapes.
  const L = 22, H = 2048, F = 5632;
  const buf = (n) => dev.createStorageBuffer(n);
  const layers = [];
  for (let l = 0; l < L; l += 1) {
    const w = (n, k) => {
      const p = { weight: buf(n * Math.ceil(k / 4) * 4), scale: buf(n * 4) };
      dev.upload(p.scale, 0, new Float32Array(n).fill(0.01));
      return p;
    };
    layers.push({ q: w(H, H), k: w(H, H), v: w(H, H), o: w(H, H), g: w(F, H), u: w(F, H), d: w(H, F) });
  }
  const x = buf(H * 4), qo = buf(H * 4), ko = buf(H * 4), vo = buf(H * 4), resid = buf(H * 4), hid = buf(F * 4);
  dev.upload(x, 0, new Float32Array(H).fill(0.5));
  dev.upload(resid, 0, new Float32Array(H));
  const ops = [];
  for (const ly of layers) {
    ops.push({ kind: "matvecQ8", ...ly.q, vector: x, output: qo, N: H, K: H });
    ops.push({ kind: "matvecQ8", ...ly.k, vector: x, output: ko, N: H, K: H });
    ops.push({ kind: "matvecQ8", ...ly.v, vector: x, output: vo, N: H, K: H });
    ops.push({ kind: "matvecQ8Residual", ...ly.o, vector: qo, residual: resid, output: resid, N: H, K: H });
    ops.push({ kind: "matvecQ8Ffn", weightGate: ly.g.weight, scaleGate: ly.g.scale, weightUp: ly.u.weight,
               scaleUp: ly.u.scale, vector: x, output: hid, N: F, K: H });
    ops.push({ kind: "matvecQ8Residual", ...ly.d, vector: hid, residual: resid, output: resid, N: H, K: F });
  }
  const launches0 = dev.stats.launches;
  await dev.batch(ops);
  const launches = dev.stats.launches - launches0;
  const steps = Math.max(20, Math.floor(calls / 4));
  const layerBytes = 4 * (H * (H / 4) * 4) + 2 * (F * (H / 4) * 4) + H * (F / 4) * 4;
  // op by op (every launch issued each step), then as the device runs a
  // repeating step list by default: captured once, one graph launch per step
  for (const [graphs, wait] of [[false, "async"], [true, "async"], [true, "block"]]) {
    dev.graphs = graphs;
    dev.wait = wait;
    const g0 = dev.stats.graphLaunches;
    us = await timeLoop(steps, () => dev.batch(ops));
    const replayed = dev.stats.graphLaunches - g0;
    results.push({ case: `N-API end to end: one decode step, ${L} layers of cfg4 shapes as one resident batch ` +
                         `(${ops.length} ops, ${launches} launches, one synchronisation), ` +
                         (graphs ? "replayed as one captured graph" : "launched op by op") +
                         (wait === "block" ? ", waiting on the JS thread" : ""),
                   us: +us.toFixed(1), us_per_layer: +(us / L).toFixed(2),
                   "GB/s": +(L * layerBytes / us / 1e3).toFixed(1), graph_launches: replayed });
  }
  dev.destroy();
  console.log(JSON.stringify({ node: process.version, results }));
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : e);
  process.exit(1);
});
