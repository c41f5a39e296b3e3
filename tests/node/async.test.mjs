// The resident batch as an asynchronous submit: the wait for the GPU runs off
// the JS thread (the reference's batch awaits queue.onSubmittedWorkDone and
// mapAsync, harness/resident.ts:321-345), batches called while others are in
// flight run after them in call order, and each reads back its own values
// through page-locked staging memory.  The non-resident runMatVecQ8
// (llm/kernels.ts:195-211, over harness/wgsl.ts:35-36 Runner.run) likewise
// returns at once and does its work on a worker thread.
import { gpuTest, assert, assertBitsEqual } from "./harness.mjs";
import { createResidentQ8Device, BufferUsage } from "../../web-xpu-ops_amd/harness/resident.js";
import { packInt8Rows } from "../../web-xpu-ops_amd/llm/weights-q8.js";
import { runMatVecQ8 } from "../../web-xpu-ops_amd/llm/kernels.js";
import * as matvec from "../../web-xpu-ops_amd/ops/matvec/index.js";
import { native } from "../../web-xpu-ops_amd/native/index.js";

const F = "async.test.mjs";

function rng(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296;
  };
}

function vec(n, seed) {
  const r = rng(seed);
  return Float32Array.from({ length: n }, () => Math.fround(2 * r() - 1));
}

function nowMs() {
  const [s, ns] = process.hrtime();
  return s * 1e3 + ns / 1e6;
}

function storage(device, data) {
  const b = device.createStorageBuffer(data.byteLength);
  device.upload(b, 0, data);
  return b;
}

gpuTest(F, "batch(): returns before the GPU is done and the event loop runs while it waits", async () => {
  const device = await createResidentQ8Device();
  const n = 4096;
  const src = storage(device, vec(n, 1));
  const dst = device.createStorageBuffer(n * 4);
  const staging = device.createStorageBuffer(n * 4, BufferUsage.MAP_READ | BufferUsage.COPY_DST);
  device.addon.spin(40000);  // 40 ms of GPU work ahead of the batch
  const t0 = nowMs();
  const pending = device.batch([{ kind: "copy", src, srcOffset: 0, dst, dstOffset: 0, size: n * 4 }],
    [{ staging, source: dst, sourceOffset: 0, length: n, type: "f32" }]);
  const issued = nowMs() - t0;
  let ticks = 0;
  const timer = setInterval(() => { ticks += 1; }, 2);
  const [got] = await pending;
  clearInterval(timer);
  const total = nowMs() - t0;
  assert.ok(issued < 20, `batch() took ${issued.toFixed(1)} ms to return its promise`);
  assert.ok(total >= 30, `the batch settled after ${total.toFixed(1)} ms, before the 40 ms of work ahead of it`);
  assert.ok(ticks >= 3, `the event loop ran ${ticks} timer ticks while the batch waited`);
  assertBitsEqual(got, vec(n, 1), "copied values");
  device.destroy();
});

gpuTest(F, "batches in flight run in call order, each reads back its own values; a staging buffer still being read into is refused", async () => {
  const device = await createResidentQ8Device();
  const n = 1000;
  const a = storage(device, vec(n, 11)), b = storage(device, vec(n, 12));
  const y = device.createStorageBuffer(n * 4);
  const sa = device.createStorageBuffer(n * 4, BufferUsage.MAP_READ | BufferUsage.COPY_DST);
  const sb = device.createStorageBuffer(n * 4, BufferUsage.MAP_READ | BufferUsage.COPY_DST);
  const copy = (src) => ({ kind: "copy", src, srcOffset: 0, dst: y, dstOffset: 0, size: n * 4 });
  const read = (staging) => ({ staging, source: y, sourceOffset: 0, length: n, type: "f32" });
  device.addon.spin(20000);
  const p1 = device.batch([copy(a)], [read(sa)]);
  const p2 = device.batch([copy(b)], [read(sb)]);
  const p3 = device.batch([], [read(undefined)]);  // pooled staging
  await assert.rejects(device.batch([], [read(sa)]), /pending map/);
  const [[r1], [r2], [r3]] = await Promise.all([p1, p2, p3]);
  assertBitsEqual(r1, vec(n, 11), "first batch");
  assertBitsEqual(r2, vec(n, 12), "second batch");
  assertBitsEqual(r3, vec(n, 12), "readback-only batch");
  const [again] = await device.batch([], [read(sa)]);  // free again once its batch settled
  assertBitsEqual(again, vec(n, 12), "staging reused");
  device.destroy();
});

gpuTest(F, "replayed graphs in flight back to back: the same bits as batches awaited one by one", async () => {
  // Each step adds two projections of x into the residual stream in place,
  // so every step's readback differs from the last; a readback that ran
  // before its step's graph would show the previous step's values.
  const N = 2048, K = 2048, steps = 6;
  const r = rng(5);
  const codes = Int8Array.from({ length: N * K }, () => Math.floor(r() * 256) - 128);
  const scale = Float32Array.from({ length: N }, () => Math.fround(0.001 * (0.5 + r())));
  const packed = packInt8Rows(codes, N, K);
  const run = async (pipelined) => {
    const device = await createResidentQ8Device();
    const w = storage(device, packed), s = storage(device, scale), x = storage(device, vec(K, 6));
    const h = storage(device, vec(N, 7));
    const ops = [
      { kind: "matvecQ8Residual", weight: w, scale: s, vector: x, residual: h, output: h, N, K },
      { kind: "matvecQ8Residual", weight: w, scale: s, vector: x, residual: h, output: h, N, K },
    ];
    const rb = [{ source: h, sourceOffset: 0, length: N, type: "f32" }];
    let out;
    if (pipelined) {
      const first = [await device.batch(ops, rb)];   // op by op
      device.addon.spin(20000);
      const rest = [];
      for (let k = 1; k < steps; k += 1) rest.push(device.batch(ops, rb));  // captured once, then replayed, none awaited
      out = first.concat(await Promise.all(rest));
    } else {
      out = [];
      for (let k = 0; k < steps; k += 1) out.push(await device.batch(ops, rb));
    }
    const stats = { ...device.stats };
    device.destroy();
    return { out: out.map((o) => o[0]), stats };
  };
  const serial = await run(false);
  const piped = await run(true);
  assert.strictEqual(piped.stats.graphsCaptured, 1);
  assert.strictEqual(piped.stats.graphLaunches, steps - 1);
  for (let k = 0; k < steps; k += 1) {
    assertBitsEqual(piped.out[k], serial.out[k], `step ${k}`);
    if (k > 0) assert.notDeepStrictEqual(Array.from(serial.out[k]), Array.from(serial.out[k - 1]), `step ${k} changed the stream`);
  }
});

gpuTest(F, "wait: \"block\" waits on the JS thread (the promise is settled on return) with the same results", async () => {
  const n = 2048;
  const out = [];
  for (const wait of ["async", "block"]) {
    const device = await createResidentQ8Device({ wait });
    const src = storage(device, vec(n, 21));
    const dst = device.createStorageBuffer(n * 4);
    device.addon.spin(20000);
    const t0 = nowMs();
    let settled = false;
    const p = device.batch([{ kind: "copy", src, srcOffset: 0, dst, dstOffset: 0, size: n * 4 }],
      [{ source: dst, sourceOffset: 0, length: n, type: "f32" }]).then((r) => { settled = true; return r; });
    const issued = nowMs() - t0;
    await null;  // one microtask turn: a settled promise's reaction has run
    await null;
    if (wait === "block") assert.ok(issued >= 15 && settled, `block: returned after ${issued.toFixed(1)} ms, settled ${settled}`);
    else assert.ok(issued < 15 && !settled, `async: returned after ${issued.toFixed(1)} ms, settled ${settled}`);
    out.push((await p)[0]);
    device.destroy();
  }
  assertBitsEqual(out[1], out[0], "block vs async");
  assertBitsEqual(out[0], vec(n, 21), "values");
});

gpuTest(F, "a batch that waits to capture a graph holds back the batches called after it (call order kept)", async () => {
  const N = 1024, K = 1024;
  const r = rng(31);
  const codes = Int8Array.from({ length: N * K }, () => Math.floor(r() * 256) - 128);
  const scale = Float32Array.from({ length: N }, () => Math.fround(0.001 * (0.5 + r())));
  const packed = packInt8Rows(codes, N, K);
  const run = async (awaitEach) => {
    const device = await createResidentQ8Device();
    const w = storage(device, packed), s = storage(device, scale), x = storage(device, vec(K, 32));
    const h = storage(device, vec(N, 33)), c = storage(device, vec(N, 34));
    const twice = [
      { kind: "matvecQ8Residual", weight: w, scale: s, vector: x, residual: h, output: h, N, K },
      { kind: "matvecQ8Residual", weight: w, scale: s, vector: x, residual: h, output: h, N, K },
    ];
    const reset = [{ kind: "copy", src: c, srcOffset: 0, dst: h, dstOffset: 0, size: N * 4 }];
    const rb = [{ source: h, sourceOffset: 0, length: N, type: "f32" }];
    const lists = [twice, twice, reset, twice];  // the second captures a graph, the fourth replays it
    let out;
    if (awaitEach) {
      out = [];
      for (const l of lists) out.push(await device.batch(l, rb));
    } else {
      device.addon.spin(20000);
      out = await Promise.all(lists.map((l) => device.batch(l, rb)));
    }
    const stats = { ...device.stats };
    device.destroy();
    return { out: out.map((o) => o[0]), stats };
  };
  const serial = await run(true);
  const piped = await run(false);
  assert.strictEqual(piped.stats.graphsCaptured, 1);
  assert.strictEqual(piped.stats.graphLaunches, 2);
  assertBitsEqual(serial.out[2], vec(N, 34), "the reset batch's readback");
  for (let k = 0; k < 4; k += 1) assertBitsEqual(piped.out[k], serial.out[k], `batch ${k}`);
});

gpuTest(F, "runMatVecQ8: returns before the work is done, the vector is taken at the call, the same bits as matvecQ8", async () => {
  const N = 4096, K = 4096;  // the weight crosses PCIe inside the call
  const r = rng(41);
  const codes = Int8Array.from({ length: N * K }, () => Math.floor(r() * 255) - 127);
  const weight = packInt8Rows(codes, N, K);
  const scale = Float32Array.from({ length: N }, () => Math.fround(0.001 * (0.5 + r())));
  const x = vec(K, 42);
  const want = matvec.matvecQ8({ weight, scale, vector: x, N, K });
  const vector = Float32Array.from(x);
  const addon = native();
  addon.init();
  addon.spin(40000);  // 40 ms of GPU work ahead of the call's copies
  const t0 = nowMs();
  const pending = runMatVecQ8(null, { weight, scale, vector, M: N, K });
  const issued = nowMs() - t0;
  vector.fill(0);  // after the call: must not change its result
  let ticks = 0;
  const timer = setInterval(() => { ticks += 1; }, 2);
  const got = await pending;
  clearInterval(timer);
  const total = nowMs() - t0;
  assert.ok(issued < 20, `runMatVecQ8 took ${issued.toFixed(1)} ms to return its promise`);
  assert.ok(total >= 30, `it settled after ${total.toFixed(1)} ms, before the 40 ms of work ahead of it`);
  assert.ok(ticks >= 3, `the event loop ran ${ticks} timer ticks while the call waited`);
  assertBitsEqual(got, want, "runMatVecQ8 against matvecQ8");
  // several in flight at once, each with its own vector
  const xs = [1, 2, 3, 4].map((k) => vec(K, 50 + k));
  const outs = await Promise.all(xs.map((v) => runMatVecQ8(null, { weight, scale, vector: v, M: N, K })));
  xs.forEach((v, k) => assertBitsEqual(outs[k], matvec.matvecQ8({ weight, scale, vector: v, N, K }), `call ${k} in flight`));
});

gpuTest(F, "BatchProfile times (harness/timing.test.ts:56-120): positive, more for more work, inside the batch's wall time", async () => {
  // A labelled batch is held on the GPU until all of it is enqueued, so a
  // short op's interval is its GPU time, not the host's issue time.
  const device = await createResidentQ8Device();
  const K = 4096, W = K / 4;
  const mk = (N) => ({ weight: device.createStorageBuffer(N * W * 4), scale: device.createStorageBuffer(N * 4),
    output: device.createStorageBuffer(N * 4), N });
  const small = mk(2048), big = mk(65536);  // 8 MB and 268 MB of weights
  const x = device.createStorageBuffer(K * 4);
  const op = (p) => ({ kind: "matvecQ8", weight: p.weight, scale: p.scale, vector: x, output: p.output, N: p.N, K });
  for (let rep = 0; rep < 3; rep += 1) {
    const sink = { submitToDoneMs: null, readbackMs: null, gpuEntries: [] };
    const t0 = nowMs();
    await device.batch([op(small), op(big)], [], { labels: ["small", "big"], sink });
    const wallMs = nowMs() - t0;
    const [s, b] = sink.gpuEntries;
    assert.deepStrictEqual(sink.gpuEntries.map((e) => e.label), ["small", "big"]);
    assert.ok(s.seconds > 0 && b.seconds > 0, `positive: ${s.seconds} ${b.seconds}`);
    assert.ok(b.seconds > 4 * s.seconds, `32x the bytes: ${b.seconds} s against ${s.seconds} s`);
    assert.ok((s.seconds + b.seconds) * 1e3 < wallMs, `GPU ${(s.seconds + b.seconds) * 1e3} ms within the wall ${wallMs} ms`);
    // a physically possible rate (harness/roofline.test.ts's < 20 TB/s)
    assert.ok(65536 * W * 4 / b.seconds < 20e12, `big: ${65536 * W * 4 / b.seconds / 1e12} TB/s`);
  }
  device.destroy();
});

gpuTest(F, "matvecQ8Async with several vectors equals the synchronous call; the gate is refused inside a capture", async () => {
  const addon = native();
  addon.init();
  const N = 3000, K = 1500, M = 6;
  const r = rng(61);
  const codes = Int8Array.from({ length: N * K }, () => Math.floor(r() * 256) - 128);
  const weight = packInt8Rows(codes, N, K);
  const scale = Float32Array.from({ length: N }, () => Math.fround(0.001 * (0.5 + r())));
  const xs = vec(M * K, 62);
  const want = addon.matvecQ8(weight, scale, xs, N, K, M);
  const got = await addon.matvecQ8Async(weight, scale, xs, N, K, M);
  assertBitsEqual(got, want, "M = 6");
  assert.throws(() => addon.matvecQ8Async(weight, scale, xs.subarray(1), N, K, M), RangeError);  // checked at the call
  addon.graphBegin();
  try {
    addon.spin(1);  // something to capture
    assert.throws(() => addon.gateHold(1000), /capture is open/);
  } finally {
    addon.graphDestroy(addon.graphEnd());
  }
  const g = addon.gateHold(100000);
  addon.gateRelease(g);
  addon.synchronize();
});
