// The TypeScript op API of this package (web-xpu-ops_amd/ops, llm, harness)
// against the ECMAScript oracle (oracle/q8_oracle.mjs).  Input generators and
// shapes are the reference's own: ops/matvec/q8.wgsl.test.ts:23-71,
// ops/quantize/wgsl.test.ts:6-56, ops/matvec/reference.test.ts:14-95,
// llm/weights-q8.test.ts:17-42.
import { test, gpuTest, assert, kat, assertBitsEqual, assertMatvecAgrees, assertResidualAgrees, assertFfnAgrees }
  from "./harness.mjs";
import * as matvec from "../../web-xpu-ops_amd/ops/matvec/index.js";
import * as quantizeOps from "../../web-xpu-ops_amd/ops/quantize/index.js";
import { packInt8Rows } from "../../web-xpu-ops_amd/llm/weights-q8.js";
import { runMatVecQ8 } from "../../web-xpu-ops_amd/llm/kernels.js";
import { createResidentQ8Device } from "../../web-xpu-ops_amd/harness/resident.js";
import { native, describe } from "../../web-xpu-ops_amd/native/index.js";
import { roofline, measureRoofline, measureMatrixRoofline } from "../../web-xpu-ops_amd/harness/roofline.js";
import * as oracle from "../../oracle/q8_oracle.mjs";

const F = "api.test.mjs";

// ------------------------------------------------------------------ no GPU needed

test(F, "exports the reference's op names", () => {
  for (const name of ["matvecQ8", "packQ8", "matvecQ8Batched", "matvecQ8Ffn", "matvecQ8Residual"]) {
    assert.strictEqual(typeof matvec[name], "function", name);
  }
  for (const name of ["quantize", "quantizePackQ8"]) assert.strictEqual(typeof quantizeOps[name], "function", name);
  assert.strictEqual(typeof packInt8Rows, "function");
  assert.strictEqual(typeof runMatVecQ8, "function");
  assert.strictEqual(typeof roofline, "function");
  assert.strictEqual(typeof measureRoofline, "function");
  assert.strictEqual(typeof measureMatrixRoofline, "function");
});

test(F, "the addon loads and exports its whole surface", () => {
  const a = native();
  for (const name of ["abiVersion", "describe", "deviceCount", "init", "synchronize", "matvecQ8", "matvecQ8Ffn",
    "matvecQ8Residual", "quantize", "packQ8", "packInt8Rows", "quantizePackQ8", "malloc", "free", "upload", "download",
    "copy", "matvecQ8Device", "matvecQ8FfnDevice", "matvecQ8ResidualDevice", "quantizeDevice", "packQ8Device",
    "packInt8RowsDevice", "quantizePackQ8Device", "roofline", "rooflineMatrix", "matvecQ8Async", "whenDone", "hostAlloc",
    "downloadAsync"]) {
    assert.strictEqual(typeof a[name], "function", name);
  }
  assert.strictEqual(a.abiVersion(), 1);
  assert.ok(describe().startsWith("wxo_q8 abi=1"));
});

test(F, "argument types and lengths are checked before the device is touched", async () => {
  const w = new Uint32Array(2), s = new Float32Array(2), x = new Float32Array(4);
  assert.throws(() => matvec.matvecQ8({ weight: new Int32Array(2), scale: s, vector: x, N: 2, K: 4 }), TypeError);
  assert.throws(() => matvec.matvecQ8({ weight: w, scale: new Float64Array(2), vector: x, N: 2, K: 4 }), TypeError);
  assert.throws(() => matvec.matvecQ8({ weight: new Uint32Array(1), scale: s, vector: x, N: 2, K: 4 }), RangeError);
  assert.throws(() => matvec.matvecQ8({ weight: w, scale: s, vector: new Float32Array(3), N: 2, K: 4 }), RangeError);
  assert.throws(() => matvec.matvecQ8({ weight: w, scale: s, vector: x, N: -1, K: 4 }), TypeError);
  assert.throws(() => matvec.matvecQ8({ weight: w, scale: s, vector: x, N: 1.5, K: 4 }), TypeError);
  assert.throws(() => quantizeOps.quantize({ input: new Float32Array(5), N: 2, D: 3 }), RangeError);
  assert.throws(() => matvec.packQ8({ codes: new Uint8Array(4), N: 1, K: 4 }), TypeError);
  assert.throws(() => packInt8Rows(new Int32Array(4), 1, 4), TypeError);
  // the asynchronous form rejects with the same errors
  await assert.rejects(runMatVecQ8(null, { weight: new Uint32Array(1), scale: s, vector: x, M: 2, K: 4 }), RangeError);
  await assert.rejects(runMatVecQ8(null, { weight: w, scale: new Float64Array(2), vector: x, M: 2, K: 4 }), TypeError);
});

test(F, "without a gfx950 GPU every op fails loudly (no CPU fallback)", async () => {
  if (native().deviceCount() > 0) return;  // covered by the GPU suite there
  assert.throws(() => matvec.matvecQ8({ weight: new Uint32Array(2), scale: new Float32Array(2), vector: new Float32Array(4), N: 2, K: 4 }),
    (e) => e.status === 2 && /no ROCm|no HIP device|no CPU fallback/.test(e.message));
  assert.throws(() => quantizeOps.quantize({ input: new Float32Array(4), N: 1, D: 4 }), (e) => e.status === 2);
  await assert.rejects(runMatVecQ8(null, { weight: new Uint32Array(2), scale: new Float32Array(2), vector: new Float32Array(4), M: 2, K: 4 }),
    (e) => e.status === 2 && /no ROCm|no HIP device|no CPU fallback/.test(e.message));
});

// ------------------------------------------------------------------ GPU

const codeWave = (n, k, phase = 0) => Int32Array.from({ length: n }, (_, i) => Math.round(Math.sin(i * k + phase) * 100));
const wave = (n, k, phase = 0) => Float32Array.from({ length: n }, (_, i) => Math.sin(i * k + phase) * 1.5);
const scaleWave = (n) => Float32Array.from({ length: n }, (_, i) => 0.02 * (i + 1) + 0.007);

gpuTest(F, "matvecQ8 KATs (ops/matvec/reference.test.ts:56-95), object and positional forms", () => {
  for (const c of kat.matvec_q8) {
    const weight = oracle.packQ8({ codes: Int32Array.from(c.codes), N: c.N, K: c.K });
    if (c.pad_patch) weight[c.pad_patch.word] |= parseInt(c.pad_patch.or, 16);
    const scale = Float32Array.from(c.scale);
    const vector = Float32Array.from(c.vector).subarray(0, c.K);
    assert.deepStrictEqual(Array.from(matvec.matvecQ8({ weight, scale, vector, N: c.N, K: c.K })), c.want);
    assert.deepStrictEqual(Array.from(matvec.matvecQ8(vector, weight, scale, c.N, c.K)), c.want);
  }
});

gpuTest(F, "matvecQ8 agrees with the reference at the WGSL test's shapes (q8.wgsl.test.ts:48-71)", () => {
  for (const [N, K] of [[1, 3], [1, 8], [5, 1024], [3, 1030], [7, 1027], [2, 2600]]) {
    const codes = codeWave(N * K, 0.37);
    const weight = matvec.packQ8({ codes, N, K });
    assertBitsEqual(weight, oracle.packQ8({ codes, N, K }), `packQ8 N=${N} K=${K}`);
    const scale = scaleWave(N);
    const vector = wave(K, 0.11, 0.8);
    const args = { weight, scale, vector, N, K };
    assertMatvecAgrees(matvec.matvecQ8(args), oracle.matvecQ8(args), args, `N=${N} K=${K}`);
  }
});

gpuTest(F, "matvecQ8 ignores words and vector entries past the row (q8.wgsl.test.ts:108-149)", () => {
  const N = 4, K = 1023, W = Math.ceil(K / 4);
  const codes = Int32Array.from({ length: N * K }, (_, i) => (Math.floor(i / K) % 5) + 1);
  const packed = oracle.packQ8({ codes, N, K });
  const weight = Uint32Array.from({ length: N * W + 256 }, (_, i) => (i < N * W ? packed[i] : 0x7f7f7f7f));
  const vector = Float32Array.from({ length: K + 256 }, (_, i) => (i < K ? 1 : 1000));
  const scale = scaleWave(N);
  const want = oracle.matvecQ8({ weight: packed, scale, vector: vector.slice(0, K), N, K });
  assertMatvecAgrees(matvec.matvecQ8({ weight, scale, vector, N, K }), want, { weight: packed, scale, vector, N, K }, "sentinel");
});

gpuTest(F, "matvecQ8Batched is M independent matvecQ8 calls", () => {
  const N = 33, K = 1030, M = 5;
  const weight = matvec.packQ8({ codes: codeWave(N * K, 0.29), N, K });
  const scale = scaleWave(N);
  const vectors = Float32Array.from({ length: M * K }, (_, i) => Math.cos(i * 0.013) * 2);
  const ys = matvec.matvecQ8Batched({ weight, scale, vectors, N, K, M });
  for (let m = 0; m < M; m += 1) {
    const vector = vectors.subarray(m * K, (m + 1) * K);
    assertMatvecAgrees(ys.subarray(m * N, (m + 1) * N), oracle.matvecQ8({ weight, scale, vector, N, K }),
      { weight, scale, vector, N, K }, `m=${m}`);
  }
});

gpuTest(F, "quantize is bit-exact at the WGSL test's shapes, scales included (ops/quantize/wgsl.test.ts:11-33)", () => {
  const qwave = (n, k = 0.37) => Float32Array.from({ length: n }, (_, i) => Math.sin(i * k) * 2);
  for (const [N, D] of [[1, 64], [2, 300]]) {
    const input = qwave(N * D, 0.41);
    const got = quantizeOps.quantize({ input, N, D });
    const want = oracle.quantize({ input, N, D });
    assertBitsEqual(got.output, want.output, `codes N=${N} D=${D}`);
    assertBitsEqual(got.scales, want.scales, `scales N=${N} D=${D}`);
  }
  const zero = quantizeOps.quantize({ input: new Float32Array(16), N: 1, D: 16 });  // wgsl.test.ts:35-55
  assertBitsEqual(zero.output, new Int32Array(16), "all-zero codes");
  assert.strictEqual(zero.scales[0], 1);
});

gpuTest(F, "quantize KATs (llm/tools/quant_common.py:73-86 rows)", () => {
  for (const c of kat.quantize) {
    const input = Float32Array.from(c.input);
    const got = quantizeOps.quantize({ input, N: 1, D: input.length });
    assert.deepStrictEqual(Array.from(got.output), c.codes);
    assert.strictEqual(new Uint32Array(got.scales.buffer)[0], parseInt(c.scale_bits, 16));
  }
});

gpuTest(F, "packQ8 / packInt8Rows KATs and equivalence (reference.test.ts:14-53, weights-q8.test.ts:17-42)", () => {
  for (const c of kat.pack_q8) {
    const words = matvec.packQ8({ codes: Int32Array.from(c.codes), N: c.N, K: c.K });
    assert.deepStrictEqual(Array.from(words, (w) => "0x" + w.toString(16).padStart(8, "0")), c.words);
  }
  for (const c of kat.pack_int8_rows) {
    const a = packInt8Rows(Int8Array.from(c.codes), c.N, c.K);
    const b = matvec.packQ8({ codes: Int32Array.from(c.codes), N: c.N, K: c.K });
    assertBitsEqual(a, b, "packInt8Rows == packQ8");
    assertBitsEqual(a, oracle.packQ8({ codes: Int32Array.from(c.codes), N: c.N, K: c.K }), "vs oracle");
  }
});

gpuTest(F, "quantize + packQ8 compose as in the reference, and the fused form equals the composition", () => {
  const N = 96, K = 1027;
  const input = Float32Array.from({ length: N * K }, (_, i) => Math.sin(i * 0.7) * 0.02 * (1 + (i % 7)));
  const q = quantizeOps.quantize({ input, N, D: K });
  const composed = matvec.packQ8({ codes: q.output, N, K });
  const fused = quantizeOps.quantizePackQ8({ input, N, K });
  const want = oracle.quantize({ input, N, D: K });
  assertBitsEqual(composed, oracle.packQ8({ codes: want.output, N, K }), "composed");
  assertBitsEqual(fused.weight, composed, "fused weight");
  assertBitsEqual(fused.scale, want.scales, "fused scale");
  const vector = wave(K, 0.05);
  const args = { weight: fused.weight, scale: fused.scale, vector, N, K };
  assertMatvecAgrees(matvec.matvecQ8(args), oracle.matvecQ8(args), args, "pipeline");
});

gpuTest(F, "matvecQ8Ffn / matvecQ8Residual KATs (ops/matvec/reference.test.ts:112-193)", () => {
  for (const c of kat.matvec_q8_ffn) {
    const weightGate = oracle.packQ8({ codes: Int32Array.from(c.gate_codes), N: c.N, K: c.K });
    const weightUp = oracle.packQ8({ codes: Int32Array.from(c.up_codes), N: c.N, K: c.K });
    const got = matvec.matvecQ8Ffn({ weightGate, scaleGate: Float32Array.from(c.scale_gate), weightUp,
      scaleUp: Float32Array.from(c.scale_up), vector: Float32Array.from(c.vector), N: c.N, K: c.K });
    c.want.forEach((w, i) => assert.ok(Math.abs(got[i] - w) < c.abs_tol, `${c.source}: row ${i} ${got[i]} vs ${w}`));
  }
  for (const c of kat.matvec_q8_residual) {
    const weight = oracle.packQ8({ codes: Int32Array.from(c.codes), N: c.N, K: c.K });
    const got = matvec.matvecQ8Residual({ weight, scale: Float32Array.from(c.scale), vector: Float32Array.from(c.vector),
      residual: Float32Array.from(c.residual), N: c.N, K: c.K });
    c.want.forEach((w, i) => assert.ok(Math.abs(got[i] - w) < c.abs_tol, `${c.source}: row ${i} ${got[i]} vs ${w}`));
  }
});

gpuTest(F, "matvecQ8Ffn / matvecQ8Residual agree with the reference's composition at decode-layer shapes", () => {
  for (const [N, K] of [[5632, 2048], [7, 1027], [300, 5632]]) {
    const weightGate = matvec.packQ8({ codes: codeWave(N * K, 0.37), N, K });
    const weightUp = matvec.packQ8({ codes: codeWave(N * K, 0.53, 1.1), N, K });
    const scaleGate = scaleWave(N), scaleUp = Float32Array.from(scaleWave(N), (v) => v * 0.5);
    const vector = wave(K, 0.11, 0.8);
    const got = matvec.matvecQ8Ffn({ weightGate, scaleGate, weightUp, scaleUp, vector, N, K });
    const ag = { weight: weightGate, scale: scaleGate, vector, N, K };
    const au = { weight: weightUp, scale: scaleUp, vector, N, K };
    assertFfnAgrees(got, oracle.matvecQ8(ag), oracle.matvecQ8(au), oracle.silu, ag, au, `ffn N=${N} K=${K}`);
    const residual = wave(N, 0.29, 0.3);
    const res = matvec.matvecQ8Residual({ weight: weightGate, scale: scaleGate, vector, residual, N, K });
    assertResidualAgrees(res, oracle.matvecQ8Residual({ weight: weightGate, scale: scaleGate, vector, residual, N, K }),
      ag, `residual N=${N} K=${K}`);
  }
});

gpuTest(F, "runMatVecQ8 keeps llm/kernels.ts's signature (M = rows)", async () => {
  const N = 70000, K = 64;  // past WebGPU's 65,535-row dispatch limit, one call here
  const weight = matvec.packQ8({ codes: codeWave(N * K, 0.31), N, K });
  const scale = scaleWave(N);
  const vector = wave(K, 0.2);
  const got = await runMatVecQ8(null, { weight, scale, vector, M: N, K });
  const args = { weight, scale, vector, N, K };
  assertMatvecAgrees(got, oracle.matvecQ8(args), args, "runMatVecQ8");
});

gpuTest(F, "ResidentQ8Device: resident weights, one sync per batch, no allocation in the loop", async () => {
  const dev = await createResidentQ8Device();
  assert.ok(dev);
  const N = 512, K = 2048, W = K / 4;
  const input = Float32Array.from({ length: N * K }, (_, i) => Math.sin(i * 0.013) * 0.02);
  const wf = dev.createStorageBuffer(N * K * 4);
  const packed = dev.createStorageBuffer(N * W * 4);
  const scales = dev.createStorageBuffer(N * 4);
  const x = dev.createStorageBuffer(K * 4);
  const y = dev.createStorageBuffer(N * 4);
  const y2 = dev.createStorageBuffer(N * 4);
  dev.upload(wf, 0, input);
  await dev.batch([{ kind: "quantizePackQ8", input: wf, N, K, packed, scales }]);
  const created = dev.stats.buffersCreated;
  const want = oracle.quantize({ input, N, D: K });
  const wantPacked = oracle.packQ8({ codes: want.output, N, K });
  for (let step = 0; step < 3; step += 1) {
    const vector = wave(K, 0.07 * (step + 1));
    dev.upload(x, 0, vector);
    const [out, out2, words] = await dev.batch(
      [{ kind: "matvecQ8", weight: packed, scale: scales, vector: x, output: y, N, K },
       { kind: "copy", src: y, srcOffset: 0, dst: y2, dstOffset: 0, size: N * 4 }],
      [{ source: y, sourceOffset: 0, length: N, type: "f32" }, { source: y2, sourceOffset: 0, length: N, type: "f32" },
       { source: packed, sourceOffset: 0, length: N * W, type: "u32" }]);
    assertBitsEqual(words, wantPacked, "resident packed weight");
    const args = { weight: wantPacked, scale: want.scales, vector, N, K };
    assertMatvecAgrees(out, oracle.matvecQ8(args), args, `step ${step}`);
    assertBitsEqual(out2, out, "copy");
  }
  assert.strictEqual(dev.stats.buffersCreated, created);
  assert.strictEqual(dev.stats.submits, 4);
  dev.destroy();
});

gpuTest(F, "ResidentQ8Device: fused FFN and an in-place residual add in one batch", async () => {
  const dev = await createResidentQ8Device();
  const N = 1024, K = 2048, W = K / 4;
  const hw = (k, p) => matvec.packQ8({ codes: codeWave(N * K, k, p), N, K });
  const wg = hw(0.37, 0), wu = hw(0.41, 0.5), wo = hw(0.23, 1.0);
  const sg = scaleWave(N), su = scaleWave(N), so = scaleWave(N);
  const buf = (a) => { const b = dev.createStorageBuffer(a.byteLength); dev.upload(b, 0, a); return b; };
  const [bwg, bwu, bwo, bsg, bsu, bso] = [wg, wu, wo, sg, su, so].map(buf);
  const vector = wave(K, 0.09), resid0 = wave(N, 0.17);
  const bx = buf(vector), bres = buf(resid0), bh = dev.createStorageBuffer(N * 4);
  const [h, r] = await dev.batch(
    [{ kind: "matvecQ8Ffn", weightGate: bwg, scaleGate: bsg, weightUp: bwu, scaleUp: bsu, vector: bx, output: bh, N, K },
     { kind: "matvecQ8Residual", weight: bwo, scale: bso, vector: bx, residual: bres, output: bres, N, K }],
    [{ source: bh, sourceOffset: 0, length: N, type: "f32" }, { source: bres, sourceOffset: 0, length: N, type: "f32" }]);
  const ag = { weight: wg, scale: sg, vector, N, K }, au = { weight: wu, scale: su, vector, N, K };
  assertFfnAgrees(h, oracle.matvecQ8(ag), oracle.matvecQ8(au), oracle.silu, ag, au, "resident ffn");
  const ao = { weight: wo, scale: so, vector, N, K };
  assertResidualAgrees(r, oracle.matvecQ8Residual({ ...ao, residual: resid0 }), ao, "resident residual in place");
  assert.strictEqual(W * 4 * N, wg.byteLength);
  dev.destroy();
});

gpuTest(F, "ResidentQ8Device: same-vector matvecQ8 runs share one launch and give the separate ops' results", async () => {
  // The engine's decode order (llm/engine-q8-resident.ts:1843-1845): wq, wk, wv
  // on one vector, then ops that depend on earlier outputs.
  const K = 1030, W = Math.ceil(K / 4);
  const shapes = { q: 256, k: 64, v: 64 };
  const mats = {};
  let p = 0;
  for (const [name, N] of Object.entries(shapes)) {
    mats[name] = { N, weight: matvec.packQ8({ codes: codeWave(N * K, 0.29 + 0.05 * p, p), N, K }), scale: scaleWave(N) };
    p += 1;
  }
  const Nd = 100, Kd = shapes.q;  // reads q's output as its vector
  const wd = matvec.packQ8({ codes: codeWave(Nd * Kd, 0.43), N: Nd, K: Kd }), sd = scaleWave(Nd);
  const vector = wave(K, 0.11);
  for (const coalesce of [true, false]) {
    const dev = await createResidentQ8Device({ coalesce });
    const buf = (a) => { const b = dev.createStorageBuffer(a.byteLength); dev.upload(b, 0, a); return b; };
    const bx = buf(vector);
    const ops = [];
    const outs = {};
    for (const [name, m] of Object.entries(mats)) {
      outs[name] = dev.createStorageBuffer(m.N * 4);
      ops.push({ kind: "matvecQ8", weight: buf(m.weight), scale: buf(m.scale), vector: bx, output: outs[name], N: m.N, K });
    }
    const yd = dev.createStorageBuffer(Nd * 4);
    ops.push({ kind: "matvecQ8", weight: buf(wd), scale: buf(sd), vector: outs.q, output: yd, N: Nd, K: Kd });
    // two ops on the same vector writing one output: in order, the second wins
    const yk2 = dev.createStorageBuffer(shapes.k * 4);
    const kop = ops[1];
    ops.push({ ...kop, output: yk2 }, { ...ops[0], N: shapes.k, output: yk2 });
    const launches0 = dev.stats.launches;
    const [q, k, v, d, k2] = await dev.batch(ops, [outs.q, outs.k, outs.v, yd, yk2].map(
      (b) => ({ source: b, sourceOffset: 0, length: b.size / 4, type: "f32" })));
    const got = { q, k, v };
    for (const [name, m] of Object.entries(mats)) {
      const args = { weight: m.weight, scale: m.scale, vector, N: m.N, K };
      assertMatvecAgrees(got[name], oracle.matvecQ8(args), args, `${name} coalesce=${coalesce}`);
    }
    const dargs = { weight: wd, scale: sd, vector: q, N: Nd, K: Kd };
    assertMatvecAgrees(d, oracle.matvecQ8(dargs), dargs, `dependent op coalesce=${coalesce}`);
    const qargs = { weight: mats.q.weight, scale: mats.q.scale, vector, N: shapes.k, K };
    assertMatvecAgrees(k2, oracle.matvecQ8(qargs), qargs, `last writer coalesce=${coalesce}`);
    // q/k/v in one launch; the dependent op and the two same-output ops alone
    assert.strictEqual(dev.stats.launches - launches0, coalesce ? 4 : 6);
    dev.destroy();
  }
});

gpuTest(F, "ResidentQ8Device: consecutive quantizePackQ8 ops with one K share a launch, bit-exact per matrix", async () => {
  const K = 520, W = Math.ceil(K / 4);
  const Ns = [40, 3, 17];
  const inputs = Ns.map((N, m) => Float32Array.from({ length: N * K }, (_, i) => Math.sin(i * 0.013 + m) * 0.02));
  inputs[0].fill(0, K, 2 * K);  // an all-zero row: scale 1, codes 0
  for (const coalesce of [true, false]) {
    const dev = await createResidentQ8Device({ coalesce });
    const ops = [], outs = [];
    Ns.forEach((N, m) => {
      const input = dev.createStorageBuffer(N * K * 4);
      dev.upload(input, 0, inputs[m]);
      const packed = dev.createStorageBuffer(N * W * 4), scales = dev.createStorageBuffer(N * 4);
      ops.push({ kind: "quantizePackQ8", input, N, K, packed, scales });
      outs.push({ source: packed, sourceOffset: 0, length: N * W, type: "u32" },
                { source: scales, sourceOffset: 0, length: N, type: "f32" });
    });
    const launches0 = dev.stats.launches;
    const got = await dev.batch(ops, outs);
    Ns.forEach((N, m) => {
      const want = oracle.quantize({ input: inputs[m], N, D: K });
      assertBitsEqual(got[2 * m], oracle.packQ8({ codes: want.output, N, K }), `packed ${m} coalesce=${coalesce}`);
      assertBitsEqual(got[2 * m + 1], want.scales, `scales ${m} coalesce=${coalesce}`);
    });
    assert.strictEqual(dev.stats.launches - launches0, coalesce ? 1 : 3);
    dev.destroy();
  }
});

gpuTest(F, "roofline(): this device's own ceilings (harness/roofline.ts:162-222), measured once per session", async () => {
  const r = await roofline();
  // a read stream cannot beat the 8 TB/s rating; the FMA rate (one-wide v_fma_f32) stays under the published FP32 peak
  assert.ok(r.bandwidth > 3e12 && r.bandwidth < 8.2e12, `bandwidth ${r.bandwidth}`);
  assert.ok(r.compute > 2e13 && r.compute < 1.6e14, `compute ${r.compute}`);
  assert.strictEqual(await roofline(), r, "cached: the same measurement object");
  // the matrix cores on matmulQ8-like operands: under the published 2.5 PFLOP/s dense bf16
  const m = await measureMatrixRoofline();
  assert.ok(m > 5e14 && m < 2.6e15, `matrix ${m}`);
});
