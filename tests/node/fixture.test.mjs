// The reference's tiny int8 Llama (llm/fixtures/tiny_q8.*, copied under
// tests/golden with the logits llm/tools/gen_fixture_q8.py baked by running
// transformers on the dequantized weights): an 8-token prefill and 4 greedy
// decode steps, held to the reference engine's own gate
// (llm/engine-q8-resident.wgsl.test.ts:69, :95-134: every logit within
// rel 1e-2 or abs 5e-3 of the fixture's, the greedy tokens equal).
//
// The projections run on the GPU through the resident device: prefill as
// matmulQ8 dispatches (the engine's prefill pipeline, uniform {N, M, K}),
// decode as the engine's q8 / q8_residual / q8_ffn dispatches built with
// pipelineFor / bindGroup / createUniformBuffer, the embedding rows through
// gatherDequantRows, every weight loaded from the fixture files and packed on
// the device.  The steps this package does not provide (rmsnorm, rope,
// attention, the prefill's residual adds and SiLU) run here in JS, in f64.
// A CPU test pins that glue first: the same model with the oracle's
// projections reaches the fixture's logits.
import { readFileSync } from "fs";
import { dirname, join } from "path";
import { fileURLToPath } from "url";
import { test, gpuTest, assert } from "./harness.mjs";
import { MATMUL_Q8, Q8, Q8_FFN, Q8_RESIDUAL } from "./wgsl_interfaces.mjs";
import { buildLlamaWeightsQ8, llamaConfigFromManifest } from "../../web-xpu-ops_amd/llm/weights-q8-io.js";
import { uploadResidentWeightsQ8 } from "../../web-xpu-ops_amd/llm/resident-weights-q8.js";
import { createResidentDevice, params } from "../../web-xpu-ops_amd/harness/resident.js";
import * as oracle from "../../oracle/q8_oracle.mjs";

const F = "fixture.test.mjs";
const golden = join(dirname(fileURLToPath(import.meta.url)), "..", "golden");
const GATE = { rel: 1e-2, abs: 5e-3 };

function fileBytes(name) {
  const b = readFileSync(join(golden, name));
  return b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength);
}

function loadFixture() {
  const manifest = JSON.parse(readFileSync(join(golden, "tiny_q8.manifest.json"), "utf8"));
  const config = llamaConfigFromManifest(manifest.config, 64);
  const weights = buildLlamaWeightsQ8(manifest.weights, fileBytes("tiny_q8.codes.bin"), fileBytes("tiny_q8.scales.bin"),
    fileBytes("tiny_q8.norms.bin"), config.numLayers);
  const logits = new Float32Array(fileBytes("tiny_q8.logits.bin"));
  const { prefill, decode } = manifest.logits;
  const rows = (part) => {
    const [n, v] = part.shape;
    return Array.from({ length: n }, (_, i) => logits.subarray(part.offset + i * v, part.offset + (i + 1) * v));
  };
  return { manifest, config, weights, prefillLogits: rows(prefill), decodeLogits: rows(decode) };
}

/** harness/agree.ts:27-46: the worst element outside both bounds, or null. */
function agree(got, want, { rel, abs }) {
  assert.strictEqual(got.length, want.length);
  let worst = null;
  for (let i = 0; i < want.length; i += 1) {
    const a = Math.abs(got[i] - want[i]);
    if (a <= abs) continue;
    const r = a / Math.max(Number.MIN_VALUE, Math.abs(want[i]));
    if (r <= rel) continue;
    if (!worst || r > worst.rel) worst = { index: i, got: got[i], want: want[i], rel: r, abs: a };
  }
  return worst;
}

/** The first index of the largest value (torch.argmax's tie rule). */
function argmax(row) {
  let best = 0;
  for (let i = 1; i < row.length; i += 1) if (row[i] > row[best]) best = i;
  return best;
}

// ------------------------------------------------------------------ the model's other steps, in JS

/** RMSNorm per row (transformers' LlamaRMSNorm, eps from the manifest). */
function rmsnormRows(x, weight, T, H, eps) {
  const out = new Float32Array(T * H);
  for (let t = 0; t < T; t += 1) {
    let ss = 0;
    for (let i = 0; i < H; i += 1) ss += x[t * H + i] * x[t * H + i];
    const r = 1 / Math.sqrt(ss / H + eps);
    for (let i = 0; i < H; i += 1) out[t * H + i] = weight[i] * Math.fround(x[t * H + i] * r);
  }
  return out;
}

/**
 * RoPE on the fixture's row order: wq and wk are stored with each head's
 * channels interleaved (row 2i = channel i, row 2i+1 = channel i + headDim/2,
 * llm/tools/gen_fixture.py:80-93), so pair (2i, 2i+1) turns by
 * pos * theta^(-2i/headDim), the rotate_half rotation of transformers.
 */
function rope(v, heads, headDim, pos, theta, halves = false) {
  const out = new Float32Array(v.length);
  const half = headDim / 2;
  for (let h = 0; h < heads; h += 1) {
    for (let i = 0; i < half; i += 1) {
      const ang = pos * Math.pow(theta, -(2 * i) / headDim);
      // `halves` pairs channel i with i + headDim/2 in the stored order: wrong for this fixture (a planted mistake)
      const ia = h * headDim + (halves ? i : 2 * i), ib = h * headDim + (halves ? i + half : 2 * i + 1);
      const a = v[ia], b = v[ib];
      out[ia] = a * Math.cos(ang) - b * Math.sin(ang);
      out[ib] = a * Math.sin(ang) + b * Math.cos(ang);
    }
  }
  return out;
}

/** Grouped-query attention of one position over the cache (every cached position is at or before it). */
function attend(q, keys, values, cfg, mistakes) {
  const { numHeads, numKvHeads, headDim } = cfg;
  const out = new Float32Array(numHeads * headDim);
  const group = numHeads / numKvHeads;
  for (let h = 0; h < numHeads; h += 1) {
    // query head h reads kv head floor(h / group); `kvModulo` plants the round-robin mistake
    const g = mistakes.kvModulo ? h % numKvHeads : Math.floor(h / group);
    const scores = keys.map((k) => {
      let s = 0;
      for (let d = 0; d < headDim; d += 1) s += q[h * headDim + d] * k[g * headDim + d];
      return s / Math.sqrt(headDim);
    });
    const m = Math.max(...scores);
    const e = scores.map((s) => Math.exp(s - m));
    const sum = e.reduce((a, b) => a + b, 0);
    for (let d = 0; d < headDim; d += 1) {
      let acc = 0;
      for (let p = 0; p < values.length; p += 1) acc += (e[p] / sum) * values[p][g * headDim + d];
      out[h * headDim + d] = acc;
    }
  }
  return out;
}

/** Prefill of the prompt, then greedy decode; the projections come from `be`. */
async function runModel(be, fx, mistakes = {}) {
  const cfg = fx.config;
  const { numLayers, hiddenSize: H, numHeads, numKvHeads, headDim, rmsNormEps: eps, ropeTheta } = cfg;
  const qDim = numHeads * headDim, kvDim = numKvHeads * headDim;
  const keys = Array.from({ length: numLayers }, () => []);
  const values = Array.from({ length: numLayers }, () => []);
  let position = 0;
  const forward = async (tokens) => {
    const T = tokens.length;
    let hidden = await be.embed(tokens);
    for (let l = 0; l < numLayers; l += 1) {
      const lw = fx.weights.layers[l];
      const { q, k, v } = await be.qkv(l, rmsnormRows(hidden, lw.attnNorm, T, H, eps), T);
      const attn = new Float32Array(T * qDim);
      for (let t = 0; t < T; t += 1) {
        const pos = position + t;
        keys[l].push(rope(k.subarray(t * kvDim, (t + 1) * kvDim), numKvHeads, headDim, pos, ropeTheta, mistakes.ropeHalves));
        values[l].push(Float32Array.from(v.subarray(t * kvDim, (t + 1) * kvDim)));
        const qt = rope(q.subarray(t * qDim, (t + 1) * qDim), numHeads, headDim, pos, ropeTheta, mistakes.ropeHalves);
        attn.set(attend(qt, keys[l], values[l], cfg, mistakes), t * qDim);
      }
      hidden = await be.attnOut(l, attn, hidden, T);
      hidden = await be.mlp(l, rmsnormRows(hidden, lw.ffnNorm, T, H, eps), hidden, T);
    }
    position += T;
    return be.lmHead(rmsnormRows(hidden, fx.weights.finalNorm, T, H, eps), T);
  };
  const V = cfg.vocabSize;
  const rowsOf = (flat, T) => Array.from({ length: T }, (_, t) => flat.subarray(t * V, (t + 1) * V));
  const prompt = fx.manifest.promptTokens;
  const prefill = rowsOf(await forward(prompt), prompt.length);
  const decodeLogits = [], decodeTokens = [];
  let next = argmax(prefill[prefill.length - 1]);
  for (let s = 0; s < fx.manifest.decodeTokens.length; s += 1) {
    const [row] = rowsOf(await forward([next]), 1);
    decodeLogits.push(row);
    next = argmax(row);
    decodeTokens.push(next);
  }
  return { prefill, decodeLogits, decodeTokens };
}

/** The largest absolute and relative differences over a set of rows. */
function worstDiff(rows, wants) {
  let abs = 0, rel = 0;
  rows.forEach((row, t) => row.forEach((v, i) => {
    const d = Math.abs(v - wants[t][i]);
    abs = Math.max(abs, d);
    rel = Math.max(rel, d / Math.max(Number.MIN_VALUE, Math.abs(wants[t][i])));
  }));
  return { abs, rel };
}

function checkAgainstFixture(run, fx, what) {
  console.log(`  ${what}: worst difference from the fixture, prefill ${JSON.stringify(worstDiff(run.prefill, fx.prefillLogits))}, `
    + `decode ${JSON.stringify(worstDiff(run.decodeLogits, fx.decodeLogits))}`);
  run.prefill.forEach((row, t) => {
    const worst = agree(row, fx.prefillLogits[t], GATE);
    assert.strictEqual(worst, null, `${what} prefill position ${t}: ${JSON.stringify(worst)}`);
  });
  run.decodeLogits.forEach((row, t) => {
    const worst = agree(row, fx.decodeLogits[t], GATE);
    assert.strictEqual(worst, null, `${what} decode step ${t}: ${JSON.stringify(worst)}`);
  });
  assert.deepStrictEqual(run.decodeTokens, fx.manifest.decodeTokens, `${what}: greedy tokens`);
}

// ------------------------------------------------------------------ projections from the oracle (CPU)

function oracleBackend(fx) {
  const w = fx.weights;
  const packed = new Map();
  const lin = (q) => {
    if (!packed.has(q)) {
      const N = q.scale.length, K = q.codes.length / N;
      packed.set(q, { weight: oracle.packInt8Rows(q.codes, N, K), scale: q.scale, N, K });
    }
    return packed.get(q);
  };
  const mm = (q, a, T) => {
    const p = lin(q);
    if (T === 1) return oracle.matvecQ8({ weight: p.weight, scale: p.scale, vector: a, N: p.N, K: p.K });
    return oracle.matmulQ8({ a, weight: p.weight, scale: p.scale, N: T, M: p.N, K: p.K });
  };
  const add = (x, y) => Float32Array.from(x, (v, i) => v + y[i]);
  return {
    embed: async (tokens) => oracle.gatherDequantRows(w.embedTokens, tokens, fx.config.hiddenSize),
    qkv: async (l, x, T) => ({ q: mm(w.layers[l].wq, x, T), k: mm(w.layers[l].wk, x, T), v: mm(w.layers[l].wv, x, T) }),
    attnOut: async (l, attn, hidden, T) => {
      if (T > 1) return add(hidden, mm(w.layers[l].wo, attn, T));
      const p = lin(w.layers[l].wo);
      return oracle.matvecQ8Residual({ weight: p.weight, scale: p.scale, vector: attn, residual: hidden, N: p.N, K: p.K });
    },
    mlp: async (l, x, hidden, T) => {
      const L = w.layers[l];
      let gated;
      if (T > 1) {
        const g = mm(L.wGate, x, T), u = mm(L.wUp, x, T);
        gated = Float32Array.from(g, (v, i) => Math.fround(oracle.silu(v)) * u[i]);
        return add(hidden, mm(L.wDown, gated, T));
      }
      const pg = lin(L.wGate), pu = lin(L.wUp), pd = lin(L.wDown);
      gated = oracle.matvecQ8Ffn({ weightGate: pg.weight, scaleGate: pg.scale, weightUp: pu.weight, scaleUp: pu.scale,
        vector: x, N: pg.N, K: pg.K });
      return oracle.matvecQ8Residual({ weight: pd.weight, scale: pd.scale, vector: gated, residual: hidden, N: pd.N, K: pd.K });
    },
    lmHead: async (x, T) => mm(w.lmHead, x, T),
  };
}

// ------------------------------------------------------------------ projections on the GPU

async function residentBackend(device, fx) {
  const cfg = fx.config;
  const H = cfg.hiddenSize, P = fx.manifest.promptTokens.length;
  const r = await uploadResidentWeightsQ8(device, fx.weights);
  const [mmPipe, mvPipe, ffnPipe, resPipe] = await Promise.all(
    [device.pipelineFor(MATMUL_Q8), device.pipelineFor(Q8), device.pipelineFor(Q8_FFN), device.pipelineFor(Q8_RESIDUAL)]);
  const buf = (floats) => device.createStorageBuffer(floats * 4);
  const uniform = (fields) => {
    const data = params(fields);
    const u = device.createUniformBuffer(data.byteLength);
    device.upload(u, 0, new Uint8Array(data));
    return u;
  };
  const maxK = Math.max(H, cfg.ffnHidden, cfg.numHeads * cfg.headDim);
  const x = buf(P * maxK), out = buf(P * Math.max(cfg.vocabSize, H)), resid = buf(H), gated = buf(cfg.ffnHidden);
  // q / k / v outputs; the first two also take gate and up in prefill
  const qkvOut = [buf(P * Math.max(r.layers[0].wq.N, cfg.ffnHidden)), buf(P * Math.max(r.layers[0].wk.N, cfg.ffnHidden)),
    buf(P * r.layers[0].wv.N)];
  const idx = device.createStorageBuffer(P * 8);
  // one matmul and one matvec bind group per projection, built once as the engine builds them
  const project = (lin, outBuf) => {
    const mmUniform = device.createUniformBuffer(12);
    return {
      lin, outBuf, mmUniform,
      mm: device.bindGroup(mmPipe, [x, lin.weight, lin.scale, outBuf, mmUniform]),
      mv: device.bindGroup(mvPipe, [lin.weight, lin.scale, x, outBuf, uniform([["u32", lin.N], ["u32", lin.K]])]),
    };
  };
  const layers = [];
  for (const L of r.layers) {
    const p = {
      wq: project(L.wq, qkvOut[0]), wk: project(L.wk, qkvOut[1]), wv: project(L.wv, qkvOut[2]),
      wo: project(L.wo, out), wGate: project(L.wGate, qkvOut[0]), wUp: project(L.wUp, qkvOut[1]), wDown: project(L.wDown, out),
    };
    for (const k of Object.keys(p)) {
      p[k].mm = await p[k].mm;
      p[k].mv = await p[k].mv;
    }
    // decode's fused forms: wo and down add into the residual in place, gate and up meet in the FFN kernel
    p.woResidual = await device.bindGroup(resPipe, [L.wo.weight, L.wo.scale, x, resid, resid, uniform([["u32", L.wo.N], ["u32", L.wo.K]])]);
    p.ffn = await device.bindGroup(ffnPipe, [L.wGate.weight, L.wGate.scale, L.wUp.weight, L.wUp.scale, x, gated,
      uniform([["u32", L.wGate.N], ["u32", L.wGate.K]])]);
    p.downResidual = await device.bindGroup(resPipe, [L.wDown.weight, L.wDown.scale, gated, resid, resid,
      uniform([["u32", L.wDown.N], ["u32", L.wDown.K]])]);
    layers.push(p);
  }
  const lmHead = project(r.lmHead, out);
  lmHead.mm = await lmHead.mm;
  lmHead.mv = await lmHead.mv;

  const read = (b, n) => ({ source: b, sourceOffset: 0, length: n, type: "f32" });
  const upload = (b, a) => device.upload(b, 0, a);
  // prefill: matmulQ8 dispatches over T tokens; decode: the q8 dispatch, one workgroup per row
  const dispatch = (p, T) => {
    if (T === 1) return { kind: "dispatch", pipeline: mvPipe, bindGroup: p.mv, workgroups: [p.lin.N] };
    device.upload(p.mmUniform, 0, new Uint8Array(params([["u32", T], ["u32", p.lin.N], ["u32", p.lin.K]])));
    return { kind: "dispatch", pipeline: mmPipe, bindGroup: p.mm, workgroups: [Math.ceil(p.lin.N / 16), Math.ceil(T / 16)] };
  };
  const run1 = async (p, a, T) => {
    upload(x, a);
    const [y] = await device.batch([dispatch(p, T)], [read(p.outBuf, T * p.lin.N)]);
    return y;
  };
  const add = (a, b) => Float32Array.from(a, (v, i) => v + b[i]);
  return {
    embed: async (tokens) => {
      upload(idx, BigInt64Array.from(tokens.map((t) => BigInt(t))));
      const e = r.embedTokens;
      const [h] = await device.batch([{ kind: "gatherDequantRows", codes: e.weight, scale: e.scale, rows: e.N, D: e.K,
        indices: idx, count: tokens.length, output: x }], [read(x, tokens.length * H)]);
      return h;
    },
    qkv: async (l, a, T) => {
      upload(x, a);
      const p = layers[l];
      const [q, k, v] = await device.batch([dispatch(p.wq, T), dispatch(p.wk, T), dispatch(p.wv, T)],
        [read(qkvOut[0], T * p.wq.lin.N), read(qkvOut[1], T * p.wk.lin.N), read(qkvOut[2], T * p.wv.lin.N)]);
      return { q, k, v };
    },
    attnOut: async (l, attn, hidden, T) => {
      const p = layers[l];
      if (T > 1) return add(hidden, await run1(p.wo, attn, T));
      upload(x, attn);
      upload(resid, hidden);
      const [h] = await device.batch([{ kind: "dispatch", pipeline: resPipe, bindGroup: p.woResidual, workgroups: [H] }],
        [read(resid, H)]);
      return h;
    },
    mlp: async (l, a, hidden, T) => {
      const p = layers[l];
      if (T > 1) {
        upload(x, a);
        const [g, u] = await device.batch([dispatch(p.wGate, T), dispatch(p.wUp, T)],
          [read(qkvOut[0], T * p.wGate.lin.N), read(qkvOut[1], T * p.wUp.lin.N)]);
        const gatedRows = Float32Array.from(g, (v, i) => Math.fround(oracle.silu(v)) * u[i]);
        return add(hidden, await run1(p.wDown, gatedRows, T));
      }
      upload(x, a);
      upload(resid, hidden);
      const [h] = await device.batch([
        { kind: "dispatch", pipeline: ffnPipe, bindGroup: p.ffn, workgroups: [cfg.ffnHidden] },
        { kind: "dispatch", pipeline: resPipe, bindGroup: p.downResidual, workgroups: [H] },
      ], [read(resid, H)]);
      return h;
    },
    lmHead: async (a, T) => run1(lmHead, a, T),
  };
}

// ------------------------------------------------------------------ tests

test(F, "the tiny_q8 model with the oracle's projections reaches the fixture's logits and greedy tokens (pins the JS steps)", async () => {
  const fx = loadFixture();
  assert.strictEqual(fx.prefillLogits.length, fx.manifest.promptTokens.length);
  const run = await runModel(oracleBackend(fx), fx);
  checkAgainstFixture(run, fx, "oracle");
  // far inside the gate: transformers' f32 forward and this f64 one differ by f32 roundings only
  const close = { rel: 0, abs: 1e-5 };
  run.prefill.forEach((row, t) => assert.strictEqual(agree(row, fx.prefillLogits[t], close), null, `prefill ${t} within 1e-5`));
  run.decodeLogits.forEach((row, t) => assert.strictEqual(agree(row, fx.decodeLogits[t], close), null, `decode ${t} within 1e-5`));
  // plausible mistakes in these steps miss the gate: rope pairs taken as halves (transformers' own layout, not the
  // fixture's interleave), query heads mapped round-robin onto the kv heads
  for (const mistakes of [{ ropeHalves: true }, { kvModulo: true }]) {
    const bad = await runModel(oracleBackend(fx), fx, mistakes);
    assert.ok(bad.prefill.some((row, t) => agree(row, fx.prefillLogits[t], GATE) !== null),
      `${JSON.stringify(mistakes)} should miss the gate`);
  }
});

gpuTest(F, "the tiny_q8 model on the GPU projections: prefill and greedy decode pass the engine's gate, and track the oracle's logits", async () => {
  const fx = loadFixture();
  const device = await createResidentDevice();
  assert.ok(device);
  try {
    const be = await residentBackend(device, fx);
    const buffers = device.stats.buffersCreated;
    const run = await runModel(be, fx);
    assert.strictEqual(device.stats.buffersCreated, buffers, "no buffer is created once the model is resident");
    checkAgainstFixture(run, fx, "GPU");
    const cpu = await runModel(oracleBackend(fx), fx);
    const tight = { rel: 1e-4, abs: 1e-5 };
    run.prefill.forEach((row, t) => assert.strictEqual(agree(row, cpu.prefill[t], tight), null, `prefill ${t} vs oracle`));
    run.decodeLogits.forEach((row, t) => assert.strictEqual(agree(row, cpu.decodeLogits[t], tight), null, `decode ${t} vs oracle`));
  } finally {
    device.destroy();
  }
});
