// The q8 weight loader (llm/weights-q8-io.js, reference llm/weights-q8-io.ts)
// and the resident upload that packs on the GPU (llm/resident-weights-q8.js),
// on the reference's committed tiny fixture (llm/fixtures/tiny_q8.*, copied
// under tests/golden) and on the reference test's own synthetic manifest
// shapes (llm/weights-q8-io.test.ts:17-80).
import { readFileSync } from "fs";
import { dirname, join } from "path";
import { fileURLToPath } from "url";
import { test, gpuTest, assert, assertBitsEqual, assertMatvecAgrees } from "./harness.mjs";
import { buildLlamaWeightsQ8, llamaConfigFromManifest } from "../../web-xpu-ops_amd/llm/weights-q8-io.js";
import { uploadResidentWeightsQ8, uploadQuantizedLinear } from "../../web-xpu-ops_amd/llm/resident-weights-q8.js";
import { createResidentQ8Device } from "../../web-xpu-ops_amd/harness/resident.js";
import * as oracle from "../../oracle/q8_oracle.mjs";

const F = "loader.test.mjs";
const golden = join(dirname(fileURLToPath(import.meta.url)), "..", "golden");

function fileBytes(name) {
  const b = readFileSync(join(golden, name));
  return b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength);
}

function loadTiny() {
  const manifest = JSON.parse(readFileSync(join(golden, "tiny_q8.manifest.json"), "utf8"));
  const codes = fileBytes("tiny_q8.codes.bin"), scales = fileBytes("tiny_q8.scales.bin"), norms = fileBytes("tiny_q8.norms.bin");
  const config = llamaConfigFromManifest(manifest.config, 64);
  const weights = buildLlamaWeightsQ8(manifest.weights, codes, scales, norms, config.numLayers);
  return { manifest, codes, scales, norms, config, weights };
}

test(F, "llamaConfigFromManifest carries every manifest field plus maxSeqLen (weights-q8-io.test.ts:31-36)", () => {
  const c = { numLayers: 1, hiddenSize: 4, numHeads: 2, numKvHeads: 1, headDim: 2, ffnHidden: 3, vocabSize: 5,
    ropeTheta: 10000, rmsNormEps: 1e-5, tieEmbeddings: false };
  assert.deepStrictEqual(llamaConfigFromManifest(c, 64), Object.assign({}, c, { maxSeqLen: 64 }));
});

test(F, "buildLlamaWeightsQ8 reads each weight at its own manifest offsets (weights-q8-io.test.ts:38-80 shapes)", () => {
  // hidden 4, q 4, kv 2, ffn 3, vocab 5: distinct enough that a swapped
  // offset or shape reads other bytes.  Codes and scales are numbered by
  // their position so every view's content names where it was read from.
  const H = 4, Q = 4, KV = 2, FF = 3, V = 5;
  const shapes = [["embedTokens", V, H], ["layers.0.wq", Q, H], ["layers.0.wk", KV, H], ["layers.0.wv", KV, H],
    ["layers.0.wo", H, Q], ["layers.0.wGate", FF, H], ["layers.0.wUp", FF, H], ["layers.0.wDown", H, FF], ["lmHead", V, H]];
  const entries = [];
  let co = 0, so = 0;
  for (const [name, n, k] of shapes) {
    entries.push({ name, kind: "quant", shape: [n, k], codesOffset: co, scaleOffset: so });
    co += n * k;
    so += n;
  }
  entries.push({ name: "layers.0.attnNorm", kind: "norm", shape: [H], offset: 0 });
  entries.push({ name: "layers.0.ffnNorm", kind: "norm", shape: [H], offset: H });
  entries.push({ name: "finalNorm", kind: "norm", shape: [H], offset: 2 * H });
  const codes = Int8Array.from({ length: co }, (_, i) => (i % 251) - 125);
  const scales = Float32Array.from({ length: so }, (_, i) => i + 0.5);
  const norms = Float32Array.from({ length: 3 * H }, (_, i) => -i);
  const w = buildLlamaWeightsQ8(entries, codes.buffer, scales.buffer, norms.buffer, 1);
  const byName = { embedTokens: w.embedTokens, lmHead: w.lmHead, "layers.0.wq": w.layers[0].wq, "layers.0.wk": w.layers[0].wk,
    "layers.0.wv": w.layers[0].wv, "layers.0.wo": w.layers[0].wo, "layers.0.wGate": w.layers[0].wGate,
    "layers.0.wUp": w.layers[0].wUp, "layers.0.wDown": w.layers[0].wDown };
  for (const e of entries.filter((x) => x.kind === "quant")) {
    const lin = byName[e.name];
    assert.deepStrictEqual(Array.from(lin.codes), Array.from(codes.subarray(e.codesOffset, e.codesOffset + e.shape[0] * e.shape[1])), e.name);
    assert.deepStrictEqual(Array.from(lin.scale), Array.from(scales.subarray(e.scaleOffset, e.scaleOffset + e.shape[0])), e.name);
  }
  assert.deepStrictEqual(Array.from(w.layers[0].ffnNorm), [-4, -5, -6, -7]);
  assert.deepStrictEqual(Array.from(w.finalNorm), [-8, -9, -10, -11]);
  assert.throws(() => buildLlamaWeightsQ8(entries.filter((e) => e.name !== "layers.0.wo"), codes.buffer, scales.buffer,
    norms.buffer, 1), /no quantized weight named "layers.0.wo"/);
  assert.throws(() => buildLlamaWeightsQ8(entries, codes.buffer, scales.buffer, norms.buffer, 2), /layers.1/);
});

test(F, "the tiny fixture loads: every entry in range, shapes as the manifest's config says", () => {
  const { config, weights, codes } = loadTiny();
  const { hiddenSize: H, numHeads, numKvHeads, headDim, ffnHidden, vocabSize } = config;
  const shape = (l) => [l.scale.length, l.codes.length / l.scale.length];
  assert.deepStrictEqual(shape(weights.embedTokens), [vocabSize, H]);
  assert.deepStrictEqual(shape(weights.lmHead), [vocabSize, H]);
  for (const l of weights.layers) {
    assert.deepStrictEqual(shape(l.wq), [numHeads * headDim, H]);
    assert.deepStrictEqual(shape(l.wk), [numKvHeads * headDim, H]);
    assert.deepStrictEqual(shape(l.wo), [H, numHeads * headDim]);
    assert.deepStrictEqual(shape(l.wGate), [ffnHidden, H]);
    assert.deepStrictEqual(shape(l.wDown), [H, ffnHidden]);
    assert.strictEqual(l.attnNorm.length, H);
  }
  assert.strictEqual(weights.layers.length, config.numLayers);
  assert.strictEqual(codes.byteLength, 106496);
});

gpuTest(F, "uploadResidentWeightsQ8: every resident weight equals packInt8Rows of its codes, scales as given", async () => {
  const dev = await createResidentQ8Device();
  const { weights } = loadTiny();
  const r = await uploadResidentWeightsQ8(dev, weights);
  const pairs = [[r.embedTokens, weights.embedTokens], [r.lmHead, weights.lmHead]];
  r.layers.forEach((l, i) => {
    for (const k of ["wq", "wk", "wv", "wo", "wGate", "wUp", "wDown"]) pairs.push([l[k], weights.layers[i][k]]);
  });
  const reads = [];
  for (const [res] of pairs) {
    reads.push({ source: res.weight, sourceOffset: 0, length: res.N * Math.ceil(res.K / 4), type: "u32" });
    reads.push({ source: res.scale, sourceOffset: 0, length: res.N, type: "f32" });
  }
  const back = await dev.batch([], reads);
  pairs.forEach(([res, src], i) => {
    assertBitsEqual(back[2 * i], oracle.packInt8Rows(src.codes, res.N, res.K), `weight ${i}`);
    assertBitsEqual(back[2 * i + 1], src.scale, `scale ${i}`);
  });
  // the resident lm_head drives a matvecQ8 like the engine's last projection
  const { N, K } = r.lmHead;
  const vector = Float32Array.from({ length: K }, (_, i) => Math.sin(i * 0.37));
  const x = dev.createStorageBuffer(K * 4), y = dev.createStorageBuffer(N * 4);
  dev.upload(x, 0, vector);
  const [logits] = await dev.batch([{ kind: "matvecQ8", weight: r.lmHead.weight, scale: r.lmHead.scale, vector: x, output: y, N, K }],
    [{ source: y, sourceOffset: 0, length: N, type: "f32" }]);
  const args = { weight: oracle.packInt8Rows(weights.lmHead.codes, N, K), scale: weights.lmHead.scale, vector, N, K };
  assertMatvecAgrees(logits, oracle.matvecQ8(args), args, "resident lm_head");
  dev.destroy();
});

gpuTest(F, "uploadQuantizedLinear packs ragged rows on the GPU (K % 4 != 0)", async () => {
  const dev = await createResidentQ8Device();
  for (const [N, K] of [[3, 7], [17, 1027], [256, 4099]]) {
    const codes = Int8Array.from({ length: N * K }, (_, i) => ((i * 37) % 255) - 127);
    const scale = Float32Array.from({ length: N }, (_, i) => 0.01 * (i + 1));
    const r = await uploadQuantizedLinear(dev, { codes, scale });
    const [words] = await dev.batch([], [{ source: r.weight, sourceOffset: 0, length: N * Math.ceil(K / 4), type: "u32" }]);
    assertBitsEqual(words, oracle.packInt8Rows(codes, N, K), `N=${N} K=${K}`);
  }
  dev.destroy();
});
