// llm/weights-q8-io: the q8 weight manifest parser, with the reference's API
// (llm/weights-q8-io.ts:1-76 types, :49-51 llamaConfigFromManifest, :76-140
// buildLlamaWeightsQ8).  Pure and buffer-agnostic: the caller reads the
// manifest and the three files (codes.bin int8, scales.bin f32, norms.bin f32)
// and passes their bytes; the result holds typed-array views into them.
// Nothing here touches the GPU; llm/resident-weights-q8.js uploads the views.

/** `WeightManifestConfig` plus `maxSeqLen` (llm/weights-q8-io.ts:49-51). */
export function llamaConfigFromManifest(config, maxSeqLen) {
  return Object.assign({}, config, { maxSeqLen });
}

function elementsOf(shape) {
  return shape.reduce((a, b) => a * b, 1);
}

/**
 * `buildLlamaWeightsQ8(entries, codesBuffer, scalesBuffer, normsBuffer, numLayers)`:
 * quantized entries `{name, kind: "quant", shape: [N, K], codesOffset (int8
 * elements), scaleOffset (f32 elements)}` become `{codes: Int8Array[N*K],
 * scale: Float32Array[N]}`; norm entries `{name, kind: "norm", shape, offset}`
 * become Float32Array views.  Returns `{embedTokens, layers[], finalNorm,
 * lmHead}` with per-layer `attnNorm, wq, wk, wv, wo, ffnNorm, wGate, wUp,
 * wDown`; a missing name throws, as the reference does.
 */
export function buildLlamaWeightsQ8(entries, codesBuffer, scalesBuffer, normsBuffer, numLayers) {
  const quant = new Map();
  const norms = new Map();
  for (const entry of entries) {
    if (entry.kind === "quant") {
      const [n, k] = entry.shape;
      quant.set(entry.name, {
        codes: new Int8Array(codesBuffer, entry.codesOffset, n * k),
        scale: new Float32Array(scalesBuffer, entry.scaleOffset * 4, n),
      });
    } else {
      norms.set(entry.name, new Float32Array(normsBuffer, entry.offset * 4, elementsOf(entry.shape)));
    }
  }
  const getQuant = (name) => {
    const found = quant.get(name);
    if (!found) throw new Error(`buildLlamaWeightsQ8: no quantized weight named ${JSON.stringify(name)}`);
    return found;
  };
  const getNorm = (name) => {
    const found = norms.get(name);
    if (!found) throw new Error(`buildLlamaWeightsQ8: no norm weight named ${JSON.stringify(name)}`);
    return found;
  };
  const layers = [];
  for (let i = 0; i < numLayers; i += 1) {
    layers.push({
      attnNorm: getNorm(`layers.${i}.attnNorm`),
      wq: getQuant(`layers.${i}.wq`),
      wk: getQuant(`layers.${i}.wk`),
      wv: getQuant(`layers.${i}.wv`),
      wo: getQuant(`layers.${i}.wo`),
      ffnNorm: getNorm(`layers.${i}.ffnNorm`),
      wGate: getQuant(`layers.${i}.wGate`),
      wUp: getQuant(`layers.${i}.wUp`),
      wDown: getQuant(`layers.${i}.wDown`),
    });
  }
  return { embedTokens: getQuant("embedTokens"), layers, finalNorm: getNorm("finalNorm"), lmHead: getQuant("lmHead") };
}
