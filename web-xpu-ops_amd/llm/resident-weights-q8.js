// llm/resident-weights-q8: a LlamaWeightsQ8 (llm/weights-q8-io.js) made
// resident on a ResidentQ8Device, packed on the GPU.  The reference's resident
// engine packs every projection on the CPU with packInt8Rows and then uploads
// the words (llm/engine-q8-resident.ts:521-538, ~0.62 GB/s per README.md:1811);
// here the int8 codes are uploaded as they are and packed on the device.
//
// packQ8's layout is the little-endian byte view of each row padded to 4
// bytes (llm/weights-q8.ts:118-139), so for K % 4 == 0 the packed weight is
// the codes' bytes unchanged: the upload is the pack.  Rows whose length is
// not a multiple of 4 go through a staging buffer and packInt8Rows on the GPU.

function shapeOf(linear) {
  const N = linear.scale.length;
  if (N === 0 || linear.codes.length % N !== 0) {
    throw new RangeError(`a quantized linear needs codes of N * K bytes for its N = ${N} scales`);
  }
  return { N, K: linear.codes.length / N };
}

async function uploadLinear(device, linear, staging) {
  const { N, K } = shapeOf(linear);
  const weight = device.createStorageBuffer(N * Math.ceil(K / 4) * 4);
  const scale = device.createStorageBuffer(N * 4);
  device.upload(scale, 0, linear.scale);
  if (K % 4 === 0) {
    device.upload(weight, 0, linear.codes);
  } else {
    device.upload(staging, 0, linear.codes);
    await device.batch([{ kind: "packInt8Rows", codes: staging, N, K, packed: weight }]);
  }
  return { weight, scale, N, K };
}

function raggedBytes(linears) {
  let bytes = 0;
  for (const l of linears) {
    const { N, K } = shapeOf(l);
    if (K % 4 !== 0) bytes = Math.max(bytes, N * K);
  }
  return bytes;
}

/**
 * `uploadQuantizedLinear(device, { codes: Int8Array[N*K], scale: Float32Array[N] })`
 * -> `{ weight, scale, N, K }`: resident packed u32 [N, ceil(K/4)] and f32 [N].
 */
export async function uploadQuantizedLinear(device, linear) {
  const bytes = raggedBytes([linear]);
  return uploadLinear(device, linear, bytes > 0 ? device.createStorageBuffer(bytes) : null);
}

/**
 * `uploadResidentWeightsQ8(device, weights)` -> `{ embedTokens, layers, finalNorm,
 * lmHead }`: every quantized linear as `{ weight, scale, N, K }`, every norm
 * as a resident f32 buffer, the layer objects keyed as in LlamaWeightsQ8.
 * One staging buffer serves every ragged matrix in turn.
 */
export async function uploadResidentWeightsQ8(device, weights) {
  const all = [weights.embedTokens, weights.lmHead];
  for (const l of weights.layers) all.push(l.wq, l.wk, l.wv, l.wo, l.wGate, l.wUp, l.wDown);
  const bytes = raggedBytes(all);
  const staging = bytes > 0 ? device.createStorageBuffer(bytes) : null;
  const lin = (l) => uploadLinear(device, l, staging);
  const norm = (a) => {
    const b = device.createStorageBuffer(a.byteLength);
    device.upload(b, 0, a);
    return b;
  };
  const layers = [];
  for (const l of weights.layers) {
    layers.push({
      attnNorm: norm(l.attnNorm), wq: await lin(l.wq), wk: await lin(l.wk), wv: await lin(l.wv), wo: await lin(l.wo),
      ffnNorm: norm(l.ffnNorm), wGate: await lin(l.wGate), wUp: await lin(l.wUp), wDown: await lin(l.wDown),
    });
  }
  return { embedTokens: await lin(weights.embedTokens), layers, finalNorm: norm(weights.finalNorm), lmHead: await lin(weights.lmHead) };
}
