// Runs one op of the ECMAScript oracle (oracle/q8_oracle.mjs) on arrays sent as
// base64 in a JSON job on stdin; prints the outputs as base64 JSON on stdout.
// Lets the Python tests hold the C oracle and the JS oracle to each other.
import { quantize, packQ8, packInt8Rows, matvecQ8, matvecQ8Ffn, matvecQ8Residual, matmulQ8, dequantizePackedQ8,
  dequantTranspose, gatherDequantRows } from "../../oracle/q8_oracle.mjs";

const typed = { f32: Float32Array, i32: Int32Array, u32: Uint32Array, i8: Int8Array, f64: Float64Array };
function decode(spec) {
  const buf = Buffer.from(spec.b64, "base64");
  const T = typed[spec.dtype];
  const copy = new Uint8Array(buf.length);
  copy.set(buf);
  return new T(copy.buffer, 0, buf.length / T.BYTES_PER_ELEMENT);
}
const encode = (arr) => Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength).toString("base64");

let text = "";
process.stdin.setEncoding("utf8");
process.stdin.on("data", (chunk) => { text += chunk; });
process.stdin.on("end", () => {
  const job = JSON.parse(text);
  const a = {};
  for (const [name, spec] of Object.entries(job.arrays || {})) a[name] = decode(spec);
  let out;
  switch (job.op) {
    case "quantize": {
      const r = quantize({ input: a.input, N: job.N, D: job.D });
      out = { output: encode(r.output), scales: encode(r.scales) };
      break;
    }
    case "packQ8":
      out = { packed: encode(packQ8({ codes: a.codes, N: job.N, K: job.K })) };
      break;
    case "packInt8Rows":
      out = { packed: encode(packInt8Rows(a.codes, job.N, job.K)) };
      break;
    case "matvecQ8":
      out = { output: encode(matvecQ8({ weight: a.weight, scale: a.scale, vector: a.vector, N: job.N, K: job.K })) };
      break;
    case "matvecQ8Ffn":
      out = { output: encode(matvecQ8Ffn({ weightGate: a.weightGate, scaleGate: a.scaleGate, weightUp: a.weightUp,
                                           scaleUp: a.scaleUp, vector: a.vector, N: job.N, K: job.K })) };
      break;
    case "matvecQ8Residual":
      out = { output: encode(matvecQ8Residual({ weight: a.weight, scale: a.scale, vector: a.vector,
                                                residual: a.residual, N: job.N, K: job.K })) };
      break;
    case "matmulQ8":
      out = { output: encode(matmulQ8({ a: a.a, weight: a.weight, scale: a.scale, N: job.N, M: job.M, K: job.K })) };
      break;
    case "dequantizePackedQ8":
      out = { output: encode(dequantizePackedQ8(a.weight, a.scale, job.N, job.K)) };
      break;
    case "dequantTranspose":
      out = { output: encode(dequantTranspose({ weight: a.weight, scale: a.scale, outFeatures: job.N,
                                                inFeatures: job.K })) };
      break;
    case "gatherDequantRows":
      out = { output: encode(gatherDequantRows({ codes: a.codes, scale: a.scale }, Array.from(a.indices), job.D)) };
      break;
    default:
      throw new Error(`unknown op ${job.op}`);
  }
  process.stdout.write(JSON.stringify(out));
});
