// WGSL texts that declare the binding interfaces of the reference's resident
// kernels (ops/matvec/wgsl/q8.wgsl:26-35, q8_ffn.wgsl:24-35,
// q8_residual.wgsl:25-35, ops/matmul/wgsl/q8.wgsl:26-36) with empty bodies:
// what a caller hands `pipelineFor` is the kernel's WGSL text, and the
// resident device reads only its interface.  Written here as interface
// declarations (the reference tree is not available to tests at run time).

function kernel(params, bindings, entry = "main") {
  return `// test interface
struct Params {
${params.map(([n, t]) => `  ${n}: ${t},`).join("\n")}
}

${bindings.map(([space, name, type], i) =>
    `@group(0) @binding(${i}) var<${space}> ${name}: ${type};`).join("\n")}

@compute @workgroup_size(256)
fn ${entry}(@builtin(workgroup_id) wg_id: vec3<u32>) {
}
`;
}

const RO = "storage, read";
const RW = "storage, read_write";

export const Q8 = kernel([["N", "u32"], ["K", "u32"]], [
  [RO, "weight", "array<u32>"], [RO, "scale", "array<f32>"], [RO, "vector", "array<f32>"],
  [RW, "output", "array<f32>"], ["uniform", "params", "Params"]]);

export const Q8_FFN = kernel([["N", "u32"], ["K", "u32"]], [
  [RO, "weight_gate", "array<u32>"], [RO, "scale_gate", "array<f32>"], [RO, "weight_up", "array<u32>"],
  [RO, "scale_up", "array<f32>"], [RO, "vector", "array<f32>"], [RW, "output", "array<f32>"],
  ["uniform", "params", "Params"]]);

export const Q8_RESIDUAL = kernel([["N", "u32"], ["K", "u32"]], [
  [RO, "weight", "array<u32>"], [RO, "scale", "array<f32>"], [RO, "vector", "array<f32>"],
  [RO, "residual", "array<f32>"], [RW, "output", "array<f32>"], ["uniform", "params", "Params"]]);

export const MATMUL_Q8 = kernel([["N", "u32"], ["M", "u32"], ["K", "u32"]], [
  [RO, "a", "array<f32>"], [RO, "weight", "array<u32>"], [RO, "scale", "array<f32>"],
  [RW, "output", "array<f32>"], ["uniform", "params", "Params"]]);

/** An rmsnorm-shaped kernel (input, weight, output, {N, eps}): not part of this build. */
export const RMSNORM_LIKE = kernel([["N", "u32"], ["eps", "f32"]], [
  [RO, "input", "array<f32>"], [RO, "weight", "array<f32>"], [RW, "output", "array<f32>"],
  ["uniform", "params", "Params"]]);

export { kernel };
