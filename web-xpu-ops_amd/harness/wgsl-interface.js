// harness/wgsl-interface: recognises which reference WGSL kernel a resident
// `pipelineFor(code, entry)` call names, from the kernel's binding
// declarations (the interface), so that a caller holding the reference's
// WGSL text -- llm/engine-q8-resident.ts:1059-1078 builds its pipelines with
// `device.pipelineFor(CODE.matvecQ8)` where CODE.matvecQ8 is the text of
// ops/matvec/wgsl/q8.wgsl -- gets the MI355X kernel behind the same binding
// order.  Nothing of the WGSL bodies is used: only the @group(0) @binding(n)
// declarations (name, address space, access, type), the uniform struct's
// fields and the existence of the @compute entry point.
//
// Recognised interfaces (binding order as declared by the reference):
//   matvecQ8          ops/matvec/wgsl/q8.wgsl:26-35
//                     weight u32[] r, scale f32[] r, vector f32[] r, output f32[] rw, params {N, K}
//   matvecQ8Ffn       ops/matvec/wgsl/q8_ffn.wgsl:24-35
//                     weight_gate, scale_gate, weight_up, scale_up, vector, output rw, params {N, K}
//   matvecQ8Residual  ops/matvec/wgsl/q8_residual.wgsl:25-35
//                     weight, scale, vector, residual, output rw, params {N, K}
//   matmulQ8          ops/matmul/wgsl/q8.wgsl:26-36
//                     a f32[] r, weight u32[] r, scale f32[] r, output f32[] rw, params {N, M, K}
// Anything else throws UnsupportedPipelineError.

/** Thrown by `pipelineFor` for a kernel this device does not run. */
export class UnsupportedPipelineError extends Error {
  constructor(message) {
    super(message);
    this.name = "UnsupportedPipelineError";
  }
}

const R = "read";
const RW = "read_write";

// [name, address space, access, element type] per binding; the uniform's
// struct fields as [name, type].
export const INTERFACES = Object.freeze([
  {
    op: "matvecQ8",
    source: "ops/matvec/wgsl/q8.wgsl",
    bindings: [["weight", "storage", R, "u32"], ["scale", "storage", R, "f32"], ["vector", "storage", R, "f32"],
      ["output", "storage", RW, "f32"], ["params", "uniform", null, null]],
    params: [["N", "u32"], ["K", "u32"]],
  },
  {
    op: "matvecQ8Ffn",
    source: "ops/matvec/wgsl/q8_ffn.wgsl",
    bindings: [["weight_gate", "storage", R, "u32"], ["scale_gate", "storage", R, "f32"],
      ["weight_up", "storage", R, "u32"], ["scale_up", "storage", R, "f32"], ["vector", "storage", R, "f32"],
      ["output", "storage", RW, "f32"], ["params", "uniform", null, null]],
    params: [["N", "u32"], ["K", "u32"]],
  },
  {
    op: "matvecQ8Residual",
    source: "ops/matvec/wgsl/q8_residual.wgsl",
    bindings: [["weight", "storage", R, "u32"], ["scale", "storage", R, "f32"], ["vector", "storage", R, "f32"],
      ["residual", "storage", R, "f32"], ["output", "storage", RW, "f32"], ["params", "uniform", null, null]],
    params: [["N", "u32"], ["K", "u32"]],
  },
  {
    op: "matmulQ8",
    source: "ops/matmul/wgsl/q8.wgsl",
    bindings: [["a", "storage", R, "f32"], ["weight", "storage", R, "u32"], ["scale", "storage", R, "f32"],
      ["output", "storage", RW, "f32"], ["params", "uniform", null, null]],
    params: [["N", "u32"], ["M", "u32"], ["K", "u32"]],
  },
]);

function stripComments(code) {
  return code.replace(/\/\*[\s\S]*?\*\//g, " ").replace(/\/\/[^\n]*/g, " ");
}

const BINDING = /@group\(\s*(\d+)\s*\)\s*@binding\(\s*(\d+)\s*\)\s*var\s*<\s*([a-z_]+)\s*(?:,\s*([a-z_]+)\s*)?>\s*([A-Za-z_]\w*)\s*:\s*([^;]+);/g;

/** The declared bindings of group 0, in binding order: { binding, space, access, name, type }. */
export function parseBindings(code) {
  const text = stripComments(code);
  const out = [];
  for (const m of text.matchAll(BINDING)) {
    if (m[1] !== "0") continue;
    out.push({ binding: Number(m[2]), space: m[3], access: m[4] || (m[3] === "storage" ? R : null), name: m[5],
      type: m[6].replace(/\s+/g, "") });
  }
  out.sort((x, y) => x.binding - y.binding);
  return out;
}

/** Fields [name, type] of `struct <name> { ... }`, or null when absent. */
export function parseStruct(code, name) {
  const text = stripComments(code);
  const m = new RegExp(`struct\\s+${name}\\s*\\{([^}]*)\\}`).exec(text);
  if (!m) return null;
  return m[1].split(",").map((f) => f.trim()).filter(Boolean).map((f) => {
    const [n, t] = f.split(":").map((x) => x.trim());
    return [n, t];
  });
}

function hasComputeEntry(code, entry) {
  const text = stripComments(code);
  const at = new RegExp(`fn\\s+${entry.replace(/[^\w]/g, "")}\\s*\\(`).exec(text);
  if (!at) return false;
  // attributes between the previous declaration and `fn entry(`
  const before = text.slice(0, at.index);
  const cut = Math.max(before.lastIndexOf("}"), before.lastIndexOf(";"));
  return /@compute\b/.test(before.slice(cut + 1));
}

function describeBindings(bs) {
  return bs.map((b) => `${b.binding}:${b.name}<${b.space}${b.access ? "," + b.access : ""}>`).join(" ");
}

/**
 * The interface (one of INTERFACES) that `code`'s entry point `entry`
 * declares, or an UnsupportedPipelineError naming what was found.
 */
export function recognise(code, entry = "main") {
  if (typeof code !== "string") throw new TypeError("pipelineFor: code must be WGSL source text");
  if (!hasComputeEntry(code, entry)) {
    throw new UnsupportedPipelineError(`resident pipeline is not valid: no @compute entry point "${entry}"`);
  }
  const bs = parseBindings(code);
  for (const iface of INTERFACES) {
    if (bs.length !== iface.bindings.length) continue;
    const same = iface.bindings.every(([name, space, access, elem], i) => {
      const b = bs[i];
      if (b.binding !== i || b.name !== name || b.space !== space) return false;
      if (space === "storage") return b.access === access && b.type === `array<${elem}>`;
      const fields = parseStruct(code, b.type);
      return fields !== null && fields.length === iface.params.length &&
        fields.every(([n, t], j) => n === iface.params[j][0] && t === iface.params[j][1]);
    });
    if (same) return iface;
  }
  throw new UnsupportedPipelineError(
    `no MI355X kernel for this WGSL entry "${entry}" (bindings ${describeBindings(bs) || "none"}); this device runs ` +
    INTERFACES.map((i) => `${i.op} (${i.source})`).join(", "));
}

/**
 * A uniform's bytes from [type, value] fields, 4 bytes each, little-endian,
 * at least 16 bytes: the layout the reference's harness/wgsl.ts:324-333
 * params() writes and its kernels' Params structs read.
 */
export function params(fields) {
  const buffer = new ArrayBuffer(Math.max(16, fields.length * 4));
  const view = new DataView(buffer);
  fields.forEach(([kind, value], index) => {
    if (kind === "f32") view.setFloat32(index * 4, value, true);
    else if (kind === "i32") view.setInt32(index * 4, value, true);
    else view.setUint32(index * 4, value, true);
  });
  return buffer;
}
