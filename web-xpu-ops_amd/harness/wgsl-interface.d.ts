export declare class UnsupportedPipelineError extends Error {
  readonly name: "UnsupportedPipelineError";
}
export interface WgslInterface {
  readonly op: "matvecQ8" | "matvecQ8Ffn" | "matvecQ8Residual" | "matmulQ8";
  readonly source: string;
  readonly bindings: readonly [string, "storage" | "uniform", "read" | "read_write" | null, string | null][];
  readonly params: readonly [string, string][];
}
export declare const INTERFACES: readonly WgslInterface[];
export declare function parseBindings(code: string): { binding: number; space: string; access: string | null; name: string; type: string }[];
export declare function parseStruct(code: string, name: string): [string, string][] | null;
export declare function recognise(code: string, entry?: string): WgslInterface;
export declare function params(fields: ["u32" | "i32" | "f32", number][]): ArrayBuffer;
