// Minimal test runner (no top-level await: Node 12) for the Node-side suites (the image has node but no
// vitest).  Usage: node tests/node/run.mjs cpu|gpu
//   cpu: tests that need no GPU; GPU tests are listed as skipped, visibly.
//   gpu: only the GPU tests.
// Prints one line per test and a summary; exit code 1 on any failure.
import { pathToFileURL } from "url";
import { dirname, join } from "path";
import { fileURLToPath } from "url";
import { readdirSync } from "fs";
import { Skip } from "./harness.mjs";

const mode = process.argv[2] || "cpu";
const here = dirname(fileURLToPath(import.meta.url));
const registry = [];
globalThis.__wxoTests = registry;

async function main() {
const files = readdirSync(here).filter((f) => f.endsWith(".test.mjs")).sort();
for (const f of files) await import(pathToFileURL(join(here, f)).href);

let passed = 0, failed = 0, skipped = 0;
for (const t of registry) {
  const wanted = mode === "gpu" ? t.gpu : true;
  if (!wanted) continue;
  if (t.gpu && mode !== "gpu") {
    skipped += 1;
    console.log(`SKIP ${t.file} > ${t.name} (needs a gfx950 GPU)`);
    continue;
  }
  try {
    await t.fn();
    passed += 1;
    console.log(`PASS ${t.file} > ${t.name}`);
  } catch (e) {
    if (e instanceof Skip) {
      skipped += 1;
      console.log(`SKIP ${t.file} > ${t.name} (${e.message})`);
      continue;
    }
    failed += 1;
    console.log(`FAIL ${t.file} > ${t.name}\n  ${e && e.stack ? e.stack.split("\n").slice(0, 4).join("\n  ") : e}`);
  }
}
console.log(`node ${mode}: ${passed} passed, ${failed} failed, ${skipped} skipped`);
process.exit(failed ? 1 : 0);
}

main().catch((e) => {
  console.log(`runner error: ${e && e.stack ? e.stack : e}`);
  process.exit(1);
});
