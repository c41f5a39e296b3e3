// Loads the Node-API addon (lib/wxo_q8.node, built by web-xpu-ops_amd/build.py).
// There is no CPU fallback: a missing addon, a missing HIP runtime or a
// missing gfx950 device surfaces as a thrown Error at the first call.
import { createRequire } from "module";
import { fileURLToPath } from "url";
import { dirname, join } from "path";

const here = dirname(fileURLToPath(import.meta.url));
export const ADDON_PATH = join(here, "..", "lib", "wxo_q8.node");

let addon = null;
let loadError = null;

/** The addon's exports; throws (with the reason) when it cannot be loaded. */
export function native() {
  if (addon) return addon;
  if (loadError) throw loadError;
  try {
    addon = createRequire(import.meta.url)(ADDON_PATH);
  } catch (cause) {
    loadError = new Error(`web-xpu-ops-mi355x: cannot load ${ADDON_PATH} (run web-xpu-ops_amd/build.py); ` +
      `the matvecQ8 path has no CPU fallback: ${cause.message}`);
    throw loadError;
  }
  return addon;
}

/** Device and build description, e.g. `wxo_q8 abi=1 ... arch=gfx950 cus=256 ...`. */
export function describe() {
  return native().describe();
}
