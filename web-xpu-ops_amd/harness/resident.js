// harness/resident: device-resident buffers and one-sync batches for a decode
// engine -- the MI355X counterpart of the reference's ResidentDevice
// (harness/resident.ts:98-145, createResidentDevice :148, batch :231-382).
//
// It takes the reference's own calls for the ops this build runs:
//   createStorageBuffer(bytes, usage?), createUniformBuffer(bytes),
//   upload(buffer, offset, data), pipelineFor(code, entry?),
//   bindGroup(pipeline, buffers), batch(ops, readback, profile?), destroy(),
//   stats { buffersCreated, pipelinesCreated, submits }, timestampsSupported
// with ops { kind: "dispatch", pipeline, bindGroup, workgroups } and
// { kind: "copy", src, srcOffset, dst, dstOffset, size }, so the engine's
// decode projections (llm/engine-q8-resident.ts:521-538 buildProjection,
// :1059-1067 pipelineFor, :1840-1881 the dispatch list) are built and run
// with the same calls.  pipelineFor recognises the reference WGSL of
// matvecQ8 (q8), matvecQ8Ffn (q8_ffn), matvecQ8Residual (q8_residual) and
// matmulQ8 by their binding declarations (./wgsl-interface.js) and throws
// UnsupportedPipelineError for any other kernel (rmsnorm, rope, attention ...
// are not part of this build).  A dispatch runs the MI355X kernel on the
// bound buffers:
//   q8, q8_ffn, q8_residual  rows = workgroups[0] (the WGSL kernels run one
//                            workgroup per output row, row = workgroup_id.x),
//                            K from the bound {N, K} uniform
//   matmulQ8                 N, M, K from the uniform; the dispatch must cover
//                            the whole [N, M] output (16 x 16 tiles: x over M,
//                            y over N), as the engine's dispatches do
// Buffer sizes are checked before anything is enqueued: where WebGPU's robust
// access would clamp a short buffer, this device throws a RangeError.
//
// It also keeps its native op kinds (matvecQ8 / matvecQ8Ffn /
// matvecQ8Residual / packInt8Rows / quantizePackQ8 / matmulQ8 /
// dequantTranspose / gatherDequantRows with named buffer fields), which the
// loader and the prefill side use.
//
// Buffers: storage buffers are HBM allocations owned by the device and freed
// by destroy(); uniform buffers live in host memory (the kernels take their
// values as arguments when a dispatch is enqueued) and MAP_READ staging
// buffers in page-locked host memory; all count in stats.buffersCreated.  Ops
// are enqueued in order on the device's stream.  batch() enqueues its ops and
// then the copies of `readback` into staging memory, and returns a Promise
// that settles when the GPU has run them: the wait happens off the JS thread
// (the reference's onSubmittedWorkDone + mapAsync, harness/resident.ts:
// 321-345), so the caller's event loop keeps running and the next batch may
// be enqueued behind this one before it finishes.  Batches run in the order
// they were called.  Nothing is allocated in a decode loop's steady state.
//
// Consecutive single-vector matvecQ8 ops (dispatch or native) on the same
// vector and K run as one launch when no op of the run reads what another
// writes (the engine's wq/wk/wv, :1843-1845, and lm_head chunks, :1869).
// Consecutive quantizePackQ8 ops with one K likewise, and consecutive matmulQ8
// ops on the same activations (a prompt's q, k, v; gate and up) run as one
// GEMM launch over their weights.  Results are those of
// the separate ops; only stats.launches changes.  { coalesce: false } turns
// it off; a batch with profile labels runs every op on its own, as the
// reference gives every dispatch its own pass when timing.
//
// One launch per step: the reference records a batch into one command
// encoder and submits it once (harness/resident.ts:231-382).  Here a batch of
// two or more ops that resolves to the same calls as the batch before it
// (same kinds, buffers, sizes and K: a decode loop's steps, new contents in
// the same buffers) is captured as a HIP graph, and replayed for as long as
// the batches keep resolving to those calls; a batch that matches neither
// the graph nor its predecessor runs op by op (a one-off list is never
// captured).  The kernels read their buffers when they run, so uploads
// between steps are seen.  stats.graphsCaptured / stats.graphLaunches count
// them; { graphs: false } issues every launch each time, and a profiled batch
// always does (its events time each op).
import { native } from "../native/index.js";
import { recognise, UnsupportedPipelineError, params } from "./wgsl-interface.js";

export { UnsupportedPipelineError, params };

const TYPED = { f32: Float32Array, i32: Int32Array, u32: Uint32Array };
// How long a profiled batch's gate may hold the GPU if the host has not
// enqueued the batch by then (it opens at once when the host has).
const GATE_MAX_US = 200000;

/** WebGPU's GPUBufferUsage bit values (the spec's), for callers without a WebGPU global. */
export const BufferUsage = Object.freeze({
  MAP_READ: 0x0001, MAP_WRITE: 0x0002, COPY_SRC: 0x0004, COPY_DST: 0x0008, INDEX: 0x0010, VERTEX: 0x0020,
  UNIFORM: 0x0040, STORAGE: 0x0080, INDIRECT: 0x0100, QUERY_RESOLVE: 0x0200,
});

const DEFAULT_USAGE = BufferUsage.STORAGE | BufferUsage.COPY_DST | BufferUsage.COPY_SRC;

export class ResidentQ8Device {
  constructor(options = {}) {
    this.addon = native();
    this.addon.init();
    // Scratch for matmulQ8 on short prompts, whose tiles' K steps are split
    // between workgroups (wxo_matmul_q8_multi_ws): one per device, made here
    // so that no batch allocates.
    this.workspaceBytes = this.addon.matmulQ8WorkspaceBytes();
    this.workspace = this.addon.malloc(this.workspaceBytes);
    this.coalesce = options.coalesce !== false;
    this.graphs = options.graphs !== false;
    // "async": a batch's wait runs off the JS thread; "block": on it (the
    // lowest latency per awaited batch, the event loop held meanwhile)
    if (options.wait !== undefined && options.wait !== "async" && options.wait !== "block") {
      throw new TypeError(`wait must be "async" or "block", got ${options.wait}`);
    }
    this.wait = options.wait || "async";
    this.stats = { buffersCreated: 0, pipelinesCreated: 0, submits: 0, launches: 0, graphsCaptured: 0,
      graphLaunches: 0 };
    this.graph = null;        // the last captured batch: { handle, key, launches }
    this.lastKey = null;      // the previous batch's calls (callKey)
    /** HIP events on the device's stream time every labelled op (BatchProfile). */
    this.timestampsSupported = true;
    this.buffers = new Set();
    this.pipelines = new Map();
    this.pipelineSet = new WeakSet();
    this.groupSet = new WeakSet();
    this.events = [];
    this.inflight = new Set();  // completion promises of batches still running
    this.pendingIssue = null;   // settles when a batch waiting to issue has issued
    this.stagingPool = new Map();  // byte size -> free page-locked buffers for readbacks without staging
  }

  /**
   * A buffer of max(4, bytes) bytes.  With the default usage (or any usage
   * without MAP_READ) an HBM allocation `{ ptr: bigint, size }`; a MAP_READ
   * staging buffer (harness/resident.ts:41-48) is page-locked host memory,
   * which a batch's readback copies into without blocking the host.
   */
  createStorageBuffer(bytes, usage = DEFAULT_USAGE) {
    const size = Math.max(4, bytes);
    if (usage & BufferUsage.MAP_READ) {
      return this.track({ ptr: null, host: new Uint8Array(this.addon.hostAlloc(size)), size, usage, kind: "staging",
        busy: false });
    }
    // WebGPU hands out zero-filled buffers, and the engine relies on it (an
    // all-zero attention mask is never uploaded, llm/engine-q8-resident.ts:
    // 1103-1110, :1424): cleared here, once, before anything else can write it.
    const ptr = this.addon.malloc(size);
    this.addon.zero(ptr, size);
    return this.track({ ptr, size, usage, kind: "storage" });
  }

  /** A uniform buffer of max(16, bytes) bytes, held in host memory (read when a dispatch is enqueued). */
  createUniformBuffer(bytes) {
    const size = Math.max(16, bytes);
    return this.track({ ptr: null, host: new Uint8Array(size), size, usage: BufferUsage.UNIFORM | BufferUsage.COPY_DST,
      kind: "uniform" });
  }

  /**
   * Registers a new buffer and gives it GPUBuffer's destroy(): the memory is
   * released at once (after the batches in flight, which may read it, have
   * run), later calls are no-ops, and any later use
   * of the buffer (upload, a bind group that holds it, an op, a readback)
   * throws.  The engine destroys its transient per-prefill buffers this way
   * (llm/engine-q8-resident.ts:1693), as runnerFromResident does its
   * per-call ones (harness/resident.ts:480-482).
   */
  track(buffer) {
    buffer.destroy = () => {
      if (!this.buffers.delete(buffer)) return;
      if (buffer.ptr !== null && this.inflight.size > 0) this.addon.synchronize();  // a batch in flight may read it
      if (buffer.ptr !== null) this.addon.free(buffer.ptr);
      buffer.ptr = null;
      buffer.host = null;
    };
    this.buffers.add(buffer);
    this.stats.buffersCreated += 1;
    return buffer;
  }

  /** `data` into `buffer` at byte `offset`: a host-to-device copy, or into a host-held buffer. */
  upload(buffer, offset, data) {
    if (!this.buffers.has(buffer)) throw new TypeError("upload: buffer was not created by this device");
    if (offset < 0 || offset + data.byteLength > buffer.size) {
      throw new RangeError(`upload of ${data.byteLength} B at ${offset} overflows a ${buffer.size} B buffer`);
    }
    if (buffer.ptr === null) {
      buffer.host.set(new Uint8Array(data.buffer, data.byteOffset, data.byteLength), offset);
    } else {
      this.addon.upload(buffer.ptr + BigInt(offset), data);
    }
  }

  /**
   * The pipeline for WGSL `code` + `entry` (cached, as harness/resident.ts
   * pipelineFor): one of the interfaces ./wgsl-interface.js recognises, or an
   * UnsupportedPipelineError.
   */
  async pipelineFor(code, entry = "main") {
    const key = `${entry} ${code}`;
    const cached = this.pipelines.get(key);
    if (cached) return cached;
    const iface = recognise(code, entry);
    const pipeline = Object.freeze({ op: iface.op, entry, interface: iface });
    this.pipelines.set(key, pipeline);
    this.pipelineSet.add(pipeline);
    this.stats.pipelinesCreated += 1;
    return pipeline;
  }

  /**
   * A bind group of whole buffers in the pipeline's binding order
   * (harness/resident.ts bindGroup): storage bindings take this device's
   * storage buffers, the uniform binding a uniform buffer.  An output that
   * aliases an input is refused (WebGPU refuses writable aliasing too), except
   * matvecQ8Residual's output over its residual: the in-place residual stream.
   */
  async bindGroup(pipeline, buffers) {
    if (!this.pipelineSet.has(pipeline)) {
      throw new TypeError("resident bind group is not valid: pipeline was not created by this device's pipelineFor");
    }
    const layout = pipeline.interface.bindings;
    if (!Array.isArray(buffers) || buffers.length !== layout.length) {
      throw new Error(`resident bind group is not valid: ${pipeline.op} binds ${layout.length} buffers ` +
        `(${layout.map((b) => b[0]).join(", ")}), got ${Array.isArray(buffers) ? buffers.length : typeof buffers}`);
    }
    layout.forEach(([name, space], i) => {
      const b = buffers[i];
      if (!this.buffers.has(b)) throw new TypeError(`resident bind group is not valid: binding ${i} (${name}) is not a buffer of this device`);
      if (space === "uniform" && b.kind !== "uniform") {
        throw new TypeError(`resident bind group is not valid: binding ${i} (${name}) needs a uniform buffer`);
      }
      if (space === "storage" && b.kind !== "storage") {
        throw new TypeError(`resident bind group is not valid: binding ${i} (${name}) needs a storage buffer`);
      }
    });
    const out = layout.findIndex((b) => b[2] === "read_write");
    layout.forEach(([name, space], i) => {
      if (i === out || space !== "storage") return;
      if (buffers[i] === buffers[out] && !(pipeline.op === "matvecQ8Residual" && name === "residual")) {
        throw new Error(`resident bind group is not valid: ${pipeline.op} output aliases its ${name} binding`);
      }
    });
    const group = Object.freeze({ pipeline, buffers: Object.freeze(buffers.slice()) });
    this.groupSet.add(group);
    return group;
  }

  /**
   * Enqueues every op in order, then the copies of `readback` ({ staging?,
   * source, sourceOffset, length, type }) into page-locked staging memory
   * (the caller's MAP_READ staging buffer when given, sized for length * 4
   * bytes, else a pooled one), and resolves to fresh typed arrays of the read
   * values once the GPU has run all of it.  Every op is checked before the
   * first is enqueued.  The wait runs off the JS thread; a batch called while
   * another is in flight is enqueued behind it at once, except that a batch
   * that captures a graph, or carries profile labels, first waits for the
   * batches in flight.  A staging buffer that an unfinished batch is reading
   * back into is refused, as WebGPU refuses a buffer with a pending map.
   * `profile` ({ labels?, sink }) as harness/resident.ts:75-96:
   * sink.submitToDoneMs (enqueue end to completion, the device-to-host copies
   * included), sink.readbackMs (the copies out of staging), and with labels
   * sink.gpuEntries [{ label, seconds }] for each labelled non-copy op, from
   * HIP events around its launch.  A labelled batch is held on the GPU until
   * it is all enqueued (wxo_gate_hold), so those intervals are the ops' GPU
   * time back to back, not the host's issue rate.
   */
  async batch(ops, readback = [], profile = undefined) {
    // Batches issue in call order: while one waits for the batches in flight
    // (below), the ones called after it wait for it to issue.
    while (this.pendingIssue) await this.pendingIssue;
    let calls = ops.map((op, i) => this.resolve(op, i));
    let reads = readback.map((r) => checkReadback(r, this.buffers));
    const labels = profile && profile.labels ? profile.labels : null;
    const coalesce = this.coalesce && !labels;
    const graphed = this.graphs && !labels && calls.length > 1;
    let key = graphed ? callKey(calls, coalesce) : null;  // built once per batch (132 ops: ~6 us)
    if ((labels || (graphed && this.wouldCapture(key))) && this.inflight.size > 0) {
      let release;
      this.pendingIssue = new Promise((r) => { release = r; });
      try {
        await this.idle();
        // checked again: a buffer may have been destroyed meanwhile
        calls = ops.map((op, i) => this.resolve(op, i));
        reads = readback.map((r) => checkReadback(r, this.buffers));
        if (graphed) key = callKey(calls, coalesce);
      } finally {
        this.pendingIssue = null;
        release();
      }
    }
    const targets = this.stagingTargets(reads);
    const a = this.addon;
    const timed = [];
    let done;
    try {
      // A labelled batch runs behind a gate that opens once all of it is
      // enqueued, so its ops run back to back and each op's interval is GPU
      // time, as timestamps inside one submit are (not the host's issue rate).
      const gate = labels ? a.gateHold(GATE_MAX_US) : 0;
      try {
        if (!(graphed && this.replay(calls, coalesce, key))) this.enqueue(calls, coalesce, labels, timed);
      } finally {
        if (labels) a.gateRelease(gate);
      }
      reads.forEach((r, k) => a.downloadAsync(r.source.ptr + BigInt(r.sourceOffset), targets[k].view));
      if (this.wait === "block") {
        a.synchronize();
        done = Promise.resolve();
      } else {
        done = a.whenDone();
      }
    } catch (err) {
      this.releaseStaging(targets);
      throw err;
    }
    this.stats.submits += 1;
    const t0 = profile ? performanceNow() : 0;
    this.inflight.add(done);
    let results, t1 = 0;
    try {
      await done;
      if (profile) profile.sink.submitToDoneMs = performanceNow() - t0;
      t1 = profile ? performanceNow() : 0;
      results = reads.map((r, k) => new TYPED[r.type](targets[k].view.slice(0, r.length * 4).buffer));
    } finally {
      this.inflight.delete(done);
      this.releaseStaging(targets);
    }
    if (profile) {
      profile.sink.readbackMs = performanceNow() - t1;
      if (labels) {
        const entries = [];
        for (const t of timed) {
          const ms = a.eventElapsedMs(t.events[0], t.events[1]);
          if (ms > 0) entries.push({ label: t.label, seconds: ms / 1e3 });
        }
        profile.sink.gpuEntries = entries;
      }
    }
    return results;
  }

  /** Settles once every batch in flight has (their failures are theirs to report). */
  async idle() {
    while (this.inflight.size > 0) await Promise.allSettled([...this.inflight]);
  }

  /**
   * Where each readback lands: { view, staging?, pooled? }, `view` a
   * Uint8Array over page-locked memory.  Taken before anything is enqueued;
   * released when the batch settles.
   */
  stagingTargets(reads) {
    const targets = [];
    try {
      for (const r of reads) {
        const bytes = r.length * 4;
        const st = r.staging;
        if (st !== undefined && st !== null && this.buffers.has(st) && st.kind === "staging") {
          if (st.size < bytes) throw new RangeError(`readback staging buffer holds ${st.size} B, ${bytes} needed`);
          if (st.busy) throw new Error("readback staging buffer is in use by a batch that has not finished (a pending map)");
          st.busy = true;
          targets.push({ view: st.host.subarray(0, bytes), staging: st });
        } else {
          const free = this.stagingPool.get(bytes);
          const view = free && free.length ? free.pop() : new Uint8Array(this.addon.hostAlloc(bytes));
          targets.push({ view, pooled: true });
        }
      }
    } catch (err) {
      this.releaseStaging(targets);
      throw err;
    }
    return targets;
  }

  releaseStaging(targets) {
    for (const t of targets) {
      if (t.staging) {
        t.staging.busy = false;
      } else if (t.pooled) {
        const list = this.stagingPool.get(t.view.byteLength) || [];
        list.push(t.view);
        this.stagingPool.set(t.view.byteLength, list);
      }
    }
  }

  /** Enqueues every call (coalesced runs as one launch), with events around labelled ones. */
  enqueue(calls, coalesce, labels, timed) {
    const a = this.addon;
    for (let i = 0; i < calls.length; i += 1) {
      const label = labels && labels[i] != null && calls[i].kind !== "copy" ? labels[i] : null;
      let events = null;
      if (label !== null) {
        events = this.eventPair(timed.length);
        a.eventRecord(events[0]);
      }
      i += this.run(calls, i, coalesce) - 1;
      if (events) {
        a.eventRecord(events[1]);
        timed.push({ label, events });
      }
    }
  }

  /** Whether replay() would capture a new graph for calls of this key (they repeat the previous batch's, not the graph's). */
  wouldCapture(key) {
    const g = this.graph;
    return (g === null || !sameKey(g.key, key)) && this.lastKey !== null && sameKey(this.lastKey, key);
  }

  /**
   * One graph launch for `calls` (whose callKey is `key`) if they match the
   * captured graph, or the previous batch (then captured now); false (nothing
   * enqueued) otherwise.
   */
  replay(calls, coalesce, key) {
    const a = this.addon;
    const g = this.graph;
    const last = this.lastKey;
    this.lastKey = key;
    if (g === null || !sameKey(g.key, key)) {
      if (last === null || !sameKey(last, key)) return false;
      if (g !== null) a.graphDestroy(g.handle);
      this.graph = null;
      const before = this.stats.launches;
      a.graphBegin();
      try {
        this.enqueue(calls, coalesce, null, null);
      } catch (err) {
        // Close the capture and free whatever it instantiated; the error to
        // report is the one the batch raised, not one from closing it.
        try {
          a.graphDestroy(a.graphEnd());
        } catch (_) { /* the capture was already invalid: nothing was instantiated */ }
        throw err;
      }
      const handle = a.graphEnd();
      this.graph = { handle, key, launches: this.stats.launches - before };
      this.stats.graphsCaptured += 1;
    } else {
      this.stats.launches += g.launches;
    }
    a.graphLaunch(this.graph.handle);
    this.stats.graphLaunches += 1;
    return true;
  }

  /** Frees every buffer and event this device created. */
  destroy() {
    if (this.inflight.size > 0) this.addon.synchronize();  // nothing in flight reads what is freed below
    if (this.workspace !== null) {
      this.addon.free(this.workspace);
      this.workspace = null;
    }
    if (this.graph !== null) {
      this.addon.graphDestroy(this.graph.handle);
      this.graph = null;
    }
    for (const b of [...this.buffers]) b.destroy();
    for (const [s, e] of this.events) {
      this.addon.eventDestroy(s);
      this.addon.eventDestroy(e);
    }
    this.events = [];
  }

  eventPair(k) {
    while (this.events.length <= k) this.events.push([this.addon.eventCreate(), this.addon.eventCreate()]);
    return this.events[k];
  }

  /** A checked native call for op `i`: { kind, ...operands } (throws before anything is enqueued). */
  resolve(op, i) {
    if (!op || typeof op !== "object") throw new TypeError(`op ${i} is not an object`);
    switch (op.kind) {
      case "dispatch":
        return this.resolveDispatch(op, i);
      case "copy": {
        for (const [b, name] of [[op.src, "src"], [op.dst, "dst"]]) {
          if (!this.buffers.has(b) || b.kind !== "storage") throw new TypeError(`op ${i}: copy ${name} must be a storage buffer of this device`);
        }
        if (op.srcOffset % 4 || op.dstOffset % 4 || op.size % 4) {
          throw new RangeError(`op ${i}: copy offsets and size must be multiples of 4 bytes`);
        }
        if (op.srcOffset < 0 || op.dstOffset < 0 || op.size < 0 || op.srcOffset + op.size > op.src.size ||
            op.dstOffset + op.size > op.dst.size) {
          throw new RangeError(`op ${i}: copy range outside its buffers`);
        }
        return op;
      }
      case "matvecQ8":
        checkMatvec(op, op.M === undefined ? 1 : op.M);
        return op;
      case "matvecQ8Ffn":
        checkFfn(op);
        return op;
      case "matvecQ8Residual":
        checkResidual(op);
        return op;
      case "packInt8Rows":
        need(op.codes, op.N * op.K, "codes");
        need(op.packed, op.N * Math.ceil(op.K / 4) * 4, "packed");
        return op;
      case "quantizePackQ8":
        checkQuantize(op);
        return op;
      case "matmulQ8":
        checkMatmul(op);
        return op;
      case "dequantTranspose":
        need(op.weight, op.outFeatures * Math.ceil(op.inFeatures / 4) * 4, "weight");
        need(op.scale, op.outFeatures * 4, "scale");
        need(op.output, op.outFeatures * op.inFeatures * 4, "output");
        return op;
      case "gatherDequantRows":
        need(op.codes, op.rows * op.D, "codes");
        need(op.scale, op.rows * 4, "scale");
        need(op.indices, op.count * 8, "indices");
        need(op.output, op.count * op.D * 4, "output");
        return op;
      default:
        throw new TypeError(`unknown resident op kind ${op.kind}`);
    }
  }

  resolveDispatch(op, i) {
    const group = op.bindGroup;
    if (!this.groupSet.has(group)) throw new TypeError(`op ${i}: bindGroup was not created by this device's bindGroup`);
    group.buffers.forEach((b, j) => {
      if (!this.buffers.has(b)) throw new TypeError(`op ${i}: binding ${j} of the bind group was destroyed`);
    });
    if (group.pipeline !== op.pipeline) {
      throw new Error(`op ${i}: bind group was made for the ${group.pipeline.op} pipeline, dispatched with ${op.pipeline && op.pipeline.op}`);
    }
    const wg = op.workgroups;
    if (!Array.isArray(wg) || wg.length < 1 || wg.length > 3 || !wg.every((n) => Number.isInteger(n) && n >= 0)) {
      throw new TypeError(`op ${i}: workgroups must be [x], [x, y] or [x, y, z] of non-negative integers`);
    }
    const [x, y = 1, z = 1] = wg;
    const b = group.buffers;
    const u = new DataView(b[b.length - 1].host.buffer);
    const empty = x === 0 || y === 0 || z === 0;
    switch (op.pipeline.op) {
      case "matvecQ8": {
        const call = { kind: "matvecQ8", weight: b[0], scale: b[1], vector: b[2], output: b[3], N: empty ? 0 : x,
          K: u.getUint32(4, true), M: 1 };
        checkMatvec(call, 1);
        return call;
      }
      case "matvecQ8Ffn": {
        const call = { kind: "matvecQ8Ffn", weightGate: b[0], scaleGate: b[1], weightUp: b[2], scaleUp: b[3],
          vector: b[4], output: b[5], N: empty ? 0 : x, K: u.getUint32(4, true) };
        checkFfn(call);
        return call;
      }
      case "matvecQ8Residual": {
        const call = { kind: "matvecQ8Residual", weight: b[0], scale: b[1], vector: b[2], residual: b[3],
          output: b[4], N: empty ? 0 : x, K: u.getUint32(4, true) };
        checkResidual(call);
        return call;
      }
      case "matmulQ8": {
        const N = u.getUint32(0, true), M = u.getUint32(4, true), K = u.getUint32(8, true);
        if (!empty && (x * 16 < M || y * 16 < N)) {
          throw new RangeError(`op ${i}: matmulQ8 dispatch [${wg}] covers part of the ${N} x ${M} output; ` +
            `this device runs whole outputs ([${Math.ceil(M / 16)}, ${Math.ceil(N / 16)}] workgroups or more)`);
        }
        const call = { kind: "matmulQ8", a: b[0], weight: b[1], scale: b[2], output: b[3], N: empty ? 0 : N, M, K };
        checkMatmul(call);
        return call;
      }
      default:
        throw new UnsupportedPipelineError(`op ${i}: no MI355X kernel for pipeline ${op.pipeline.op}`);
    }
  }

  /** Enqueues call `i` (and any run coalesced with it); returns how many calls it consumed. */
  run(calls, i, coalesce) {
    const a = this.addon;
    const op = calls[i];
    this.stats.launches += 1;
    switch (op.kind) {
      case "matvecQ8": {
        const M = op.M === undefined ? 1 : op.M;
        const n = coalesce && M === 1 ? sameVectorRun(calls, i) : 1;
        if (n > 1) {
          const group = calls.slice(i, i + n);
          a.matvecQ8MultiDevice(group.map((g) => [g.weight.ptr, g.scale.ptr, g.output.ptr, g.N]), op.vector.ptr, op.K);
          return n;
        }
        a.matvecQ8Device(op.weight.ptr, op.scale.ptr, op.vector.ptr, op.output.ptr, op.N, op.K, M);
        return 1;
      }
      case "matvecQ8Ffn":
        a.matvecQ8FfnDevice(op.weightGate.ptr, op.scaleGate.ptr, op.weightUp.ptr, op.scaleUp.ptr, op.vector.ptr,
                            op.output.ptr, op.N, op.K);
        return 1;
      case "matvecQ8Residual":
        a.matvecQ8ResidualDevice(op.weight.ptr, op.scale.ptr, op.vector.ptr, op.residual.ptr, op.output.ptr, op.N,
                                 op.K);
        return 1;
      case "packInt8Rows":
        a.packInt8RowsDevice(op.codes.ptr, op.N, op.K, op.packed.ptr);
        return 1;
      case "quantizePackQ8": {
        const n = coalesce ? quantizeRun(calls, i) : 1;
        if (n > 1) {
          const group = calls.slice(i, i + n);
          a.quantizePackQ8MultiDevice(group.map((g) => [g.input.ptr, g.N, g.packed.ptr, g.scales.ptr]), op.K);
          return n;
        }
        a.quantizePackQ8Device(op.input.ptr, op.N, op.K, op.packed.ptr, op.scales.ptr);
        return 1;
      }
      case "matmulQ8": {
        const n = coalesce ? sameActivationRun(calls, i) : 1;
        const group = calls.slice(i, i + n);
        a.matmulQ8MultiDevice(group.map((g) => [g.weight.ptr, g.scale.ptr, g.output.ptr, g.M]), op.a.ptr, op.N, op.K,
          this.workspace, this.workspaceBytes);
        return n;
      }
      case "dequantTranspose":
        a.dequantTransposeDevice(op.weight.ptr, op.scale.ptr, op.outFeatures, op.inFeatures, op.output.ptr);
        return 1;
      case "gatherDequantRows":
        a.gatherDequantRowsDevice(op.codes.ptr, op.scale.ptr, op.rows, op.D, op.indices.ptr, op.count, op.output.ptr);
        return 1;
      case "copy":
        if (op.size > 0) a.copy(op.dst.ptr + BigInt(op.dstOffset), op.src.ptr + BigInt(op.srcOffset), op.size);
        return 1;
      default:
        throw new TypeError(`unknown resident op kind ${op.kind}`);
    }
  }
}

/**
 * The values that decide what a batch enqueues: every call's kind, its
 * buffers' addresses and its numbers (sizes, K, offsets), in order.
 */
function callKey(calls, coalesce) {
  const key = [coalesce];
  for (const c of calls) {
    for (const k in c) {
      const v = c[k];
      if (typeof v === "number" || typeof v === "string") key.push(v);
      else if (v !== null && typeof v === "object" && typeof v.ptr === "bigint") key.push(v.ptr);
    }
    key.push(null);
  }
  return key;
}

function sameKey(a, b) {
  if (a.length !== b.length) return false;
  for (let i = 0; i < a.length; i += 1) if (a[i] !== b[i]) return false;
  return true;
}

function performanceNow() {
  const [s, ns] = process.hrtime();
  return s * 1e3 + ns / 1e6;
}

function checkReadback(r, owned) {
  const T = TYPED[r.type];
  if (!T) throw new TypeError(`unknown readback type ${r.type}`);
  if (!owned.has(r.source) || r.source.kind !== "storage") throw new TypeError("readback source must be a storage buffer of this device");
  if (r.sourceOffset % 4 || r.sourceOffset < 0 || r.sourceOffset + r.length * 4 > r.source.size) {
    throw new RangeError("readback outside its buffer");
  }
  return r;
}

function checkMatvec(op, M) {
  const W = Math.ceil(op.K / 4);
  need(op.weight, op.N * W * 4, "weight");
  need(op.scale, op.N * 4, "scale");
  need(op.vector, M * op.K * 4, "vector");
  need(op.output, M * op.N * 4, "output");
}

function checkFfn(op) {
  const bytes = op.N * Math.ceil(op.K / 4) * 4;
  need(op.weightGate, bytes, "weightGate");
  need(op.scaleGate, op.N * 4, "scaleGate");
  need(op.weightUp, bytes, "weightUp");
  need(op.scaleUp, op.N * 4, "scaleUp");
  need(op.vector, op.K * 4, "vector");
  need(op.output, op.N * 4, "output");
}

function checkResidual(op) {
  need(op.weight, op.N * Math.ceil(op.K / 4) * 4, "weight");
  need(op.scale, op.N * 4, "scale");
  need(op.vector, op.K * 4, "vector");
  need(op.residual, op.N * 4, "residual");
  need(op.output, op.N * 4, "output");
}

function checkQuantize(op) {
  need(op.input, op.N * op.K * 4, "input");
  need(op.packed, op.N * Math.ceil(op.K / 4) * 4, "packed");
  need(op.scales, op.N * 4, "scales");
}

function checkMatmul(op) {
  need(op.a, op.N * op.K * 4, "a");
  need(op.weight, op.M * Math.ceil(op.K / 4) * 4, "weight");
  need(op.scale, op.M * 4, "scale");
  need(op.output, op.N * op.M * 4, "output");
}

/**
 * How many calls from `start` on (at least 1) form a run of quantizePackQ8
 * calls with the same K, none writing what another of the run reads or writes.
 */
/**
 * How many calls from `start` on (at least 1) form a run of matmulQ8 calls on
 * the same activations (buffer, N, K), none writing the activations or what
 * another of the run reads or writes: a prompt's q, k and v, or gate and up.
 */
function sameActivationRun(calls, start) {
  const first = calls[start];
  const act = span(first.a, first.N * first.K * 4);
  const outs = [];
  const ins = [];
  let n = 0;
  for (let j = start; j < calls.length; j += 1) {
    const op = calls[j];
    if (op.kind !== "matmulQ8" || op.a.ptr !== first.a.ptr || op.N !== first.N || op.K !== first.K) break;
    if (op.N === 0 || op.M === 0) break;
    const out = span(op.output, op.N * op.M * 4);
    const reads = [span(op.weight, op.M * Math.ceil(op.K / 4) * 4), span(op.scale, op.M * 4)];
    if (overlaps(out, act) || outs.some((o) => overlaps(o, out)) ||
        reads.some((r) => outs.some((o) => overlaps(o, r))) || ins.some((r) => overlaps(r, out))) {
      break;
    }
    outs.push(out);
    ins.push(...reads);
    n += 1;
  }
  return Math.max(n, 1);
}

function quantizeRun(calls, start) {
  const K = calls[start].K;
  const ins = [];
  const outs = [];
  let n = 0;
  for (let j = start; j < calls.length; j += 1) {
    const op = calls[j];
    if (op.kind !== "quantizePackQ8" || op.K !== K) break;
    const input = span(op.input, op.N * op.K * 4);
    const own = [span(op.packed, op.N * Math.ceil(op.K / 4) * 4), span(op.scales, op.N * 4)];
    if (overlaps(own[0], own[1]) || own.some((o) => overlaps(o, input) || ins.some((r) => overlaps(o, r)) ||
        outs.some((w) => overlaps(o, w))) || outs.some((w) => overlaps(w, input))) {
      break;
    }
    ins.push(input);
    outs.push(...own);
    n += 1;
  }
  return Math.max(n, 1);
}

/** [start, end) byte range of `bytes` bytes at a resident buffer's address. */
function span(buffer, bytes) {
  return [buffer.ptr, buffer.ptr + BigInt(bytes)];
}

function overlaps(x, y) {
  return x[0] < y[1] && y[0] < x[1] && x[0] < x[1] && y[0] < y[1];
}

/**
 * How many calls from `start` on (at least 1) form a run of single-vector
 * matvecQ8 calls on the same vector and K with no call of the run reading
 * what another writes, so that one launch gives what the calls in order would.
 */
function sameVectorRun(calls, start) {
  const first = calls[start];
  const vec = span(first.vector, first.K * 4);
  const outs = [];
  const ins = [];
  let n = 0;
  for (let j = start; j < calls.length; j += 1) {
    const op = calls[j];
    if (op.kind !== "matvecQ8" || (op.M !== undefined && op.M !== 1)) break;
    if (op.K !== first.K || op.vector.ptr !== first.vector.ptr || op.N === 0) break;
    const out = span(op.output, op.N * 4);
    const reads = [span(op.weight, op.N * Math.ceil(op.K / 4) * 4), span(op.scale, op.N * 4)];
    if (overlaps(out, vec) || outs.some((o) => overlaps(o, out)) ||
        reads.some((r) => outs.some((o) => overlaps(o, r))) || ins.some((r) => overlaps(r, out))) {
      break;
    }
    outs.push(out);
    ins.push(...reads);
    n += 1;
  }
  return Math.max(n, 1);
}

function need(buffer, bytes, name) {
  if (!buffer || typeof buffer.ptr !== "bigint") throw new TypeError(`${name} must be a resident storage buffer`);
  if (bytes > buffer.size) throw new RangeError(`${name} buffer holds ${buffer.size} B, ${bytes} B needed`);
}

/**
 * Resolves to null when no gfx950 device is visible (as harness/resident.ts:148
 * does without an adapter).  Installs `GPUBufferUsage` (the spec's bit
 * values) on globalThis when no WebGPU global provides it, as the reference's
 * createResidentDevice installs the webgpu package's globals, so callers that
 * create staging buffers with `GPUBufferUsage.COPY_DST | GPUBufferUsage.MAP_READ`
 * run unchanged.
 */
export async function createResidentQ8Device(options = {}) {
  const a = native();
  if (a.deviceCount() === 0) return null;
  if (typeof globalThis.GPUBufferUsage === "undefined") globalThis.GPUBufferUsage = BufferUsage;
  return new ResidentQ8Device(options);
}

/** The reference's name for the same factory (harness/resident.ts:148, re-exported by harness/index.ts:5). */
export const createResidentDevice = createResidentQ8Device;

/**
 * harness/resident.ts:429-485: a Runner's run(dispatch) over a resident
 * device, for one-off dispatches.  Each call makes its own buffers (an
 * upload per "storage" and "uniform" binding, an empty buffer per "out" and
 * "scratch" one), binds them in the dispatch's order, runs the one dispatch
 * with a readback of every "out" binding, and destroys every buffer it made,
 * results or not.  The pipeline comes from pipelineFor, so the dispatch's
 * WGSL must be one of the interfaces it recognises.
 */
export function runnerFromResident(device) {
  return async function run(dispatch) {
    const { code, entry = "main", bindings, workgroups } = dispatch;
    const pipeline = await device.pipelineFor(code, entry);
    const made = [];
    const keep = (b) => {
      made.push(b);
      return b;
    };
    try {
      const outs = [];
      const bound = bindings.map((binding) => {
        switch (binding.kind) {
          case "out": {
            const b = keep(device.createStorageBuffer(binding.length * 4));
            outs.push({ buffer: b, length: binding.length, type: binding.type });
            return b;
          }
          case "scratch":
            return keep(device.createStorageBuffer(Math.max(4, binding.length * 4)));
          case "uniform": {
            const b = keep(device.createUniformBuffer(binding.data.byteLength));
            device.upload(b, 0, new Uint8Array(binding.data));
            return b;
          }
          case "storage": {
            const b = keep(device.createStorageBuffer(binding.data.byteLength));
            device.upload(b, 0, binding.data);
            return b;
          }
          default:
            throw new TypeError(`unknown binding kind ${binding.kind}`);
        }
      });
      const bindGroup = await device.bindGroup(pipeline, bound);
      const readback = outs.map((o) => ({
        staging: keep(device.createStorageBuffer(o.length * 4, BufferUsage.COPY_DST | BufferUsage.MAP_READ)),
        source: o.buffer, sourceOffset: 0, length: o.length, type: o.type,
      }));
      return await device.batch([{ kind: "dispatch", pipeline, bindGroup, workgroups }], readback);
    } finally {
      for (const b of made) b.destroy();
    }
  };
}
