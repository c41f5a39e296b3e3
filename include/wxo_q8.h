/*
 * wxo_q8.h -- C ABI of the MI355X (gfx950) matvecQ8 path.
 *
 * A drop-in backend for web-xpu-ops' W8A32 GEMV and the quantize/packQ8 steps
 * that produce its operands.  Plain C: no HIP, torch or C++ types cross this
 * boundary, so a Node-API addon (gcc), ctypes or any other FFI binds it
 * directly.  Entry points and the reference interface each one replaces:
 *
 *   wxo_matvec_q8             ops/matvec/reference.ts:117-131 (matvecQ8) and the
 *                             WGSL dispatch it backs: ops/matvec/wgsl/q8.wgsl:26-35
 *                             bindings {weight, scale, vector, output, {N,K}},
 *                             called from llm/kernels.ts:195-211 (runMatVecQ8) and
 *                             llm/engine-q8-resident.ts:1843-1845, :1869
 *                             M > 1: M independent matvecQ8 calls on one weight
 *   wxo_matvec_q8_multi       several consecutive matvecQ8 dispatches on one vector, as
 *                             the resident decode issues them: wq/wk/wv at
 *                             llm/engine-q8-resident.ts:1843-1845 and the lm_head
 *                             chunks at :1869 (each a q8.wgsl dispatch); one launch
 *                             for up to 4 projections (no single reference function)
 *   wxo_matvec_q8_residual    ops/matvec/reference.ts:235-243 (matvecQ8Residual) and
 *                             its WGSL form ops/matvec/wgsl/q8_residual.wgsl, used for
 *                             o_proj / down_proj at llm/engine-q8-resident.ts:1857, :1866
 *   wxo_matvec_q8_ffn         ops/matvec/reference.ts:196-207 (matvecQ8Ffn) and
 *                             ops/matvec/wgsl/q8_ffn.wgsl, the gate/up projection at
 *                             llm/engine-q8-resident.ts:1863
 *   wxo_quantize              ops/quantize/reference.ts:13-38 (quantize)
 *   wxo_pack_q8               ops/matvec/reference.ts:267-283 (packQ8)
 *   wxo_pack_int8_rows        llm/weights-q8.ts:137-139 (packInt8Rows)
 *   wxo_quantize_pack_q8      packQ8(quantize(w).output, N, K) + quantize(w).scales
 *                             in one pass (the composition at ops/matvec/reference.ts:87-90)
 *   wxo_quantize_pack_q8_multi  several consecutive quantize+packQ8 of matrices with one
 *                             K in one launch (no single reference function; each
 *                             matrix is wxo_quantize_pack_q8's result)
 *   wxo_matmul_q8             ops/matmul/reference.ts:124-137 (matmulQ8, the prefill
 *                             GEMM over the same packed weight) and its WGSL dispatch
 *                             ops/matmul/wgsl/q8.wgsl:26-35 bindings {a, weight, scale,
 *                             output, {N,M,K}}, called from llm/engine-q8-resident.ts:1078
 *                             (runPrefillResident's projections)
 *   wxo_dequantize_packed_q8  llm/weights-q8.ts:161-177 (dequantizePackedQ8)
 *   wxo_dequant_transpose     ops/dequant_transpose/reference.ts:40-59 (dequantTranspose)
 *   wxo_gather_dequant_rows   llm/weights-q8.ts:207-222 (gatherDequantRows, the
 *                             embedding gather of llm/engine-q8-resident.ts before decode)
 *   wxo_*_host                the same ops on host arrays, synchronous: the TS op
 *                             API's calling convention (typed arrays in, fresh
 *                             typed arrays out)
 *   wxo_malloc/free/memcpy/   device buffers for resident weights:
 *   stream/event              harness/resident.ts:98-145 (createStorageBuffer,
 *                             upload, batch, readback) and harness/wgsl.ts:37-52 (time)
 *
 * Data formats (identical to the reference's wire format):
 *   weight  u32 [N, ceil(K/4)] row-major; code 4w+l of a row in bits 8l..8l+7
 *           of word w (least-significant byte first), two's complement; pad
 *           lanes past K are never read by wxo_matvec_q8 and written as 0 by
 *           the pack entry points.
 *   scale   f32 [N], applied once per row after the dot product.
 *   vector  f32 [M, K] row-major (M = 1 for plain matvecQ8); output f32 [M, N].
 *
 * Errors: every entry point returns a wxo_status; nothing throws or aborts
 * across the ABI.  On failure wxo_last_error() gives a message for the calling
 * thread.  Unlike the reference (which reads `undefined` -> NaN on short
 * inputs), sizes are validated: N*ceil(K/4), M*K etc. must fit in 2^40
 * elements, M must be >= 1, and non-empty operands need non-NULL pointers.
 *
 * Streams: wxo_stream_t is a HIP stream (hipStream_t); NULL means the device's
 * null stream.  Device entry points are asynchronous on that stream and
 * allocate nothing; *_host entry points are synchronous and copy in and out.
 */
#ifndef WXO_Q8_H
#define WXO_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WXO_ABI_VERSION 1

typedef enum wxo_status {
    WXO_OK = 0,
    WXO_ERR_INVALID = 1,   /* bad argument: sizes, NULL pointers, overflow */
    WXO_ERR_NO_DEVICE = 2, /* no gfx950 GPU visible, or HIP runtime unusable */
    WXO_ERR_DEVICE = 3,    /* a HIP call failed (launch, copy, sync) */
    WXO_ERR_OOM = 4        /* device allocation failed */
} wxo_status;

typedef struct wxo_stream_opaque* wxo_stream_t; /* hipStream_t */
typedef struct wxo_event_opaque* wxo_event_t;   /* hipEvent_t */
typedef struct wxo_graph_opaque* wxo_graph_t;   /* hipGraphExec_t */

/* ---- library / device ---------------------------------------------------- */
int wxo_abi_version(void);
/* Message for the last failing call on this thread ("" if none). */
const char* wxo_last_error(void);
/* The kernel instance the calling thread's last successful op launched, e.g.
 * "matvec_q8_m1 xreg waves=4 rows=16 slots=1 vectors=1 grid=688x1" ("" before
 * any op; "none empty" when the op had nothing to do).  The reference resolves
 * its kernel variant explicitly and says which it picked (harness/resolve.ts:211
 * resolve(), harness/target.ts:74-93 detectTarget()); here the choice is made per
 * call from the shape, and this reports it.  Thread-local; valid until the
 * thread's next call. */
const char* wxo_last_variant(void);
/* Initialises the HIP runtime on the current device and checks it is gfx950. */
int wxo_init(void);
/* One line: device name, arch, CU count, HBM size, library build, kernels, and
 * the calling thread's last variant (last="..."). */
const char* wxo_describe(void);
int wxo_device_count(int* count);
int wxo_set_device(int ordinal);

/* ---- memory, streams, events ---------------------------------------------- */
int wxo_malloc(void** ptr, size_t bytes);
int wxo_free(void* ptr);
int wxo_memcpy_htod(void* dst, const void* src, size_t bytes, wxo_stream_t stream);
int wxo_memcpy_dtoh(void* dst, const void* src, size_t bytes, wxo_stream_t stream);
/* Sets `bytes` bytes at the device address `ptr` to (value & 0xff), on
 * `stream`, with a fill kernel (so it may be captured into a HIP graph).  No
 * counterpart in the reference: WebGPU hands out zero-filled buffers, which the
 * engine relies on (llm/engine-q8-resident.ts:1103-1110, :1424), and the
 * resident device clears every new storage buffer with this. */
int wxo_memset(void* ptr, int value, size_t bytes, wxo_stream_t stream);
int wxo_memcpy_dtod(void* dst, const void* src, size_t bytes, wxo_stream_t stream);
/* wxo_memcpy_htod / wxo_memcpy_dtoh return once the copy is done (their stream
 * synchronised).  wxo_memcpy_dtoh_async only enqueues the copy on `stream`,
 * after the work already there: with `dst` from wxo_host_malloc the host
 * thread does not wait, and the bytes are in `dst` once an event recorded
 * after it on `stream` has completed.  This is the resident batch's readback
 * (harness/resident.ts:321-345: copyBufferToBuffer into the caller's MAP_READ
 * staging buffer inside the batch's one submit, then mapAsync). */
int wxo_memcpy_dtoh_async(void* dst, const void* src, size_t bytes, wxo_stream_t stream);
/* Page-locked host memory, the counterpart of a WebGPU MAP_READ | COPY_DST
 * staging buffer (harness/resident.ts:41-48): device-to-host copies into it
 * run asynchronously on their stream.  bytes = 0 gives NULL.  Freeing NULL is
 * a no-op. */
int wxo_host_malloc(void** ptr, size_t bytes);
int wxo_host_free(void* ptr);
int wxo_synchronize(void);
int wxo_stream_create(wxo_stream_t* stream);
int wxo_stream_destroy(wxo_stream_t stream);
int wxo_stream_synchronize(wxo_stream_t stream);
int wxo_event_create(wxo_event_t* event);
/* An event for timing only: recording it performs no system-scope memory
 * fence (no cache write-back or invalidation around the timed work, which
 * otherwise lands inside a short timed interval).  Synchronising on it still
 * waits for the work before it; it does not make device writes visible to the
 * host (copies do that).  The reference times with GPU timestamp queries
 * inside its passes (harness/wgsl.ts:37-52, harness/resident.ts:75-96). */
int wxo_event_create_timer(wxo_event_t* event);
int wxo_event_destroy(wxo_event_t event);
int wxo_event_record(wxo_event_t event, wxo_stream_t stream);
int wxo_event_synchronize(wxo_event_t event);
int wxo_event_elapsed_ms(float* ms, wxo_event_t start, wxo_event_t stop);
/* A one-wave kernel on `stream` that returns after `us` microseconds of the
 * GPU's constant 100 MHz clock (us <= 1,000,000, else WXO_ERR_INVALID).  A
 * measurement aid with no counterpart in the reference: launches enqueued
 * behind it are all queued by the time the GPU reaches them, so events around
 * them time back-to-back execution rather than the host's issue rate. */
int wxo_spin(uint32_t us, wxo_stream_t stream);
/* Holds `stream` until wxo_gate_release(*gate) or until `max_us` microseconds
 * of the GPU's 100 MHz clock have passed (max_us <= 1,000,000, else
 * WXO_ERR_INVALID), whichever comes first: a one-wave kernel polls a flag in
 * page-locked, coherent host memory.  A measurement aid with no counterpart in
 * the reference, whose timestamps sit inside one submit
 * (harness/resident.ts:75-96): work enqueued behind a held gate runs back to
 * back once it opens, so events around that work time the GPU, not the host's
 * issue rate.  Gates are numbered in order; releasing one also opens every
 * gate held before it. */
int wxo_gate_hold(uint32_t max_us, wxo_stream_t stream, uint32_t* gate);
int wxo_gate_release(uint32_t gate);
/* This device's own ceilings, measured now; replaces measureRoofline
 * (harness/roofline.ts:162-198, the same method).  *bandwidth: the best
 * sustained read rate from HBM in bytes/s -- two 512 MiB buffers filled with
 * hashed words, swept once per launch with dwordx4 loads, alternately (each
 * sweep's data was last read 512 MiB earlier, so none comes from the 256 MB
 * Infinity Cache), fastest of three timed regions of eight back-to-back sweeps,
 * each sweep's launch cost included.  *compute: the best sustained one-wide
 * f32 FMA rate in flop/s (an FMA counts 2).  Either pointer may be NULL to skip
 * that part, not both.  Synchronous; allocates and frees 1 GiB of device
 * memory and a stream of its own; takes tens of milliseconds.  A measurement
 * aid: ops are reported as a fraction of it beside the nominal 8 TB/s. */
int wxo_roofline(double* bandwidth, double* compute);
/* The best sustained rate of the bf16 matrix cores (v_mfma_f32_16x16x32_bf16)
 * in flop/s, on every CU with two waves per SIMD (as matmulQ8 runs them), over
 * operands of matmulQ8's own kinds (int8 codes against bf16 parts of random
 * sign, mantissa and exponent).  No counterpart in the reference, whose
 * roofline measures HBM and f32 FMA only; a measurement aid like
 * wxo_roofline: the clock sags under matrix work by how much the operands'
 * bits toggle, so the nominal 2.5 PFLOP/s is not what real operands get.
 * Synchronous; allocates and frees 1 MiB of device memory and a stream of its
 * own; takes a few milliseconds. */
int wxo_roofline_matrix(double* flops);

/* ---- captured batches ------------------------------------------------------
 * The reference encodes a resident batch's passes into one command encoder
 * and submits it once (harness/resident.ts:231-382, one submit per decode
 * step).  Here the same batch is captured once as a HIP graph and replayed:
 * one launch call per step instead of one per op.
 *
 * wxo_graph_capture_begin: from now on, the calling thread's work on `stream`
 *   (not NULL) is recorded, not run.  Thread-local capture mode: a call of
 *   this thread that cannot be recorded fails instead of running early.
 * wxo_graph_capture_end: ends the capture and instantiates it into *graph.  On
 *   any failure the capture is closed anyway and *graph is NULL.
 * wxo_graph_launch: runs the graph on `stream` (the kernels read their buffers
 *   when they run, so buffers keep their addresses and may change contents).
 * wxo_graph_destroy: frees it (NULL is a no-op).
 * No op of this library records a memset node. */
int wxo_graph_capture_begin(wxo_stream_t stream);
int wxo_graph_capture_end(wxo_stream_t stream, wxo_graph_t* graph);
int wxo_graph_launch(wxo_graph_t graph, wxo_stream_t stream);
int wxo_graph_destroy(wxo_graph_t graph);

/* ---- ops on device pointers (asynchronous on `stream`) --------------------- */

/* output[m*N + n] = (sum_{k<K} sext8(byte k of row n) * vector[m*K + k]) * scale[n]
 * for m < M, n < N.  f32 accumulation; |y - y_ref| <= 1e-5 * sum_k|s q x| + 1e-7
 * against the reference's f64 sum. */
int wxo_matvec_q8(const uint32_t* weight, const float* scale, const float* vector, float* output,
                  uint32_t N, uint32_t K, uint32_t M, wxo_stream_t stream);

/* Several projections of one vector: for p < count, outputs[p][n] =
 * matvecQ8(weights[p], scales[p], vector, Ns[p], K)[n], exactly what count
 * wxo_matvec_q8 calls with M = 1 would write (same kernel body, same
 * tolerance).  The arrays of pointers and row counts are host memory; the
 * operands are device memory.  Up to 4 projections share one launch (more
 * are run 4 at a time).  Outputs run concurrently, so an output that
 * overlaps the vector or another output is rejected.  A projection with
 * Ns[p] = 0 is skipped. */
int wxo_matvec_q8_multi(const uint32_t* const* weights, const float* const* scales,
                        float* const* outputs, const uint32_t* Ns, uint32_t count,
                        const float* vector, uint32_t K, wxo_stream_t stream);

/* matvecQ8Residual: output[n] = residual[n] + (matvecQ8 row n), the sum rounded
 * to f32 after the scaled dot product is (two roundings, as the reference).
 * M = 1.  output may be the residual buffer itself. */
int wxo_matvec_q8_residual(const uint32_t* weight, const float* scale, const float* vector,
                           const float* residual, float* output, uint32_t N, uint32_t K,
                           wxo_stream_t stream);

/* matvecQ8Ffn: output[n] = silu(g[n]) * u[n] with g, u the matvecQ8 rows of the
 * gate and up weights (same shape, same vector); silu(g) = g / (1 + e^-g)
 * evaluated in f64 and rounded to f32, then one f32 product.  Both weights are
 * streamed in one pass.  M = 1. */
int wxo_matvec_q8_ffn(const uint32_t* weight_gate, const float* scale_gate, const uint32_t* weight_up,
                      const float* scale_up, const float* vector, float* output, uint32_t N, uint32_t K,
                      wxo_stream_t stream);

/* Per-row absmax quantization, bit-exact to ops/quantize/reference.ts:13-38:
 * output int32 [N, D] codes in [-127, 127], scales f32 [N]. */
int wxo_quantize(const float* input, uint32_t N, uint32_t D, int32_t* output, float* scales,
                 wxo_stream_t stream);

/* packQ8: int32 codes [N, K] -> u32 [N, ceil(K/4)], each code taken & 0xff. */
int wxo_pack_q8(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed, wxo_stream_t stream);

/* packInt8Rows: int8 codes [N, K] -> u32 [N, ceil(K/4)]. */
int wxo_pack_int8_rows(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed,
                       wxo_stream_t stream);

/* quantize + packQ8 in one pass: f32 [N, K] -> packed u32 [N, ceil(K/4)] and
 * scales f32 [N]; bit-exact to packQ8(quantize(w).output, N, K). */
int wxo_quantize_pack_q8(const float* input, uint32_t N, uint32_t K, uint32_t* packed, float* scales,
                         wxo_stream_t stream);

/* quantize+packQ8 of several matrices with the same row length K: matrix p
 * (inputs[p] f32 [Ns[p], K]) gets packed[p] u32 [Ns[p], ceil(K/4)] and
 * scales[p] f32 [Ns[p]], bit-exact to wxo_quantize_pack_q8 on it alone.  The
 * arrays of pointers and row counts are host memory.  Up to 8 matrices share
 * one launch (more run 8 at a time); the matrices run concurrently, so an
 * output that overlaps any input or another output is rejected. */
int wxo_quantize_pack_q8_multi(const float* const* inputs, const uint32_t* Ns, uint32_t* const* packed,
                               float* const* scales, uint32_t count, uint32_t K, wxo_stream_t stream);

/* matmulQ8: output[n*M + m] = (sum_{k<K} a[n*K + k] * sext8(byte k of weight row m)) * scale[m]
 * for n < N (tokens), m < M (weight rows).  a f32 [N, K], weight u32 [M, ceil(K/4)],
 * scale f32 [M], output f32 [N, M].  f32 accumulation on the matrix cores (exact
 * products); |y - y_ref| <= 1e-5 * sum_k |a * q * s| + 1e-7 against the reference's f64
 * sum of per-term dequantized products.  K = 0 gives zeros.  K <= 2^22. */
int wxo_matmul_q8(const float* a, const uint32_t* weight, const float* scale, float* output, uint32_t N,
                  uint32_t M, uint32_t K, wxo_stream_t stream);
/* matmulQ8 of several weights on the same activations a [N, K]: outputs[p]
 * f32 [N, Ms[p]] = wxo_matmul_q8(a, weights[p], scales[p], N, Ms[p], K), in one
 * launch per 4 projections (their tiles shared out together: a prompt's q, k, v
 * or gate and up).  The reference issues one matmulQ8 dispatch per
 * projection (ops/matmul/reference.ts:124-137 per call); results are within the
 * same bound of it, not bit-equal to the single calls (the tile shape follows
 * the launch's total work).  The arrays are host memory; outputs must not
 * overlap a, each other, or any weight or scale. */
int wxo_matmul_q8_multi(const float* a, const uint32_t* const* weights, const float* const* scales,
                        float* const* outputs, const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K,
                        wxo_stream_t stream);
/* wxo_matmul_q8_multi with a caller-owned workspace: device memory of
 * workspace_bytes (16-byte aligned) that touches no input or output.  No
 * counterpart in the reference, which has no workspace.  With room in it,
 * some tiles split their K steps between workgroups whose partial sums meet in
 * a second launch (added in a fixed order: deterministic, and within the same
 * bound of the reference): all of a short prompt's tiles, which would leave
 * most CUs idle, and the last tiles of a prompt whose tiles fill one round of
 * the CUs unevenly, so that every CU holds the same work.  wxo_matmul_q8_workspace_bytes gives the size that allows every
 * split on the current device; less (or NULL and 0) allows fewer splits or
 * none, never an error.  The workspace's contents are scratch between calls;
 * calls that share one workspace must not overlap in time. */
int wxo_matmul_q8_multi_ws(const float* a, const uint32_t* const* weights, const float* const* scales,
                           float* const* outputs, const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K,
                           void* workspace, size_t workspace_bytes, wxo_stream_t stream);
int wxo_matmul_q8_workspace_bytes(size_t* bytes);
/* wxo_matmul_q8_multi_ws with the library's own workspace instead of one the
 * caller passes: no counterpart in the reference.  For callers that cannot
 * allocate device memory at all (code under HIP graph capture, serving loops
 * or harnesses that forbid hipMalloc): it allocates nothing and calls no
 * allocating routine.  The workspace is a 16 MiB array in the library's code
 * object (each GPU holds its own from the library's load until the process
 * ends); a split that would need more runs with fewer parts, so no size is
 * refused for it.  The array keeps the last call's contents and needs no
 * clearing (a call reads only what it wrote).  Every call on one GPU shares
 * that GPU's array: calls that overlap in time on one GPU (other streams,
 * other threads) race and give wrong results. */
int wxo_matmul_q8_multi_static(const float* a, const uint32_t* const* weights, const float* const* scales,
                               float* const* outputs, const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K,
                               wxo_stream_t stream);

/* dequantizePackedQ8: output f32 [N, K], output[n*K + k] = q[n, k] * scale[n] rounded to
 * f32 once (bit-exact to the reference). */
int wxo_dequantize_packed_q8(const uint32_t* weight, const float* scale, uint32_t N, uint32_t K, float* output,
                             wxo_stream_t stream);

/* dequantTranspose: output f32 [in_features, out_features],
 * output[k*out_features + n] = q[n, k] * scale[n] (bit-exact). */
int wxo_dequant_transpose(const uint32_t* weight, const float* scale, uint32_t out_features,
                          uint32_t in_features, float* output, wxo_stream_t stream);

/* gatherDequantRows: codes int8 [rows, D] (the unpacked table), scale f32 [rows],
 * indices int64 [count] -> output f32 [count, D]; row i is codes[indices[i]] * scale
 * (bit-exact), or zeros when indices[i] is outside [0, rows). */
int wxo_gather_dequant_rows(const int8_t* codes, const float* scale, uint32_t rows, uint32_t D,
                            const int64_t* indices, uint32_t count, float* output, wxo_stream_t stream);

/* ---- the same ops on host arrays (synchronous; copy in, run, copy out) ----- */
int wxo_matvec_q8_host(const uint32_t* weight, const float* scale, const float* vector, float* output,
                       uint32_t N, uint32_t K, uint32_t M);
int wxo_matvec_q8_residual_host(const uint32_t* weight, const float* scale, const float* vector,
                                const float* residual, float* output, uint32_t N, uint32_t K);
int wxo_matvec_q8_ffn_host(const uint32_t* weight_gate, const float* scale_gate, const uint32_t* weight_up,
                           const float* scale_up, const float* vector, float* output, uint32_t N, uint32_t K);
int wxo_quantize_host(const float* input, uint32_t N, uint32_t D, int32_t* output, float* scales);
int wxo_pack_q8_host(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed);
int wxo_pack_int8_rows_host(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed);
int wxo_quantize_pack_q8_host(const float* input, uint32_t N, uint32_t K, uint32_t* packed,
                              float* scales);
int wxo_matmul_q8_host(const float* a, const uint32_t* weight, const float* scale, float* output, uint32_t N,
                       uint32_t M, uint32_t K);
int wxo_dequantize_packed_q8_host(const uint32_t* weight, const float* scale, uint32_t N, uint32_t K,
                                  float* output);
int wxo_dequant_transpose_host(const uint32_t* weight, const float* scale, uint32_t out_features,
                               uint32_t in_features, float* output);
int wxo_gather_dequant_rows_host(const int8_t* codes, const float* scale, uint32_t rows, uint32_t D,
                                 const int64_t* indices, uint32_t count, float* output);

#ifdef __cplusplus
}
#endif

#endif /* WXO_Q8_H */
