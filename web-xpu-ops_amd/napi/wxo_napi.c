/*
 * wxo_napi.c -- Node-API addon over the C ABI in include/wxo_q8.h.
 *
 * Plain C against node_api.h (N-API 8, Node >= 12.22), built by
 * web-xpu-ops_amd/build.py into lib/wxo_q8.node with an $ORIGIN rpath to
 * lib/libwxo_q8.so.  It is the binding the TypeScript op API
 * (ops/matvec, ops/quantize, llm/weights-q8, harness/resident in this
 * package) calls; the reference's own WebGPU binding sits at the same place
 * (harness/wgsl.ts:77-99 createRunner; harness/resident.ts:148).
 *
 * Host-array functions take typed arrays and plain numbers, validate types
 * and lengths before touching the device, and return fresh typed arrays:
 *   matvecQ8(weight: Uint32Array, scale: Float32Array, vector: Float32Array,
 *            N, K, M = 1) -> Float32Array [M*N]
 *   matvecQ8Async(weight, scale, vector, N, K, M = 1) -> Promise<Float32Array [M*N]>
 *            (the same call on a libuv worker thread; scale and vector are
 *            copied when it is made, the weight is read while it is pending)
 *   quantize(input: Float32Array, N, D) -> { output: Int32Array, scales: Float32Array }
 *   packQ8(codes: Int32Array, N, K) -> Uint32Array
 *   packInt8Rows(codes: Int8Array, N, K) -> Uint32Array
 *   quantizePackQ8(input: Float32Array, N, K) -> { weight: Uint32Array, scale: Float32Array }
 *   matmulQ8(a: Float32Array, weight: Uint32Array, scale: Float32Array, N, M, K) -> Float32Array [N*M]
 *   dequantizePackedQ8(weight, scale, N, K) -> Float32Array [N*K]
 *   dequantTranspose(weight, scale, outFeatures, inFeatures) -> Float32Array [inF*outF]
 *   gatherDequantRows(codes: Int8Array, scale: Float32Array, indices, D) -> Float32Array
 * Device-resident functions take BigInt device addresses (from malloc):
 *   malloc(bytes) -> bigint, free(ptr), upload(ptr, typedArray),
 *   download(ptr, typedArray), copy(dst, src, bytes), synchronize(),
 *   matvecQ8Device(w, s, x, y, N, K, M), quantizeDevice(in, N, D, out, scales),
 *   packQ8Device(codes, N, K, packed), packInt8RowsDevice(codes, N, K, packed),
 *   quantizePackQ8Device(in, N, K, packed, scales), matmulQ8Device(a, w, s, y, N, M, K),
 *   matmulQ8MultiDevice([[w, s, y, M], ...], a, N, K),
 *   dequantizePackedQ8Device(w, s, N, K, y), dequantTransposeDevice(w, s, outF, inF, y),
 *   gatherDequantRowsDevice(codes, s, rows, D, indices, count, y)
 *   lastVariant() -> string (wxo_last_variant: the kernel instance of the last op)
 *   eventCreate() -> bigint, eventRecord(ev), eventElapsedMs(start, stop), eventDestroy(ev)
 *   graphBegin(), graphEnd() -> bigint, graphLaunch(graph), graphDestroy(graph)
 *   hostAlloc(bytes) -> ArrayBuffer (page-locked: a MAP_READ staging buffer),
 *   downloadAsync(ptr, typedArray) (enqueued, the host does not wait),
 *   whenDone() -> Promise<void> (settles when everything enqueued before it
 *   has run, waited for off the JS thread), spin(us),
 *   gateHold(maxUs) -> number, gateRelease(number) (the stream held until the
 *   host has enqueued what follows: a profiled batch's timings)
 * Device functions are stream-ordered on the null stream (on the capture
 * stream while a capture is open); synchronize() (or any download) waits for
 * them.
 * Errors: a TypeError/RangeError for bad arguments, an Error carrying
 * wxo_last_error() (and a numeric `status` property) for a failed call.
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "wxo_q8.h"

#define CHECK_NAPI(env, call)                                              \
    do {                                                                   \
        if ((call) != napi_ok) {                                           \
            napi_throw_error((env), "WXO_NAPI", "internal N-API failure"); \
            return NULL;                                                   \
        }                                                                  \
    } while (0)

static napi_value throw_status(napi_env env, int status, const char* what) {
    char msg[768];
    snprintf(msg, sizeof msg, "%s failed (wxo status %d): %s", what, status, wxo_last_error());
    napi_value text, err, code;
    napi_create_string_utf8(env, msg, NAPI_AUTO_LENGTH, &text);
    napi_create_error(env, NULL, text, &err);
    napi_create_int32(env, status, &code);
    napi_set_named_property(env, err, "status", code);
    napi_throw(env, err);
    return NULL;
}

static int type_error(napi_env env, const char* fmt, const char* a) {
    char msg[256];
    snprintf(msg, sizeof msg, fmt, a);
    napi_throw_type_error(env, NULL, msg);
    return 0;
}

static int range_error(napi_env env, const char* msg) {
    napi_throw_range_error(env, NULL, msg);
    return 0;
}

static int get_args(napi_env env, napi_callback_info info, size_t want_min, size_t* argc, napi_value* argv) {
    size_t n = *argc;
    if (napi_get_cb_info(env, info, &n, argv, NULL, NULL) != napi_ok) return type_error(env, "%s", "bad call");
    if (n < want_min) {
        char msg[96];
        snprintf(msg, sizeof msg, "expected at least %zu arguments, got %zu", want_min, n);
        napi_throw_type_error(env, NULL, msg);
        return 0;
    }
    *argc = n;
    return 1;
}

/* A non-negative integer number below 2^32 (what the reference's u32 uniforms hold). */
static int get_u32(napi_env env, napi_value v, uint32_t* out, const char* name) {
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_number) return type_error(env, "%s must be a number", name);
    double d;
    napi_get_value_double(env, v, &d);
    if (!(d >= 0.0 && d <= 4294967295.0) || d != (double)(uint64_t)d)
        return type_error(env, "%s must be an integer in [0, 2^32)", name);
    *out = (uint32_t)d;
    return 1;
}

static const char* typed_name(napi_typedarray_type t) {
    switch (t) {
        case napi_int8_array: return "Int8Array";
        case napi_uint8_array: return "Uint8Array";
        case napi_int32_array: return "Int32Array";
        case napi_uint32_array: return "Uint32Array";
        case napi_float32_array: return "Float32Array";
        default: return "typed array";
    }
}

static int get_typed(napi_env env, napi_value v, napi_typedarray_type want, void** data, size_t* length,
                     const char* name) {
    bool is_typed = false;
    napi_is_typedarray(env, v, &is_typed);
    if (!is_typed) {
        char msg[160];
        snprintf(msg, sizeof msg, "%s must be a %s", name, typed_name(want));
        napi_throw_type_error(env, NULL, msg);
        return 0;
    }
    napi_typedarray_type t;
    napi_value ab;
    size_t off;
    if (napi_get_typedarray_info(env, v, &t, length, data, &ab, &off) != napi_ok) return type_error(env, "%s", name);
    if (t != want) {
        char msg[160];
        snprintf(msg, sizeof msg, "%s must be a %s, got a %s", name, typed_name(want), typed_name(t));
        napi_throw_type_error(env, NULL, msg);
        return 0;
    }
    return 1;
}

static int need_len(napi_env env, size_t have, uint64_t need, const char* name) {
    if ((uint64_t)have < need) {
        char msg[200];
        snprintf(msg, sizeof msg, "%s has %zu elements, %llu needed", name, have, (unsigned long long)need);
        napi_throw_range_error(env, NULL, msg);
        return 0;
    }
    return 1;
}

static napi_value new_typed(napi_env env, napi_typedarray_type type, size_t elem, size_t length, void** data) {
    napi_value ab, arr;
    if (napi_create_arraybuffer(env, length * elem, data, &ab) != napi_ok) return NULL;
    if (napi_create_typedarray(env, type, length, ab, 0, &arr) != napi_ok) return NULL;
    return arr;
}

static int get_ptr(napi_env env, napi_value v, uint64_t* out, const char* name) {
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_bigint) return type_error(env, "%s must be a bigint device address", name);
    bool lossless = false;
    napi_get_value_bigint_uint64(env, v, out, &lossless);
    if (!lossless) return type_error(env, "%s is not a 64-bit device address", name);
    return 1;
}

static uint64_t words_per_row(uint32_t K) { return ((uint64_t)K + 3) / 4; }

/* ---------------------------------------------------------------- library */

static napi_value js_abi_version(napi_env env, napi_callback_info info) {
    (void)info;
    napi_value r;
    napi_create_int32(env, wxo_abi_version(), &r);
    return r;
}

static napi_value js_describe(napi_env env, napi_callback_info info) {
    (void)info;
    napi_value r;
    napi_create_string_utf8(env, wxo_describe(), NAPI_AUTO_LENGTH, &r);
    return r;
}

static napi_value js_device_count(napi_env env, napi_callback_info info) {
    (void)info;
    int n = 0;
    int st = wxo_device_count(&n);
    if (st != WXO_OK) return throw_status(env, st, "deviceCount");
    napi_value r;
    napi_create_int32(env, n, &r);
    return r;
}

static napi_value js_init(napi_env env, napi_callback_info info) {
    (void)info;
    int st = wxo_init();
    if (st != WXO_OK) return throw_status(env, st, "init");
    return NULL;
}

static napi_value js_synchronize(napi_env env, napi_callback_info info) {
    (void)info;
    int st = wxo_synchronize();
    if (st != WXO_OK) return throw_status(env, st, "synchronize");
    return NULL;
}

/* roofline() -> {bandwidth, compute}: this device's best sustained HBM read
 * bytes/s and one-wide f32 FMA flop/s, measured now (wxo_roofline); the
 * reference's measureRoofline(runner) (harness/roofline.ts:162-198) returns
 * the same two fields. */
static napi_value js_roofline(napi_env env, napi_callback_info info) {
    (void)info;
    double bw = 0.0, fl = 0.0;
    int st = wxo_roofline(&bw, &fl);
    if (st != WXO_OK) return throw_status(env, st, "roofline");
    napi_value r, v;
    napi_create_object(env, &r);
    napi_create_double(env, bw, &v);
    napi_set_named_property(env, r, "bandwidth", v);
    napi_create_double(env, fl, &v);
    napi_set_named_property(env, r, "compute", v);
    return r;
}

/* rooflineMatrix() -> number: the bf16 matrix cores' sustained rate in flop/s
 * on every CU with operands of matmulQ8's kinds (wxo_roofline_matrix); no
 * counterpart in the reference, whose roofline measures HBM and FMA only. */
static napi_value js_roofline_matrix(napi_env env, napi_callback_info info) {
    (void)info;
    double fl = 0.0;
    int st = wxo_roofline_matrix(&fl);
    if (st != WXO_OK) return throw_status(env, st, "rooflineMatrix");
    napi_value v;
    napi_create_double(env, fl, &v);
    return v;
}

/* ---------------------------------------------------------------- streams and captured batches
 * Device-pointer ops enqueue on g_stream: the null stream, except while a
 * batch is being captured (graphBegin .. graphEnd), when it is the addon's
 * capture stream.  graphBegin() starts recording; graphEnd() -> bigint closes
 * the capture and instantiates it (wxo_graph_capture_end); graphLaunch(g)
 * replays it on the null stream; graphDestroy(g) frees it.  synchronize()
 * waits for every stream.  upload/download stay synchronous on the null
 * stream. */
static wxo_stream_t g_stream = NULL;
static wxo_stream_t g_capture = NULL;

static napi_value js_graph_begin(napi_env env, napi_callback_info info) {
    (void)info;
    if (g_stream != NULL) {
        napi_throw_error(env, "WXO_NAPI", "graphBegin: a capture is already open");
        return NULL;
    }
    int st = WXO_OK;
    if (g_capture == NULL) st = wxo_stream_create(&g_capture);
    if (st == WXO_OK) st = wxo_graph_capture_begin(g_capture);
    if (st != WXO_OK) return throw_status(env, st, "graphBegin");
    g_stream = g_capture;
    return NULL;
}

static napi_value js_graph_end(napi_env env, napi_callback_info info) {
    (void)info;
    if (g_stream == NULL) {
        napi_throw_error(env, "WXO_NAPI", "graphEnd: no capture is open");
        return NULL;
    }
    wxo_graph_t g = NULL;
    int st = wxo_graph_capture_end(g_capture, &g);
    g_stream = NULL;
    if (st != WXO_OK) return throw_status(env, st, "graphEnd");
    napi_value r;
    napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)g, &r);
    return r;
}

/* The replay runs on the null stream, in order with every other op and
 * readback the addon enqueues there (the capture itself needs a stream of its
 * own; the graph does not), so callers need not synchronise between
 * batches. */
static napi_value js_graph_launch(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint64_t g;
    if (!get_args(env, info, 1, &argc, argv) || !get_ptr(env, argv[0], &g, "graph")) return NULL;
    if (g_stream != NULL) {
        napi_throw_error(env, "WXO_NAPI", "graphLaunch: a capture is open");
        return NULL;
    }
    int st = wxo_graph_launch((wxo_graph_t)(uintptr_t)g, NULL);
    if (st != WXO_OK) return throw_status(env, st, "graphLaunch");
    return NULL;
}

static napi_value js_graph_destroy(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint64_t g;
    if (!get_args(env, info, 1, &argc, argv) || !get_ptr(env, argv[0], &g, "graph")) return NULL;
    int st = wxo_graph_destroy((wxo_graph_t)(uintptr_t)g);
    if (st != WXO_OK) return throw_status(env, st, "graphDestroy");
    return NULL;
}

/* ---------------------------------------------------------------- asynchronous completion
 * hostAlloc(bytes) -> ArrayBuffer over page-locked host memory (freed when the
 * buffer is collected): what a WebGPU MAP_READ | COPY_DST staging buffer is
 * (harness/resident.ts:41-48).  downloadAsync(ptr, typedArray) enqueues the
 * copy of typedArray.byteLength bytes at ptr into it after the work already
 * enqueued; the bytes are there once a later whenDone() has settled.
 * whenDone() -> Promise<void>: records an event on the ops stream and waits
 * for it on a libuv worker thread, so the JS thread keeps running meanwhile
 * (the reference's queue.onSubmittedWorkDone() / mapAsync,
 * harness/resident.ts:321-345).  It rejects with the library's error text if
 * the wait fails.  spin(us): wxo_spin on the ops stream (a test aid that keeps
 * the GPU busy for `us` microseconds). */

static int typed_bytes(napi_env env, napi_value v, void** data, size_t* bytes);

static void host_finalize(napi_env env, void* data, void* hint) {
    (void)env;
    (void)hint;
    (void)wxo_host_free(data);
}

static napi_value js_host_alloc(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint32_t bytes;
    if (!get_args(env, info, 1, &argc, argv) || !get_u32(env, argv[0], &bytes, "bytes")) return NULL;
    void* p = NULL;
    int st = wxo_host_malloc(&p, bytes > 0 ? bytes : 1);
    if (st != WXO_OK) return throw_status(env, st, "hostAlloc");
    napi_value ab;
    if (napi_create_external_arraybuffer(env, p, bytes, host_finalize, NULL, &ab) != napi_ok) {
        (void)wxo_host_free(p);
        napi_throw_error(env, "WXO_NAPI", "hostAlloc: cannot wrap the page-locked buffer");
        return NULL;
    }
    return ab;
}

static napi_value js_download_async(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    uint64_t p;
    void* data;
    size_t bytes;
    if (!get_args(env, info, 2, &argc, argv) || !get_ptr(env, argv[0], &p, "ptr") ||
        !typed_bytes(env, argv[1], &data, &bytes))
        return NULL;
    if (g_stream != NULL) {
        napi_throw_error(env, "WXO_NAPI", "downloadAsync: a capture is open");
        return NULL;
    }
    int st = wxo_memcpy_dtoh_async(data, (const void*)(uintptr_t)p, bytes, NULL);
    if (st != WXO_OK) return throw_status(env, st, "downloadAsync");
    return NULL;
}

typedef struct {
    napi_async_work work;
    napi_deferred deferred;
    wxo_event_t event;
    int status;
    char message[512];
} DoneWait;

static void done_execute(napi_env env, void* data) {
    (void)env;
    DoneWait* w = (DoneWait*)data;
    w->status = wxo_event_synchronize(w->event);
    if (w->status != WXO_OK) snprintf(w->message, sizeof w->message, "whenDone failed (wxo status %d): %s", w->status, wxo_last_error());
}

static void done_complete(napi_env env, napi_status status, void* data) {
    DoneWait* w = (DoneWait*)data;
    (void)wxo_event_destroy(w->event);
    if (status == napi_ok && w->status == WXO_OK) {
        napi_value undef;
        napi_get_undefined(env, &undef);
        napi_resolve_deferred(env, w->deferred, undef);
    } else {
        napi_value text, err, code;
        napi_create_string_utf8(env, w->status != WXO_OK ? w->message : "whenDone: the wait was cancelled",
                                NAPI_AUTO_LENGTH, &text);
        napi_create_error(env, NULL, text, &err);
        napi_create_int32(env, w->status, &code);
        napi_set_named_property(env, err, "status", code);
        napi_reject_deferred(env, w->deferred, err);
    }
    napi_delete_async_work(env, w->work);
    free(w);
}

static napi_value js_when_done(napi_env env, napi_callback_info info) {
    (void)info;
    if (g_stream != NULL) {
        napi_throw_error(env, "WXO_NAPI", "whenDone: a capture is open");
        return NULL;
    }
    DoneWait* w = (DoneWait*)calloc(1, sizeof *w);
    if (w == NULL) {
        napi_throw_error(env, "WXO_NAPI", "whenDone: out of host memory");
        return NULL;
    }
    int st = wxo_event_create(&w->event);
    if (st == WXO_OK) st = wxo_event_record(w->event, NULL);
    if (st != WXO_OK) {
        (void)wxo_event_destroy(w->event);
        free(w);
        return throw_status(env, st, "whenDone");
    }
    napi_value promise, name;
    napi_create_string_utf8(env, "wxo.whenDone", NAPI_AUTO_LENGTH, &name);
    if (napi_create_promise(env, &w->deferred, &promise) != napi_ok ||
        napi_create_async_work(env, NULL, name, done_execute, done_complete, w, &w->work) != napi_ok ||
        napi_queue_async_work(env, w->work) != napi_ok) {
        (void)wxo_event_destroy(w->event);
        free(w);
        napi_throw_error(env, "WXO_NAPI", "whenDone: cannot queue the wait");
        return NULL;
    }
    return promise;
}

static napi_value js_spin(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint32_t us;
    if (!get_args(env, info, 1, &argc, argv) || !get_u32(env, argv[0], &us, "us")) return NULL;
    int st = wxo_spin(us, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "spin");
    return NULL;
}

/* gateHold(maxUs) -> number: holds the ops stream until gateRelease(number)
 * or maxUs of GPU time (wxo_gate_hold); gateRelease(number). */
static napi_value js_gate_hold(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint32_t us, gate = 0;
    if (!get_args(env, info, 1, &argc, argv) || !get_u32(env, argv[0], &us, "maxUs")) return NULL;
    if (g_stream != NULL) {
        napi_throw_error(env, "WXO_NAPI", "gateHold: a capture is open");
        return NULL;
    }
    int st = wxo_gate_hold(us, NULL, &gate);
    if (st != WXO_OK) return throw_status(env, st, "gateHold");
    napi_value r;
    napi_create_uint32(env, gate, &r);
    return r;
}

static napi_value js_gate_release(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint32_t gate;
    if (!get_args(env, info, 1, &argc, argv) || !get_u32(env, argv[0], &gate, "gate")) return NULL;
    int st = wxo_gate_release(gate);
    if (st != WXO_OK) return throw_status(env, st, "gateRelease");
    return NULL;
}

static napi_value js_last_variant(napi_env env, napi_callback_info info) {
    (void)info;
    napi_value r;
    napi_create_string_utf8(env, wxo_last_variant(), NAPI_AUTO_LENGTH, &r);
    return r;
}

/* ---------------------------------------------------------------- events
 * GPU timestamps on the null stream, for per-op timing inside a resident
 * batch: eventCreate() -> bigint (a timing-only event, wxo_event_create_timer),
 * eventRecord(ev), eventElapsedMs(start, stop) (waits for `stop`),
 * eventDestroy(ev). */

static napi_value js_event_create(napi_env env, napi_callback_info info) {
    (void)info;
    wxo_event_t ev = NULL;
    int st = wxo_event_create_timer(&ev);
    if (st != WXO_OK) return throw_status(env, st, "eventCreate");
    napi_value r;
    napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)ev, &r);
    return r;
}

static napi_value js_event_destroy(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint64_t ev;
    if (!get_args(env, info, 1, &argc, argv) || !get_ptr(env, argv[0], &ev, "event")) return NULL;
    int st = wxo_event_destroy((wxo_event_t)(uintptr_t)ev);
    if (st != WXO_OK) return throw_status(env, st, "eventDestroy");
    return NULL;
}

static napi_value js_event_record(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint64_t ev;
    if (!get_args(env, info, 1, &argc, argv) || !get_ptr(env, argv[0], &ev, "event")) return NULL;
    int st = wxo_event_record((wxo_event_t)(uintptr_t)ev, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "eventRecord");
    return NULL;
}

static napi_value js_event_elapsed_ms(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    uint64_t a, b;
    if (!get_args(env, info, 2, &argc, argv) || !get_ptr(env, argv[0], &a, "start") ||
        !get_ptr(env, argv[1], &b, "stop"))
        return NULL;
    int st = wxo_event_synchronize((wxo_event_t)(uintptr_t)b);
    float ms = 0.0f;
    if (st == WXO_OK) st = wxo_event_elapsed_ms(&ms, (wxo_event_t)(uintptr_t)a, (wxo_event_t)(uintptr_t)b);
    if (st != WXO_OK) return throw_status(env, st, "eventElapsedMs");
    napi_value r;
    napi_create_double(env, (double)ms, &r);
    return r;
}

/* ---------------------------------------------------------------- host-array ops */

static napi_value js_matvec_q8(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    if (!get_args(env, info, 5, &argc, argv)) return NULL;
    void *w, *s, *x;
    size_t lw, ls, lx;
    uint32_t N, K, M = 1;
    if (!get_typed(env, argv[0], napi_uint32_array, &w, &lw, "weight") ||
        !get_typed(env, argv[1], napi_float32_array, &s, &ls, "scale") ||
        !get_typed(env, argv[2], napi_float32_array, &x, &lx, "vector") || !get_u32(env, argv[3], &N, "N") ||
        !get_u32(env, argv[4], &K, "K"))
        return NULL;
    if (argc > 5) {
        napi_valuetype t;
        napi_typeof(env, argv[5], &t);
        if (t != napi_undefined && !get_u32(env, argv[5], &M, "M")) return NULL;
    }
    if (M == 0) {
        range_error(env, "M must be >= 1");
        return NULL;
    }
    if (!need_len(env, lw, (uint64_t)N * words_per_row(K), "weight") || !need_len(env, ls, N, "scale") ||
        !need_len(env, lx, (uint64_t)M * K, "vector"))
        return NULL;
    void* y;
    napi_value out = new_typed(env, napi_float32_array, 4, (size_t)M * N, &y);
    if (!out) return NULL;
    int st = wxo_matvec_q8_host(w, s, x, y, N, K, M);
    if (st != WXO_OK) return throw_status(env, st, "matvecQ8");
    return out;
}

/* matvecQ8Async(weight u32, scale f32, vector f32, N, K, M = 1) -> Promise<Float32Array[M*N]>
 *
 * The reference's non-resident dispatch returns a promise and waits for the
 * GPU without holding the JS thread (harness/wgsl.ts:35-36 Runner.run, used by
 * llm/kernels.ts:195-211 runMatVecQ8).  Here the whole host call (device
 * buffers, the copies in, the kernel, the copy out) runs on a libuv worker
 * thread.  Arguments are checked on the calling thread (a bad one throws
 * there).  As WebGPU's queue.writeBuffer does, the call takes its inputs when
 * it is made: scale and vector are copied then (they are small and an engine
 * reuses its activation buffers); the weight, megabytes of static model data,
 * is held by reference and read on the worker, so it must not change while
 * the promise is pending.  The result array is handed over only on success;
 * a failed call rejects with the library's error text and `status`. */
typedef struct {
    napi_async_work work;
    napi_deferred deferred;
    napi_ref weight_ref, out_ref;
    const void* weight;
    float *scale, *vector;
    void* out;
    uint32_t N, K, M;
    int status;
    char message[512];
} HostMatvec;

static void host_matvec_execute(napi_env env, void* data) {
    (void)env;
    HostMatvec* h = (HostMatvec*)data;
    h->status = wxo_matvec_q8_host((const uint32_t*)h->weight, h->scale, h->vector, (float*)h->out, h->N, h->K, h->M);
    if (h->status != WXO_OK)
        snprintf(h->message, sizeof h->message, "matvecQ8Async failed (wxo status %d): %s", h->status, wxo_last_error());
}

static void host_matvec_free(napi_env env, HostMatvec* h) {
    if (h->weight_ref != NULL) napi_delete_reference(env, h->weight_ref);
    if (h->out_ref != NULL) napi_delete_reference(env, h->out_ref);
    free(h->scale);
    free(h->vector);
    free(h);
}

static void host_matvec_complete(napi_env env, napi_status status, void* data) {
    HostMatvec* h = (HostMatvec*)data;
    napi_value out;
    if (status == napi_ok && h->status == WXO_OK && napi_get_reference_value(env, h->out_ref, &out) == napi_ok) {
        napi_resolve_deferred(env, h->deferred, out);
    } else {
        napi_value text, err, code;
        napi_create_string_utf8(env, h->status != WXO_OK ? h->message : "matvecQ8Async: the call was cancelled",
                                NAPI_AUTO_LENGTH, &text);
        napi_create_error(env, NULL, text, &err);
        napi_create_int32(env, h->status != WXO_OK ? h->status : WXO_ERR_DEVICE, &code);
        napi_set_named_property(env, err, "status", code);
        napi_reject_deferred(env, h->deferred, err);
    }
    napi_delete_async_work(env, h->work);
    host_matvec_free(env, h);
}

static napi_value js_matvec_q8_async(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    if (!get_args(env, info, 5, &argc, argv)) return NULL;
    void *w, *s, *x;
    size_t lw, ls, lx;
    uint32_t N, K, M = 1;
    if (!get_typed(env, argv[0], napi_uint32_array, &w, &lw, "weight") ||
        !get_typed(env, argv[1], napi_float32_array, &s, &ls, "scale") ||
        !get_typed(env, argv[2], napi_float32_array, &x, &lx, "vector") || !get_u32(env, argv[3], &N, "N") ||
        !get_u32(env, argv[4], &K, "K"))
        return NULL;
    if (argc > 5) {
        napi_valuetype t;
        napi_typeof(env, argv[5], &t);
        if (t != napi_undefined && !get_u32(env, argv[5], &M, "M")) return NULL;
    }
    if (M == 0) {
        range_error(env, "M must be >= 1");
        return NULL;
    }
    if (!need_len(env, lw, (uint64_t)N * words_per_row(K), "weight") || !need_len(env, ls, N, "scale") ||
        !need_len(env, lx, (uint64_t)M * K, "vector"))
        return NULL;
    HostMatvec* h = (HostMatvec*)calloc(1, sizeof *h);
    if (h == NULL) {
        napi_throw_error(env, "WXO_NAPI", "matvecQ8Async: out of host memory");
        return NULL;
    }
    h->weight = w;
    h->N = N;
    h->K = K;
    h->M = M;
    const size_t sb = (size_t)N * 4, xb = (size_t)M * K * 4;
    h->scale = (float*)malloc(sb > 0 ? sb : 1);
    h->vector = (float*)malloc(xb > 0 ? xb : 1);
    napi_value out = NULL, promise, name;
    if (h->scale != NULL && h->vector != NULL) out = new_typed(env, napi_float32_array, 4, (size_t)M * N, &h->out);
    if (out == NULL) {
        host_matvec_free(env, h);
        bool pending = false;
        napi_is_exception_pending(env, &pending);
        if (!pending) napi_throw_error(env, "WXO_NAPI", "matvecQ8Async: out of host memory");
        return NULL;
    }
    if (sb > 0) memcpy(h->scale, s, sb);
    if (xb > 0) memcpy(h->vector, x, xb);
    napi_create_string_utf8(env, "wxo.matvecQ8Async", NAPI_AUTO_LENGTH, &name);
    if (napi_create_reference(env, argv[0], 1, &h->weight_ref) != napi_ok ||
        napi_create_reference(env, out, 1, &h->out_ref) != napi_ok ||
        napi_create_promise(env, &h->deferred, &promise) != napi_ok ||
        napi_create_async_work(env, NULL, name, host_matvec_execute, host_matvec_complete, h, &h->work) != napi_ok) {
        host_matvec_free(env, h);
        napi_throw_error(env, "WXO_NAPI", "matvecQ8Async: cannot queue the call");
        return NULL;
    }
    if (napi_queue_async_work(env, h->work) != napi_ok) {
        napi_delete_async_work(env, h->work);
        host_matvec_free(env, h);
        napi_throw_error(env, "WXO_NAPI", "matvecQ8Async: cannot queue the call");
        return NULL;
    }
    return promise;
}

/* matvecQ8Residual(weight u32, scale f32, vector f32, residual f32, N, K) -> Float32Array[N] */
static napi_value js_matvec_q8_residual(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    if (!get_args(env, info, 6, &argc, argv)) return NULL;
    void *w, *s, *x, *r;
    size_t lw, ls, lx, lr;
    uint32_t N, K;
    if (!get_typed(env, argv[0], napi_uint32_array, &w, &lw, "weight") ||
        !get_typed(env, argv[1], napi_float32_array, &s, &ls, "scale") ||
        !get_typed(env, argv[2], napi_float32_array, &x, &lx, "vector") ||
        !get_typed(env, argv[3], napi_float32_array, &r, &lr, "residual") || !get_u32(env, argv[4], &N, "N") ||
        !get_u32(env, argv[5], &K, "K"))
        return NULL;
    if (!need_len(env, lw, (uint64_t)N * words_per_row(K), "weight") || !need_len(env, ls, N, "scale") ||
        !need_len(env, lx, K, "vector") || !need_len(env, lr, N, "residual"))
        return NULL;
    void* y;
    napi_value out = new_typed(env, napi_float32_array, 4, N, &y);
    if (!out) return NULL;
    int st = wxo_matvec_q8_residual_host(w, s, x, r, y, N, K);
    if (st != WXO_OK) return throw_status(env, st, "matvecQ8Residual");
    return out;
}

/* matvecQ8Ffn(weightGate u32, scaleGate f32, weightUp u32, scaleUp f32, vector f32, N, K) -> Float32Array[N] */
static napi_value js_matvec_q8_ffn(napi_env env, napi_callback_info info) {
    size_t argc = 7;
    napi_value argv[7];
    if (!get_args(env, info, 7, &argc, argv)) return NULL;
    void *wg, *sg, *wu, *su, *x;
    size_t lwg, lsg, lwu, lsu, lx;
    uint32_t N, K;
    if (!get_typed(env, argv[0], napi_uint32_array, &wg, &lwg, "weightGate") ||
        !get_typed(env, argv[1], napi_float32_array, &sg, &lsg, "scaleGate") ||
        !get_typed(env, argv[2], napi_uint32_array, &wu, &lwu, "weightUp") ||
        !get_typed(env, argv[3], napi_float32_array, &su, &lsu, "scaleUp") ||
        !get_typed(env, argv[4], napi_float32_array, &x, &lx, "vector") || !get_u32(env, argv[5], &N, "N") ||
        !get_u32(env, argv[6], &K, "K"))
        return NULL;
    const uint64_t nw = (uint64_t)N * words_per_row(K);
    if (!need_len(env, lwg, nw, "weightGate") || !need_len(env, lsg, N, "scaleGate") ||
        !need_len(env, lwu, nw, "weightUp") || !need_len(env, lsu, N, "scaleUp") || !need_len(env, lx, K, "vector"))
        return NULL;
    void* y;
    napi_value out = new_typed(env, napi_float32_array, 4, N, &y);
    if (!out) return NULL;
    int st = wxo_matvec_q8_ffn_host(wg, sg, wu, su, x, y, N, K);
    if (st != WXO_OK) return throw_status(env, st, "matvecQ8Ffn");
    return out;
}

static napi_value js_quantize(napi_env env, napi_callback_info info) {
    size_t argc = 3;
    napi_value argv[3];
    if (!get_args(env, info, 3, &argc, argv)) return NULL;
    void* in;
    size_t lin;
    uint32_t N, D;
    if (!get_typed(env, argv[0], napi_float32_array, &in, &lin, "input") || !get_u32(env, argv[1], &N, "N") ||
        !get_u32(env, argv[2], &D, "D"))
        return NULL;
    if (!need_len(env, lin, (uint64_t)N * D, "input")) return NULL;
    void *codes, *scales;
    napi_value a = new_typed(env, napi_int32_array, 4, (size_t)N * D, &codes);
    napi_value b = new_typed(env, napi_float32_array, 4, N, &scales);
    if (!a || !b) return NULL;
    int st = wxo_quantize_host(in, N, D, codes, scales);
    if (st != WXO_OK) return throw_status(env, st, "quantize");
    napi_value obj;
    CHECK_NAPI(env, napi_create_object(env, &obj));
    napi_set_named_property(env, obj, "output", a);
    napi_set_named_property(env, obj, "scales", b);
    return obj;
}

static napi_value pack_common(napi_env env, napi_callback_info info, int int8) {
    size_t argc = 3;
    napi_value argv[3];
    if (!get_args(env, info, 3, &argc, argv)) return NULL;
    void* codes;
    size_t lc;
    uint32_t N, K;
    if (!get_typed(env, argv[0], int8 ? napi_int8_array : napi_int32_array, &codes, &lc, "codes") ||
        !get_u32(env, argv[1], &N, "N") || !get_u32(env, argv[2], &K, "K"))
        return NULL;
    if (!need_len(env, lc, (uint64_t)N * K, "codes")) return NULL;
    void* packed;
    napi_value out = new_typed(env, napi_uint32_array, 4, (size_t)(N * words_per_row(K)), &packed);
    if (!out) return NULL;
    int st = int8 ? wxo_pack_int8_rows_host(codes, N, K, packed) : wxo_pack_q8_host(codes, N, K, packed);
    if (st != WXO_OK) return throw_status(env, st, int8 ? "packInt8Rows" : "packQ8");
    return out;
}

static napi_value js_pack_q8(napi_env env, napi_callback_info info) { return pack_common(env, info, 0); }
static napi_value js_pack_int8_rows(napi_env env, napi_callback_info info) { return pack_common(env, info, 1); }

static napi_value js_quantize_pack_q8(napi_env env, napi_callback_info info) {
    size_t argc = 3;
    napi_value argv[3];
    if (!get_args(env, info, 3, &argc, argv)) return NULL;
    void* in;
    size_t lin;
    uint32_t N, K;
    if (!get_typed(env, argv[0], napi_float32_array, &in, &lin, "input") || !get_u32(env, argv[1], &N, "N") ||
        !get_u32(env, argv[2], &K, "K"))
        return NULL;
    if (!need_len(env, lin, (uint64_t)N * K, "input")) return NULL;
    void *packed, *scales;
    napi_value a = new_typed(env, napi_uint32_array, 4, (size_t)(N * words_per_row(K)), &packed);
    napi_value b = new_typed(env, napi_float32_array, 4, N, &scales);
    if (!a || !b) return NULL;
    int st = wxo_quantize_pack_q8_host(in, N, K, packed, scales);
    if (st != WXO_OK) return throw_status(env, st, "quantizePackQ8");
    napi_value obj;
    CHECK_NAPI(env, napi_create_object(env, &obj));
    napi_set_named_property(env, obj, "weight", a);
    napi_set_named_property(env, obj, "scale", b);
    return obj;
}

/* matmulQ8(a f32 [N*K], weight u32 [M*ceil(K/4)], scale f32 [M], N, M, K) -> Float32Array [N*M] */
static napi_value js_matmul_q8(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    if (!get_args(env, info, 6, &argc, argv)) return NULL;
    void *a, *w, *s;
    size_t la, lw, ls;
    uint32_t N, M, K;
    if (!get_typed(env, argv[0], napi_float32_array, &a, &la, "a") ||
        !get_typed(env, argv[1], napi_uint32_array, &w, &lw, "weight") ||
        !get_typed(env, argv[2], napi_float32_array, &s, &ls, "scale") || !get_u32(env, argv[3], &N, "N") ||
        !get_u32(env, argv[4], &M, "M") || !get_u32(env, argv[5], &K, "K"))
        return NULL;
    if (!need_len(env, la, (uint64_t)N * K, "a") || !need_len(env, lw, (uint64_t)M * words_per_row(K), "weight") ||
        !need_len(env, ls, M, "scale"))
        return NULL;
    void* y;
    napi_value out = new_typed(env, napi_float32_array, 4, (size_t)N * M, &y);
    if (!out) return NULL;
    int st = wxo_matmul_q8_host(a, w, s, y, N, M, K);
    if (st != WXO_OK) return throw_status(env, st, "matmulQ8");
    return out;
}

/* dequantizePackedQ8(weight u32, scale f32, N, K) -> Float32Array [N*K];
 * dequantTranspose(weight u32, scale f32, outFeatures, inFeatures) -> Float32Array
 * [inFeatures*outFeatures], with the reference's exact-length checks
 * (ops/dequant_transpose/reference.ts:42-47) */
static napi_value dequant_common(napi_env env, napi_callback_info info, int transpose) {
    size_t argc = 4;
    napi_value argv[4];
    if (!get_args(env, info, 4, &argc, argv)) return NULL;
    void *w, *s;
    size_t lw, ls;
    uint32_t N, K;
    if (!get_typed(env, argv[0], napi_uint32_array, &w, &lw, "weight") ||
        !get_typed(env, argv[1], napi_float32_array, &s, &ls, "scale") ||
        !get_u32(env, argv[2], &N, transpose ? "outFeatures" : "N") ||
        !get_u32(env, argv[3], &K, transpose ? "inFeatures" : "K"))
        return NULL;
    if (transpose) {
        char msg[160];
        if ((uint64_t)lw != (uint64_t)N * words_per_row(K)) {
            snprintf(msg, sizeof msg, "dequantTranspose(): expected %llu packed words, got %zu",
                     (unsigned long long)((uint64_t)N * words_per_row(K)), lw);
            napi_throw_error(env, NULL, msg);
            return NULL;
        }
        if ((uint64_t)ls != N) {
            snprintf(msg, sizeof msg, "dequantTranspose(): expected %u scales, got %zu", N, ls);
            napi_throw_error(env, NULL, msg);
            return NULL;
        }
    } else if (!need_len(env, lw, (uint64_t)N * words_per_row(K), "weight") || !need_len(env, ls, N, "scale")) {
        return NULL;
    }
    void* y;
    napi_value out = new_typed(env, napi_float32_array, 4, (size_t)N * K, &y);
    if (!out) return NULL;
    int st = transpose ? wxo_dequant_transpose_host(w, s, N, K, y) : wxo_dequantize_packed_q8_host(w, s, N, K, y);
    if (st != WXO_OK) return throw_status(env, st, transpose ? "dequantTranspose" : "dequantizePackedQ8");
    return out;
}

static napi_value js_dequantize_packed_q8(napi_env env, napi_callback_info info) {
    return dequant_common(env, info, 0);
}
static napi_value js_dequant_transpose(napi_env env, napi_callback_info info) { return dequant_common(env, info, 1); }

/* Request indices as int64: a JS array of integers or an Int32Array /
 * Uint32Array / BigInt64Array.  Returns a malloc'd array (caller frees). */
static int64_t* get_indices(napi_env env, napi_value v, uint32_t* count) {
    bool is_array = false, is_typed = false;
    napi_is_array(env, v, &is_array);
    napi_is_typedarray(env, v, &is_typed);
    if (is_array) {
        uint32_t n = 0;
        napi_get_array_length(env, v, &n);
        int64_t* out = (int64_t*)malloc((n ? n : 1) * sizeof(int64_t));
        for (uint32_t i = 0; i < n; ++i) {
            napi_value e;
            napi_get_element(env, v, i, &e);
            napi_valuetype t;
            napi_typeof(env, e, &t);
            double d;
            if (t != napi_number || napi_get_value_double(env, e, &d) != napi_ok || d != d || d < -9.0e15 ||
                d > 9.0e15 || d != (double)(int64_t)d) {
                free(out);
                napi_throw_type_error(env, NULL, "indices must hold integers");
                return NULL;
            }
            out[i] = (int64_t)d;
        }
        *count = n;
        return out;
    }
    if (is_typed) {
        napi_typedarray_type t;
        size_t n;
        void* data;
        napi_value ab;
        size_t off;
        napi_get_typedarray_info(env, v, &t, &n, &data, &ab, &off);
        if (n > 0xffffffffu) {
            napi_throw_range_error(env, NULL, "too many indices");
            return NULL;
        }
        if (t != napi_int32_array && t != napi_uint32_array && t != napi_bigint64_array) {
            napi_throw_type_error(env, NULL, "indices must be an array, Int32Array, Uint32Array or BigInt64Array");
            return NULL;
        }
        int64_t* out = (int64_t*)malloc((n ? n : 1) * sizeof(int64_t));
        for (size_t i = 0; i < n; ++i)
            out[i] = t == napi_int32_array ? (int64_t)((const int32_t*)data)[i]
                     : t == napi_uint32_array ? (int64_t)((const uint32_t*)data)[i]
                                              : ((const int64_t*)data)[i];
        *count = (uint32_t)n;
        return out;
    }
    napi_throw_type_error(env, NULL, "indices must be an array, Int32Array, Uint32Array or BigInt64Array");
    return NULL;
}

/* gatherDequantRows(codes Int8Array [rows*D], scale Float32Array [rows], indices, D)
 * -> Float32Array [indices.length * D]; rows = scale.length (llm/weights-q8.ts:207-222) */
static napi_value js_gather_dequant_rows(napi_env env, napi_callback_info info) {
    size_t argc = 4;
    napi_value argv[4];
    if (!get_args(env, info, 4, &argc, argv)) return NULL;
    void *c, *s;
    size_t lc, ls;
    uint32_t D;
    if (!get_typed(env, argv[0], napi_int8_array, &c, &lc, "codes") ||
        !get_typed(env, argv[1], napi_float32_array, &s, &ls, "scale") || !get_u32(env, argv[3], &D, "D"))
        return NULL;
    if (ls > 0xffffffffu) {
        range_error(env, "too many rows");
        return NULL;
    }
    const uint32_t rows = (uint32_t)ls;
    if (!need_len(env, lc, (uint64_t)rows * D, "codes")) return NULL;
    uint32_t count = 0;
    int64_t* idx = get_indices(env, argv[2], &count);
    if (!idx) return NULL;
    void* y;
    napi_value out = new_typed(env, napi_float32_array, 4, (size_t)count * D, &y);
    if (!out) {
        free(idx);
        return NULL;
    }
    int st = wxo_gather_dequant_rows_host(c, s, rows, D, idx, count, y);
    free(idx);
    if (st != WXO_OK) return throw_status(env, st, "gatherDequantRows");
    return out;
}

/* ---------------------------------------------------------------- device memory */

static napi_value js_malloc(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    if (!get_args(env, info, 1, &argc, argv)) return NULL;
    napi_valuetype t;
    napi_typeof(env, argv[0], &t);
    double d = -1;
    if (t == napi_number) napi_get_value_double(env, argv[0], &d);
    if (!(d >= 0 && d <= 9007199254740991.0) || d != (double)(uint64_t)d) {
        napi_throw_type_error(env, NULL, "bytes must be a non-negative integer");
        return NULL;
    }
    void* p = NULL;
    int st = wxo_malloc(&p, (size_t)d);
    if (st != WXO_OK) return throw_status(env, st, "malloc");
    napi_value r;
    napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &r);
    return r;
}

static napi_value js_free(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    uint64_t p;
    if (!get_args(env, info, 1, &argc, argv) || !get_ptr(env, argv[0], &p, "ptr")) return NULL;
    int st = wxo_free((void*)(uintptr_t)p);
    if (st != WXO_OK) return throw_status(env, st, "free");
    return NULL;
}

static int typed_bytes(napi_env env, napi_value v, void** data, size_t* bytes) {
    bool is_typed = false;
    napi_is_typedarray(env, v, &is_typed);
    if (!is_typed) return type_error(env, "%s", "expected a typed array");
    napi_typedarray_type t;
    size_t len, off;
    napi_value ab;
    napi_get_typedarray_info(env, v, &t, &len, data, &ab, &off);
    size_t elem = (t == napi_int8_array || t == napi_uint8_array || t == napi_uint8_clamped_array) ? 1
                  : (t == napi_int16_array || t == napi_uint16_array)                                 ? 2
                  : (t == napi_float64_array || t == napi_bigint64_array || t == napi_biguint64_array) ? 8
                                                                                                      : 4;
    *bytes = len * elem;
    return 1;
}

/* upload(ptr, typedArray) / download(ptr, typedArray): whole typed array. */
static napi_value js_upload(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    uint64_t p;
    void* data;
    size_t bytes;
    if (!get_args(env, info, 2, &argc, argv) || !get_ptr(env, argv[0], &p, "ptr") ||
        !typed_bytes(env, argv[1], &data, &bytes))
        return NULL;
    int st = wxo_memcpy_htod((void*)(uintptr_t)p, data, bytes, NULL);
    if (st != WXO_OK) return throw_status(env, st, "upload");
    return NULL;
}

static napi_value js_download(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    uint64_t p;
    void* data;
    size_t bytes;
    if (!get_args(env, info, 2, &argc, argv) || !get_ptr(env, argv[0], &p, "ptr") ||
        !typed_bytes(env, argv[1], &data, &bytes))
        return NULL;
    int st = wxo_memcpy_dtoh(data, (const void*)(uintptr_t)p, bytes, NULL);
    if (st != WXO_OK) return throw_status(env, st, "download");
    return argv[1];
}

/* zero(ptr, bytes): the bytes cleared on the null stream, done before it
 * returns (a new buffer's WebGPU contents; set-up, never inside a batch). */
static napi_value js_zero(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    uint64_t p;
    if (!get_args(env, info, 2, &argc, argv) || !get_ptr(env, argv[0], &p, "ptr")) return NULL;
    double d = -1;
    napi_get_value_double(env, argv[1], &d);
    if (!(d >= 0) || d != (double)(uint64_t)d) {
        napi_throw_type_error(env, NULL, "bytes must be a non-negative integer");
        return NULL;
    }
    int st = wxo_memset((void*)(uintptr_t)p, 0, (size_t)d, NULL);
    if (st == WXO_OK) st = wxo_stream_synchronize(NULL);
    if (st != WXO_OK) return throw_status(env, st, "zero");
    return NULL;
}

static napi_value js_copy(napi_env env, napi_callback_info info) {
    size_t argc = 3;
    napi_value argv[3];
    uint64_t dst, src;
    if (!get_args(env, info, 3, &argc, argv) || !get_ptr(env, argv[0], &dst, "dst") ||
        !get_ptr(env, argv[1], &src, "src"))
        return NULL;
    double d = -1;
    napi_get_value_double(env, argv[2], &d);
    if (!(d >= 0) || d != (double)(uint64_t)d) {
        napi_throw_type_error(env, NULL, "bytes must be a non-negative integer");
        return NULL;
    }
    int st = wxo_memcpy_dtod((void*)(uintptr_t)dst, (const void*)(uintptr_t)src, (size_t)d, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "copy");
    return NULL;
}

/* ---------------------------------------------------------------- device-pointer ops */

static napi_value js_matvec_q8_device(napi_env env, napi_callback_info info) {
    size_t argc = 7;
    napi_value argv[7];
    uint64_t w, s, x, y;
    uint32_t N, K, M = 1;
    if (!get_args(env, info, 6, &argc, argv) || !get_ptr(env, argv[0], &w, "weight") ||
        !get_ptr(env, argv[1], &s, "scale") || !get_ptr(env, argv[2], &x, "vector") ||
        !get_ptr(env, argv[3], &y, "output") || !get_u32(env, argv[4], &N, "N") || !get_u32(env, argv[5], &K, "K"))
        return NULL;
    if (argc > 6 && !get_u32(env, argv[6], &M, "M")) return NULL;
    int st = wxo_matvec_q8((const uint32_t*)(uintptr_t)w, (const float*)(uintptr_t)s, (const float*)(uintptr_t)x,
                           (float*)(uintptr_t)y, N, K, M, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "matvecQ8Device");
    return NULL;
}

/* matvecQ8MultiDevice([[weight, scale, output, N], ...], vector, K): several
 * projections of one vector (device addresses), one launch per 4. */
static napi_value js_matvec_q8_multi_device(napi_env env, napi_callback_info info) {
    size_t argc = 3;
    napi_value argv[3];
    uint64_t x;
    uint32_t K, count = 0;
    bool is_array = false;
    if (!get_args(env, info, 3, &argc, argv)) return NULL;
    if (napi_is_array(env, argv[0], &is_array) != napi_ok || !is_array)
        return type_error(env, "%s must be an array of [weight, scale, output, N]", "projections"), NULL;
    if (!get_ptr(env, argv[1], &x, "vector") || !get_u32(env, argv[2], &K, "K")) return NULL;
    napi_get_array_length(env, argv[0], &count);
    const size_t n = count > 0 ? count : 1;
    const uint32_t** ws = (const uint32_t**)calloc(n, sizeof *ws);
    const float** ss = (const float**)calloc(n, sizeof *ss);
    float** ys = (float**)calloc(n, sizeof *ys);
    uint32_t* ns = (uint32_t*)calloc(n, sizeof *ns);
    napi_value result = NULL;
    int okay = ws && ss && ys && ns;
    if (!okay) napi_throw_error(env, NULL, "matvecQ8MultiDevice: out of host memory");
    for (uint32_t i = 0; okay && i < count; ++i) {
        napi_value e, f[4];
        uint32_t len = 0;
        uint64_t w, sc, y;
        okay = napi_get_element(env, argv[0], i, &e) == napi_ok && napi_is_array(env, e, &is_array) == napi_ok &&
               is_array && napi_get_array_length(env, e, &len) == napi_ok && len == 4;
        if (!okay) {
            char idx[16];
            snprintf(idx, sizeof idx, "%u", i);
            type_error(env, "projection %s must be [weight, scale, output, N]", idx);
            break;
        }
        for (uint32_t j = 0; j < 4; ++j) napi_get_element(env, e, j, &f[j]);
        okay = get_ptr(env, f[0], &w, "weight") && get_ptr(env, f[1], &sc, "scale") &&
               get_ptr(env, f[2], &y, "output") && get_u32(env, f[3], &ns[i], "N");
        ws[i] = (const uint32_t*)(uintptr_t)w;
        ss[i] = (const float*)(uintptr_t)sc;
        ys[i] = (float*)(uintptr_t)y;
    }
    if (okay) {
        int st = wxo_matvec_q8_multi(ws, ss, ys, ns, count, (const float*)(uintptr_t)x, K, g_stream);
        if (st != WXO_OK) throw_status(env, st, "matvecQ8MultiDevice");
    }
    free(ws);
    free(ss);
    free(ys);
    free(ns);
    return result;
}

/* quantizePackQ8MultiDevice([[input, N, packed, scales], ...], K): quantize +
 * packQ8 of several matrices with one K (device addresses), one launch per 8. */
static napi_value js_quantize_pack_q8_multi_device(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    uint32_t K, count = 0;
    bool is_array = false;
    if (!get_args(env, info, 2, &argc, argv)) return NULL;
    if (napi_is_array(env, argv[0], &is_array) != napi_ok || !is_array)
        return type_error(env, "%s must be an array of [input, N, packed, scales]", "matrices"), NULL;
    if (!get_u32(env, argv[1], &K, "K")) return NULL;
    napi_get_array_length(env, argv[0], &count);
    const size_t n = count > 0 ? count : 1;
    const float** ins = (const float**)calloc(n, sizeof *ins);
    uint32_t* ns = (uint32_t*)calloc(n, sizeof *ns);
    uint32_t** ps = (uint32_t**)calloc(n, sizeof *ps);
    float** ss = (float**)calloc(n, sizeof *ss);
    int okay = ins && ns && ps && ss;
    if (!okay) napi_throw_error(env, NULL, "quantizePackQ8MultiDevice: out of host memory");
    for (uint32_t i = 0; okay && i < count; ++i) {
        napi_value e, f[4];
        uint32_t len = 0;
        uint64_t in, p, sc;
        okay = napi_get_element(env, argv[0], i, &e) == napi_ok && napi_is_array(env, e, &is_array) == napi_ok &&
               is_array && napi_get_array_length(env, e, &len) == napi_ok && len == 4;
        if (!okay) {
            char idx[16];
            snprintf(idx, sizeof idx, "%u", i);
            type_error(env, "matrix %s must be [input, N, packed, scales]", idx);
            break;
        }
        for (uint32_t j = 0; j < 4; ++j) napi_get_element(env, e, j, &f[j]);
        okay = get_ptr(env, f[0], &in, "input") && get_u32(env, f[1], &ns[i], "N") &&
               get_ptr(env, f[2], &p, "packed") && get_ptr(env, f[3], &sc, "scales");
        ins[i] = (const float*)(uintptr_t)in;
        ps[i] = (uint32_t*)(uintptr_t)p;
        ss[i] = (float*)(uintptr_t)sc;
    }
    if (okay) {
        int st = wxo_quantize_pack_q8_multi(ins, ns, ps, ss, count, K, g_stream);
        if (st != WXO_OK) throw_status(env, st, "quantizePackQ8MultiDevice");
    }
    free(ins);
    free(ns);
    free(ps);
    free(ss);
    return NULL;
}

/* matvecQ8ResidualDevice(weight, scale, vector, residual, output, N, K): device addresses */
static napi_value js_matvec_q8_residual_device(napi_env env, napi_callback_info info) {
    size_t argc = 7;
    napi_value argv[7];
    uint64_t w, s, x, r, y;
    uint32_t N, K;
    if (!get_args(env, info, 7, &argc, argv) || !get_ptr(env, argv[0], &w, "weight") ||
        !get_ptr(env, argv[1], &s, "scale") || !get_ptr(env, argv[2], &x, "vector") ||
        !get_ptr(env, argv[3], &r, "residual") || !get_ptr(env, argv[4], &y, "output") ||
        !get_u32(env, argv[5], &N, "N") || !get_u32(env, argv[6], &K, "K"))
        return NULL;
    int st = wxo_matvec_q8_residual((const uint32_t*)(uintptr_t)w, (const float*)(uintptr_t)s,
                                    (const float*)(uintptr_t)x, (const float*)(uintptr_t)r, (float*)(uintptr_t)y, N,
                                    K, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "matvecQ8ResidualDevice");
    return NULL;
}

/* matvecQ8FfnDevice(weightGate, scaleGate, weightUp, scaleUp, vector, output, N, K): device addresses */
static napi_value js_matvec_q8_ffn_device(napi_env env, napi_callback_info info) {
    size_t argc = 8;
    napi_value argv[8];
    uint64_t wg, sg, wu, su, x, y;
    uint32_t N, K;
    if (!get_args(env, info, 8, &argc, argv) || !get_ptr(env, argv[0], &wg, "weightGate") ||
        !get_ptr(env, argv[1], &sg, "scaleGate") || !get_ptr(env, argv[2], &wu, "weightUp") ||
        !get_ptr(env, argv[3], &su, "scaleUp") || !get_ptr(env, argv[4], &x, "vector") ||
        !get_ptr(env, argv[5], &y, "output") || !get_u32(env, argv[6], &N, "N") || !get_u32(env, argv[7], &K, "K"))
        return NULL;
    int st = wxo_matvec_q8_ffn((const uint32_t*)(uintptr_t)wg, (const float*)(uintptr_t)sg,
                               (const uint32_t*)(uintptr_t)wu, (const float*)(uintptr_t)su,
                               (const float*)(uintptr_t)x, (float*)(uintptr_t)y, N, K, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "matvecQ8FfnDevice");
    return NULL;
}

static napi_value js_quantize_device(napi_env env, napi_callback_info info) {
    size_t argc = 5;
    napi_value argv[5];
    uint64_t in, out, sc;
    uint32_t N, D;
    if (!get_args(env, info, 5, &argc, argv) || !get_ptr(env, argv[0], &in, "input") ||
        !get_u32(env, argv[1], &N, "N") || !get_u32(env, argv[2], &D, "D") || !get_ptr(env, argv[3], &out, "output") ||
        !get_ptr(env, argv[4], &sc, "scales"))
        return NULL;
    int st = wxo_quantize((const float*)(uintptr_t)in, N, D, (int32_t*)(uintptr_t)out, (float*)(uintptr_t)sc, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "quantizeDevice");
    return NULL;
}

static napi_value pack_device_common(napi_env env, napi_callback_info info, int int8) {
    size_t argc = 4;
    napi_value argv[4];
    uint64_t codes, packed;
    uint32_t N, K;
    if (!get_args(env, info, 4, &argc, argv) || !get_ptr(env, argv[0], &codes, "codes") ||
        !get_u32(env, argv[1], &N, "N") || !get_u32(env, argv[2], &K, "K") || !get_ptr(env, argv[3], &packed, "packed"))
        return NULL;
    int st = int8 ? wxo_pack_int8_rows((const int8_t*)(uintptr_t)codes, N, K, (uint32_t*)(uintptr_t)packed, NULL)
                  : wxo_pack_q8((const int32_t*)(uintptr_t)codes, N, K, (uint32_t*)(uintptr_t)packed, g_stream);
    if (st != WXO_OK) return throw_status(env, st, int8 ? "packInt8RowsDevice" : "packQ8Device");
    return NULL;
}

static napi_value js_pack_q8_device(napi_env env, napi_callback_info info) { return pack_device_common(env, info, 0); }
static napi_value js_pack_int8_rows_device(napi_env env, napi_callback_info info) {
    return pack_device_common(env, info, 1);
}

static napi_value js_quantize_pack_q8_device(napi_env env, napi_callback_info info) {
    size_t argc = 5;
    napi_value argv[5];
    uint64_t in, packed, sc;
    uint32_t N, K;
    if (!get_args(env, info, 5, &argc, argv) || !get_ptr(env, argv[0], &in, "input") ||
        !get_u32(env, argv[1], &N, "N") || !get_u32(env, argv[2], &K, "K") ||
        !get_ptr(env, argv[3], &packed, "packed") || !get_ptr(env, argv[4], &sc, "scales"))
        return NULL;
    int st = wxo_quantize_pack_q8((const float*)(uintptr_t)in, N, K, (uint32_t*)(uintptr_t)packed,
                                  (float*)(uintptr_t)sc, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "quantizePackQ8Device");
    return NULL;
}

/* matmulQ8Device(a, weight, scale, output, N, M, K): device addresses */
/* matmulQ8MultiDevice([[weight, scale, output, M], ...], a, N, K): several
 * projections of the same activations a [N, K] (device addresses), one launch
 * per 4. */
/* matmulQ8WorkspaceBytes(): the workspace size that allows every split on the current device. */
static napi_value js_matmul_q8_workspace_bytes(napi_env env, napi_callback_info info) {
    (void)info;
    size_t bytes = 0;
    int st = wxo_matmul_q8_workspace_bytes(&bytes);
    if (st != WXO_OK) return throw_status(env, st, "matmulQ8WorkspaceBytes"), NULL;
    napi_value r;
    napi_create_double(env, (double)bytes, &r);
    return r;
}

/* matmulQ8MultiDevice(projections, a, N, K[, workspace, workspaceBytes]):
 * with a workspace (a device address and its size), wxo_matmul_q8_multi_ws. */
static napi_value js_matmul_q8_multi_device(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    uint64_t a, wsp = 0;
    uint32_t N, K, count = 0, wsb = 0;
    bool is_array = false, with_ws = false;
    if (!get_args(env, info, 4, &argc, argv)) return NULL;
    if (napi_is_array(env, argv[0], &is_array) != napi_ok || !is_array)
        return type_error(env, "%s must be an array of [weight, scale, output, M]", "projections"), NULL;
    if (!get_ptr(env, argv[1], &a, "a") || !get_u32(env, argv[2], &N, "N") || !get_u32(env, argv[3], &K, "K"))
        return NULL;
    if (argc >= 6) {
        napi_valuetype t;
        napi_typeof(env, argv[4], &t);
        with_ws = t != napi_undefined && t != napi_null;
        if (with_ws && (!get_ptr(env, argv[4], &wsp, "workspace") || !get_u32(env, argv[5], &wsb, "workspaceBytes")))
            return NULL;
    }
    napi_get_array_length(env, argv[0], &count);
    const size_t n = count > 0 ? count : 1;
    const uint32_t** ws = (const uint32_t**)calloc(n, sizeof *ws);
    const float** ss = (const float**)calloc(n, sizeof *ss);
    float** ys = (float**)calloc(n, sizeof *ys);
    uint32_t* ms = (uint32_t*)calloc(n, sizeof *ms);
    int okay = ws && ss && ys && ms;
    if (!okay) napi_throw_error(env, NULL, "matmulQ8MultiDevice: out of host memory");
    for (uint32_t i = 0; okay && i < count; ++i) {
        napi_value e, f[4];
        uint32_t len = 0;
        uint64_t w, sc, y;
        okay = napi_get_element(env, argv[0], i, &e) == napi_ok && napi_is_array(env, e, &is_array) == napi_ok &&
               is_array && napi_get_array_length(env, e, &len) == napi_ok && len == 4;
        if (!okay) {
            char idx[16];
            snprintf(idx, sizeof idx, "%u", i);
            type_error(env, "projection %s must be [weight, scale, output, M]", idx);
            break;
        }
        for (uint32_t j = 0; j < 4; ++j) napi_get_element(env, e, j, &f[j]);
        okay = get_ptr(env, f[0], &w, "weight") && get_ptr(env, f[1], &sc, "scale") &&
               get_ptr(env, f[2], &y, "output") && get_u32(env, f[3], &ms[i], "M");
        ws[i] = (const uint32_t*)(uintptr_t)w;
        ss[i] = (const float*)(uintptr_t)sc;
        ys[i] = (float*)(uintptr_t)y;
    }
    if (okay) {
        int st = with_ws ? wxo_matmul_q8_multi_ws((const float*)(uintptr_t)a, ws, ss, ys, ms, count, N, K,
                                                  (void*)(uintptr_t)wsp, wsb, g_stream)
                         : wxo_matmul_q8_multi((const float*)(uintptr_t)a, ws, ss, ys, ms, count, N, K, g_stream);
        if (st != WXO_OK) throw_status(env, st, "matmulQ8MultiDevice");
    }
    free(ws);
    free(ss);
    free(ys);
    free(ms);
    return NULL;
}

static napi_value js_matmul_q8_device(napi_env env, napi_callback_info info) {
    size_t argc = 7;
    napi_value argv[7];
    uint64_t a, w, s, y;
    uint32_t N, M, K;
    if (!get_args(env, info, 7, &argc, argv) || !get_ptr(env, argv[0], &a, "a") ||
        !get_ptr(env, argv[1], &w, "weight") || !get_ptr(env, argv[2], &s, "scale") ||
        !get_ptr(env, argv[3], &y, "output") || !get_u32(env, argv[4], &N, "N") || !get_u32(env, argv[5], &M, "M") ||
        !get_u32(env, argv[6], &K, "K"))
        return NULL;
    int st = wxo_matmul_q8((const float*)(uintptr_t)a, (const uint32_t*)(uintptr_t)w, (const float*)(uintptr_t)s,
                           (float*)(uintptr_t)y, N, M, K, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "matmulQ8Device");
    return NULL;
}

/* dequantizePackedQ8Device / dequantTransposeDevice(weight, scale, N, K, output) */
static napi_value dequant_device_common(napi_env env, napi_callback_info info, int transpose) {
    size_t argc = 5;
    napi_value argv[5];
    uint64_t w, s, y;
    uint32_t N, K;
    if (!get_args(env, info, 5, &argc, argv) || !get_ptr(env, argv[0], &w, "weight") ||
        !get_ptr(env, argv[1], &s, "scale") || !get_u32(env, argv[2], &N, "N") || !get_u32(env, argv[3], &K, "K") ||
        !get_ptr(env, argv[4], &y, "output"))
        return NULL;
    const uint32_t* wp = (const uint32_t*)(uintptr_t)w;
    const float* sp = (const float*)(uintptr_t)s;
    int st = transpose ? wxo_dequant_transpose(wp, sp, N, K, (float*)(uintptr_t)y, NULL)
                       : wxo_dequantize_packed_q8(wp, sp, N, K, (float*)(uintptr_t)y, g_stream);
    if (st != WXO_OK) return throw_status(env, st, transpose ? "dequantTransposeDevice" : "dequantizePackedQ8Device");
    return NULL;
}
static napi_value js_dequantize_packed_q8_device(napi_env env, napi_callback_info info) {
    return dequant_device_common(env, info, 0);
}
static napi_value js_dequant_transpose_device(napi_env env, napi_callback_info info) {
    return dequant_device_common(env, info, 1);
}

/* gatherDequantRowsDevice(codes, scale, rows, D, indices (int64 device array), count, output) */
static napi_value js_gather_dequant_rows_device(napi_env env, napi_callback_info info) {
    size_t argc = 7;
    napi_value argv[7];
    uint64_t c, s, ix, y;
    uint32_t rows, D, count;
    if (!get_args(env, info, 7, &argc, argv) || !get_ptr(env, argv[0], &c, "codes") ||
        !get_ptr(env, argv[1], &s, "scale") || !get_u32(env, argv[2], &rows, "rows") || !get_u32(env, argv[3], &D, "D") ||
        !get_ptr(env, argv[4], &ix, "indices") || !get_u32(env, argv[5], &count, "count") ||
        !get_ptr(env, argv[6], &y, "output"))
        return NULL;
    int st = wxo_gather_dequant_rows((const int8_t*)(uintptr_t)c, (const float*)(uintptr_t)s, rows, D,
                                     (const int64_t*)(uintptr_t)ix, count, (float*)(uintptr_t)y, g_stream);
    if (st != WXO_OK) return throw_status(env, st, "gatherDequantRowsDevice");
    return NULL;
}

/* ---------------------------------------------------------------- module */

static napi_value init_module(napi_env env, napi_value exports) {
    napi_property_descriptor props[] = {
        {"abiVersion", NULL, js_abi_version, NULL, NULL, NULL, napi_enumerable, NULL},
        {"describe", NULL, js_describe, NULL, NULL, NULL, napi_enumerable, NULL},
        {"lastVariant", NULL, js_last_variant, NULL, NULL, NULL, napi_enumerable, NULL},
        {"graphBegin", NULL, js_graph_begin, NULL, NULL, NULL, napi_enumerable, NULL},
        {"graphEnd", NULL, js_graph_end, NULL, NULL, NULL, napi_enumerable, NULL},
        {"graphLaunch", NULL, js_graph_launch, NULL, NULL, NULL, napi_enumerable, NULL},
        {"graphDestroy", NULL, js_graph_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
        {"eventCreate", NULL, js_event_create, NULL, NULL, NULL, napi_enumerable, NULL},
        {"eventDestroy", NULL, js_event_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
        {"eventRecord", NULL, js_event_record, NULL, NULL, NULL, napi_enumerable, NULL},
        {"eventElapsedMs", NULL, js_event_elapsed_ms, NULL, NULL, NULL, napi_enumerable, NULL},
        {"deviceCount", NULL, js_device_count, NULL, NULL, NULL, napi_enumerable, NULL},
        {"init", NULL, js_init, NULL, NULL, NULL, napi_enumerable, NULL},
        {"synchronize", NULL, js_synchronize, NULL, NULL, NULL, napi_enumerable, NULL},
        {"roofline", NULL, js_roofline, NULL, NULL, NULL, napi_enumerable, NULL},
        {"rooflineMatrix", NULL, js_roofline_matrix, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8", NULL, js_matvec_q8, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8Async", NULL, js_matvec_q8_async, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8Residual", NULL, js_matvec_q8_residual, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8Ffn", NULL, js_matvec_q8_ffn, NULL, NULL, NULL, napi_enumerable, NULL},
        {"quantize", NULL, js_quantize, NULL, NULL, NULL, napi_enumerable, NULL},
        {"packQ8", NULL, js_pack_q8, NULL, NULL, NULL, napi_enumerable, NULL},
        {"packInt8Rows", NULL, js_pack_int8_rows, NULL, NULL, NULL, napi_enumerable, NULL},
        {"quantizePackQ8", NULL, js_quantize_pack_q8, NULL, NULL, NULL, napi_enumerable, NULL},
        {"malloc", NULL, js_malloc, NULL, NULL, NULL, napi_enumerable, NULL},
        {"free", NULL, js_free, NULL, NULL, NULL, napi_enumerable, NULL},
        {"upload", NULL, js_upload, NULL, NULL, NULL, napi_enumerable, NULL},
        {"download", NULL, js_download, NULL, NULL, NULL, napi_enumerable, NULL},
        {"downloadAsync", NULL, js_download_async, NULL, NULL, NULL, napi_enumerable, NULL},
        {"hostAlloc", NULL, js_host_alloc, NULL, NULL, NULL, napi_enumerable, NULL},
        {"whenDone", NULL, js_when_done, NULL, NULL, NULL, napi_enumerable, NULL},
        {"spin", NULL, js_spin, NULL, NULL, NULL, napi_enumerable, NULL},
        {"gateHold", NULL, js_gate_hold, NULL, NULL, NULL, napi_enumerable, NULL},
        {"gateRelease", NULL, js_gate_release, NULL, NULL, NULL, napi_enumerable, NULL},
        {"copy", NULL, js_copy, NULL, NULL, NULL, napi_enumerable, NULL},
        {"zero", NULL, js_zero, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8Device", NULL, js_matvec_q8_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8MultiDevice", NULL, js_matvec_q8_multi_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8ResidualDevice", NULL, js_matvec_q8_residual_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"quantizePackQ8MultiDevice", NULL, js_quantize_pack_q8_multi_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecQ8FfnDevice", NULL, js_matvec_q8_ffn_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"quantizeDevice", NULL, js_quantize_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"packQ8Device", NULL, js_pack_q8_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"packInt8RowsDevice", NULL, js_pack_int8_rows_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"quantizePackQ8Device", NULL, js_quantize_pack_q8_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matmulQ8", NULL, js_matmul_q8, NULL, NULL, NULL, napi_enumerable, NULL},
        {"dequantizePackedQ8", NULL, js_dequantize_packed_q8, NULL, NULL, NULL, napi_enumerable, NULL},
        {"dequantTranspose", NULL, js_dequant_transpose, NULL, NULL, NULL, napi_enumerable, NULL},
        {"gatherDequantRows", NULL, js_gather_dequant_rows, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matmulQ8Device", NULL, js_matmul_q8_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matmulQ8MultiDevice", NULL, js_matmul_q8_multi_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matmulQ8WorkspaceBytes", NULL, js_matmul_q8_workspace_bytes, NULL, NULL, NULL, napi_enumerable, NULL},
        {"dequantizePackedQ8Device", NULL, js_dequantize_packed_q8_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"dequantTransposeDevice", NULL, js_dequant_transpose_device, NULL, NULL, NULL, napi_enumerable, NULL},
        {"gatherDequantRowsDevice", NULL, js_gather_dequant_rows_device, NULL, NULL, NULL, napi_enumerable, NULL},
    };
    if (napi_define_properties(env, exports, sizeof props / sizeof props[0], props) != napi_ok) return NULL;
    return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init_module)
