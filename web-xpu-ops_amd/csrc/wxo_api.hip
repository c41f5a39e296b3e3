// wxo_api.hip -- the C ABI (include/wxo_q8.h) over the gfx950 kernels.
//
// Status codes instead of exceptions; a per-thread message for the last
// failure; sizes validated before any launch (the reference reads `undefined`
// -> NaN on short inputs, this layer refuses them).  Device entry points are
// asynchronous on the caller's stream and allocate nothing.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/wxo_q8.h"
#include "kernels.hpp"

#ifndef WXO_BUILD_ID
#define WXO_BUILD_ID "dev"
#endif

namespace {

thread_local char g_error[512] = {0};
// The kernel instance the calling thread's last successful op launched.
thread_local wxo::Variant g_variant;
thread_local char g_variant_text[256] = {0};

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return status;
}

int ok() {
    g_error[0] = '\0';
    return WXO_OK;
}

int hip_fail(hipError_t e, const char* what) {
    // The error is reported here; consume the runtime's per-thread copy so
    // that a later launch's hipGetLastError does not report it again.
    (void)hipGetLastError();
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return fail(WXO_ERR_OOM, "%s: %s", what, hipGetErrorString(e));
    if (e == hipErrorNoDevice || e == hipErrorInsufficientDriver)
        return fail(WXO_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
    return fail(WXO_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
wxo::DeviceInfo g_dev[kMaxDevices];
std::mutex g_dev_mu;
char g_describe[1024] = {0};

// The workspace of wxo_matmul_q8_multi_static: the largest split workspace
// wxo_matmul_q8_multi_ws ever uses on a 256-CU device (64 KiB per CU, 16 MiB).  Each
// GPU holds its own copy from the code object's load until the process ends.
// Host code never passes the array's name to a kernel or a copy (on the host
// it is only a stand-in for the symbol): it uses g_scratch[device], the
// device address that hipGetSymbolAddress gives once per device at set-up.
constexpr size_t kScratchBytes = 256u * wxo::kMatmulWorkspaceBytesPerCu;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
void* g_scratch[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};

// Device info for the current HIP device, probed once per device.
int current_device(const wxo::DeviceInfo** out) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(WXO_ERR_NO_DEVICE, "no HIP device visible (hipGetDeviceCount: %s); the matvecQ8 path has no CPU "
                                       "fallback", e != hipSuccess ? hipGetErrorString(e) : "0 devices");
    int ordinal = 0;
    if ((e = hipGetDevice(&ordinal)) != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (ordinal < 0 || ordinal >= kMaxDevices) return fail(WXO_ERR_NO_DEVICE, "device ordinal %d out of range", ordinal);
    std::lock_guard<std::mutex> lock(g_dev_mu);
    wxo::DeviceInfo& d = g_dev[ordinal];
    if (d.ordinal != ordinal) {
        hipDeviceProp_t prop;
        if ((e = hipGetDeviceProperties(&prop, ordinal)) != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return fail(WXO_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 (MI355X) only", ordinal,
                        prop.gcnArchName);
        d.cu_count = prop.multiProcessorCount;
        d.hbm_bytes = prop.totalGlobalMem;
        snprintf(d.name, sizeof d.name, "%s", prop.name);
        snprintf(d.arch, sizeof d.arch, "%s", prop.gcnArchName);
        // this device is current: its copy of the scratch array
        void* p = nullptr;
        g_scratch_err[ordinal] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch[ordinal] = g_scratch_err[ordinal] == hipSuccess ? p : nullptr;
        // A failed probe is reported by wxo_matmul_q8_multi_static alone (from
        // g_scratch_err); clear the runtime's last error so the next launch's
        // hipGetLastError does not report it against an unrelated op.
        if (g_scratch_err[ordinal] != hipSuccess) (void)hipGetLastError();
        d.ordinal = ordinal;
    }
    *out = &d;
    return WXO_OK;
}

constexpr uint64_t kMaxElems = 1ull << 40;

bool too_big(uint64_t a, uint64_t b) { return a != 0 && b > kMaxElems / a; }

int check_ptr(const void* p, uint64_t elems, const char* name) {
    if (elems > 0 && p == nullptr) return fail(WXO_ERR_INVALID, "%s is NULL but %llu elements are needed", name,
                                               (unsigned long long)elems);
    return WXO_OK;
}

#define WXO_TRY(expr)              \
    do {                           \
        int _s = (expr);           \
        if (_s != WXO_OK) return _s; \
    } while (0)

int validate_matvec(const uint32_t* w, const float* s, const float* x, const float* y, uint32_t N, uint32_t K,
                    uint32_t M) {
    if (M == 0) return fail(WXO_ERR_INVALID, "M (vectors) must be >= 1, got 0");
    // Kernels address a block of rows and the vector with 32-bit buffer offsets.
    if (K >= (1u << 27)) return fail(WXO_ERR_INVALID, "K=%u exceeds the supported maximum 2^27 - 1", K);
    const uint64_t W = ((uint64_t)K + 3) / 4;
    if (too_big(N, W) || too_big(M, K) || too_big(M, N))
        return fail(WXO_ERR_INVALID, "sizes N=%u K=%u M=%u exceed 2^40 elements", N, K, M);
    WXO_TRY(check_ptr(w, (uint64_t)N * W, "weight"));
    WXO_TRY(check_ptr(s, N, "scale"));
    WXO_TRY(check_ptr(x, (uint64_t)M * K, "vector"));
    WXO_TRY(check_ptr(y, (uint64_t)M * N, "output"));
    return WXO_OK;
}

int validate_rows(const void* in, uint32_t N, uint32_t K, const char* in_name) {
    // Kernels address one row with 32-bit buffer offsets.
    if (K >= (1u << 27)) return fail(WXO_ERR_INVALID, "row length %u exceeds the supported maximum 2^27 - 1", K);
    if (too_big(N, K)) return fail(WXO_ERR_INVALID, "sizes N=%u K=%u exceed 2^40 elements", N, K);
    return check_ptr(in, (uint64_t)N * K, in_name);
}

int validate_matmul(const float* a, const uint32_t* w, const float* s, const float* y, uint32_t N, uint32_t M,
                    uint32_t K) {
    // A workgroup addresses 64 activation rows and 128 weight rows with 32-bit
    // buffer offsets.
    if (K > (1u << 22)) return fail(WXO_ERR_INVALID, "K=%u exceeds the supported maximum 2^22 for matmulQ8", K);
    const uint64_t W = ((uint64_t)K + 3) / 4;
    if (too_big(N, K) || too_big(M, W) || too_big(N, M))
        return fail(WXO_ERR_INVALID, "sizes N=%u M=%u K=%u exceed 2^40 elements", N, M, K);
    WXO_TRY(check_ptr(a, (uint64_t)N * K, "a"));
    WXO_TRY(check_ptr(w, (uint64_t)M * W, "weight"));
    WXO_TRY(check_ptr(s, M, "scale"));
    WXO_TRY(check_ptr(y, (uint64_t)N * M, "output"));
    return WXO_OK;
}

int validate_dequant(const uint32_t* w, const float* s, const float* y, uint32_t N, uint32_t K) {
    const uint64_t W = ((uint64_t)K + 3) / 4;
    if (too_big(N, K)) return fail(WXO_ERR_INVALID, "sizes N=%u K=%u exceed 2^40 elements", N, K);
    WXO_TRY(check_ptr(w, (uint64_t)N * W, "weight"));
    WXO_TRY(check_ptr(s, N, "scale"));
    return check_ptr(y, (uint64_t)N * K, "output");
}

int validate_gather(const int8_t* codes, const float* s, const int64_t* idx, const float* y, uint32_t rows,
                    uint32_t D, uint32_t count) {
    if (too_big(rows, D) || too_big(count, D))
        return fail(WXO_ERR_INVALID, "sizes rows=%u D=%u count=%u exceed 2^40 elements", rows, D, count);
    WXO_TRY(check_ptr(codes, (uint64_t)rows * D, "codes"));
    WXO_TRY(check_ptr(s, rows, "scale"));
    WXO_TRY(check_ptr(idx, count, "indices"));
    return check_ptr(y, (uint64_t)count * D, "output");
}

hipStream_t as_hip(wxo_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Result of a launch: on success the chosen instance becomes this thread's
// last variant; an op that launched nothing (no rows) records "none".
int launched(hipError_t e, const wxo::Variant& v, const char* what) {
    if (e != hipSuccess) return hip_fail(e, what);
    g_variant = v;
    if (!g_variant.kernel || !g_variant.kernel[0]) g_variant = wxo::Variant{"none", "empty", 0, 0, 0, 0, 0, 0};
    return ok();
}

wxo::Variant named(const char* kernel, const char* form = "") { return wxo::Variant{kernel, form, 0, 0, 0, 0, 0, 0}; }

// RAII device buffer for the *_host entry points.
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t bytes) {
        if (bytes == 0) return WXO_OK;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            p = nullptr;
            return hip_fail(e, "hipMalloc");
        }
        return WXO_OK;
    }
    int upload(const void* src, size_t bytes) {
        if (bytes == 0) return WXO_OK;
        hipError_t e = hipMemcpy(p, src, bytes, hipMemcpyHostToDevice);
        return e == hipSuccess ? WXO_OK : hip_fail(e, "hipMemcpy H2D");
    }
    int download(void* dst, size_t bytes) const {
        if (bytes == 0) return WXO_OK;
        hipError_t e = hipMemcpy(dst, p, bytes, hipMemcpyDeviceToHost);
        return e == hipSuccess ? WXO_OK : hip_fail(e, "hipMemcpy D2H");
    }
};

}  // namespace

extern "C" {

int wxo_abi_version(void) { return WXO_ABI_VERSION; }

const char* wxo_last_error(void) { return g_error; }

const char* wxo_last_variant(void) {
    const wxo::Variant& v = g_variant;
    char* b = g_variant_text;
    const size_t cap = sizeof g_variant_text;
    b[0] = '\0';
    if (!v.kernel || !v.kernel[0]) return b;
    size_t n = (size_t)snprintf(b, cap, "%s", v.kernel);
    auto add = [&](const char* fmt, auto... xs) {
        if (n < cap) n += (size_t)snprintf(b + n, cap - n, fmt, xs...);
    };
    if (v.form && v.form[0]) add(" %s", v.form);
    if (v.waves) add(" waves=%d", v.waves);
    if (v.rows) add(" rows=%d", v.rows);
    if (v.slots) add(" slots=%d", v.slots);
    if (v.vectors) add(" vectors=%d", v.vectors);
    if (v.grid_x) add(" grid=%ux%u", v.grid_x, v.grid_y ? v.grid_y : 1u);
    return b;
}

int wxo_init(void) {
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    return ok();
}

const char* wxo_describe(void) {
    const wxo::DeviceInfo* d = nullptr;
    if (current_device(&d) != WXO_OK) {
        snprintf(g_describe, sizeof g_describe, "wxo_q8 abi=%d build=%s device=none (%s)", WXO_ABI_VERSION,
                 WXO_BUILD_ID, g_error);
        return g_describe;
    }
    snprintf(g_describe, sizeof g_describe,
             "wxo_q8 abi=%d build=%s device=%d name=\"%s\" arch=%s cus=%d hbm_gib=%.1f kernels=matvec_q8_m1(plain|"
             "residual|ffn),matvec_q8_multi,matvec_q8_mv(valu),matvec_q8_mfma(bf16x3),quantize_rows(reg|twopass),pack_q8,"
             "pack_int8_rows,matmul_q8(bf16x3),dequantize_packed,dequant_transpose,gather_dequant_rows last=\"%s\"",
             WXO_ABI_VERSION, WXO_BUILD_ID, d->ordinal, d->name, d->arch, d->cu_count,
             (double)d->hbm_bytes / (1024.0 * 1024.0 * 1024.0), wxo_last_variant());
    return g_describe;
}

int wxo_device_count(int* count) {
    if (!count) return fail(WXO_ERR_INVALID, "count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        if (e == hipErrorNoDevice) return ok();
        return hip_fail(e, "hipGetDeviceCount");
    }
    *count = n;
    return ok();
}

int wxo_set_device(int ordinal) {
    hipError_t e = hipSetDevice(ordinal);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    return wxo_init();
}

int wxo_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(WXO_ERR_INVALID, "ptr is NULL");
    *ptr = nullptr;
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    if (bytes == 0) return ok();
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return hip_fail(e, "hipMalloc");
    }
    return ok();
}

int wxo_free(void* ptr) {
    if (!ptr) return ok();
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? ok() : hip_fail(e, "hipFree");
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, wxo_stream_t stream, const char* what) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(WXO_ERR_INVALID, "%s: NULL pointer", what);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, as_hip(stream));
    if (e == hipSuccess && kind != hipMemcpyDeviceToDevice) e = hipStreamSynchronize(as_hip(stream));
    return e == hipSuccess ? ok() : hip_fail(e, what);
}

int wxo_memcpy_htod(void* dst, const void* src, size_t bytes, wxo_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyHostToDevice, stream, "memcpy H2D");
}
int wxo_memcpy_dtoh(void* dst, const void* src, size_t bytes, wxo_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream, "memcpy D2H");
}
int wxo_memcpy_dtod(void* dst, const void* src, size_t bytes, wxo_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream, "memcpy D2D");
}
int wxo_memcpy_dtoh_async(void* dst, const void* src, size_t bytes, wxo_stream_t stream) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(WXO_ERR_INVALID, "memcpy D2H async: NULL pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_hip(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "memcpy D2H async");
}

int wxo_host_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(WXO_ERR_INVALID, "ptr is NULL");
    *ptr = nullptr;
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    if (bytes == 0) return ok();
    hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return hip_fail(e, "hipHostMalloc");
    }
    return ok();
}

int wxo_host_free(void* ptr) {
    if (!ptr) return ok();
    hipError_t e = hipHostFree(ptr);
    return e == hipSuccess ? ok() : hip_fail(e, "hipHostFree");
}

namespace {
// Sets bytes [0, head) and [head + 16 body, + tail) one by one and the 16-byte
// aligned body between them with 16-byte stores (head, tail < 16).
__global__ __launch_bounds__(256) void fill_bytes_kernel(uint8_t* p, uint32_t v4, size_t head, size_t body, size_t tail) {
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
    uint4* b = reinterpret_cast<uint4*>(p + head);
    for (size_t i = tid; i < body; i += stride) b[i] = make_uint4(v4, v4, v4, v4);
    if (tid < head) p[tid] = (uint8_t)v4;
    if (tid < tail) p[head + 16u * body + tid] = (uint8_t)v4;
}
}  // namespace

int wxo_memset(void* ptr, int value, size_t bytes, wxo_stream_t stream) {
    if (bytes == 0) return ok();
    if (!ptr) return fail(WXO_ERR_INVALID, "memset: NULL pointer");
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    const uintptr_t a = (uintptr_t)ptr;
    size_t head = (16u - (a & 15u)) & 15u;
    if (head > bytes) head = bytes;
    const size_t body = (bytes - head) / 16u, tail = bytes - head - 16u * body;
    const uint32_t v = (uint32_t)(value & 0xff) * 0x01010101u;
    const size_t blocks = (body + 255u) / 256u;
    const uint32_t grid = (uint32_t)(blocks < 4096u ? (blocks > 0u ? blocks : 1u) : 4096u);
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(grid), dim3(256), 0, as_hip(stream), static_cast<uint8_t*>(ptr), v, head,
                       body, tail);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ok() : hip_fail(e, "fill launch");
}

int wxo_synchronize(void) {
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? ok() : hip_fail(e, "hipDeviceSynchronize");
}

int wxo_stream_create(wxo_stream_t* stream) {
    if (!stream) return fail(WXO_ERR_INVALID, "stream is NULL");
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);  // default priority
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
    *stream = reinterpret_cast<wxo_stream_t>(s);
    return ok();
}

int wxo_stream_destroy(wxo_stream_t stream) {
    if (!stream) return ok();
    hipError_t e = hipStreamDestroy(as_hip(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "hipStreamDestroy");
}

int wxo_stream_synchronize(wxo_stream_t stream) {
    hipError_t e = hipStreamSynchronize(as_hip(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "hipStreamSynchronize");
}

int wxo_event_create(wxo_event_t* event) {
    if (!event) return fail(WXO_ERR_INVALID, "event is NULL");
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
    *event = reinterpret_cast<wxo_event_t>(ev);
    return ok();
}

int wxo_event_create_timer(wxo_event_t* event) {
    if (!event) return fail(WXO_ERR_INVALID, "event is NULL");
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableSystemFence);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags");
    *event = reinterpret_cast<wxo_event_t>(ev);
    return ok();
}

int wxo_event_destroy(wxo_event_t event) {
    if (!event) return ok();
    hipError_t e = hipEventDestroy(reinterpret_cast<hipEvent_t>(event));
    return e == hipSuccess ? ok() : hip_fail(e, "hipEventDestroy");
}

int wxo_event_record(wxo_event_t event, wxo_stream_t stream) {
    hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_hip(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "hipEventRecord");
}

int wxo_event_synchronize(wxo_event_t event) {
    hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(event));
    return e == hipSuccess ? ok() : hip_fail(e, "hipEventSynchronize");
}

int wxo_event_elapsed_ms(float* ms, wxo_event_t start, wxo_event_t stop) {
    if (!ms) return fail(WXO_ERR_INVALID, "ms is NULL");
    hipError_t e = hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop));
    return e == hipSuccess ? ok() : hip_fail(e, "hipEventElapsedTime");
}

namespace {
// Waits `ticks` of the 100 MHz real-time counter; every lane leaves once the
// counter has moved that far, whatever the shader clock does meanwhile.
__global__ __launch_bounds__(64) void spin_kernel(uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

// Waits until the host has released gate `gen` (the flag has reached it; the
// difference taken as signed, so the count may wrap) or `ticks` of the 100 MHz
// counter have passed.  The flag lives in coherent page-locked host memory and
// is read with system-scope loads (they bypass the GPU's caches), so each poll
// sees the host's latest store.  Relaxed: nothing after the wait depends on
// the flag's ordering (stream order carries the work behind the gate), and an
// acquire would invalidate the caches on every poll.
__global__ __launch_bounds__(64) void gate_kernel(const uint32_t* flag, uint32_t gen, uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while ((int32_t)(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) - gen) < 0 &&
           __builtin_amdgcn_s_memrealtime() - t0 < ticks)
        __builtin_amdgcn_s_sleep(2);
}

// One flag per process: hold hands out the next number, release raises the
// flag to it (never lowers it).
std::mutex g_gate_mu;
uint32_t* g_gate_host = nullptr;   // the flag, as the host writes it
uint32_t* g_gate_dev = nullptr;    // the same flag, as kernels read it
uint32_t g_gate_next = 0;
}  // namespace

int wxo_graph_capture_begin(wxo_stream_t stream) {
    if (!stream) return fail(WXO_ERR_INVALID, "graph capture needs a stream of its own, not the null stream");
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipError_t e = hipStreamBeginCapture(as_hip(stream), hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? ok() : hip_fail(e, "hipStreamBeginCapture");
}

int wxo_graph_capture_end(wxo_stream_t stream, wxo_graph_t* graph) {
    if (!graph) return fail(WXO_ERR_INVALID, "graph is NULL");
    *graph = nullptr;
    if (!stream) return fail(WXO_ERR_INVALID, "graph capture needs a stream of its own, not the null stream");
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(as_hip(stream), &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return hip_fail(e, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph = reinterpret_cast<wxo_graph_t>(exec);
    return ok();
}

int wxo_graph_launch(wxo_graph_t graph, wxo_stream_t stream) {
    if (!graph) return fail(WXO_ERR_INVALID, "graph is NULL");
    hipError_t e = hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), as_hip(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "hipGraphLaunch");
}

int wxo_graph_destroy(wxo_graph_t graph) {
    if (!graph) return ok();
    hipError_t e = hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph));
    return e == hipSuccess ? ok() : hip_fail(e, "hipGraphExecDestroy");
}

int wxo_spin(uint32_t us, wxo_stream_t stream) {
    if (us > 1000000u) return fail(WXO_ERR_INVALID, "spin longer than 1 s");
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(64), 0, as_hip(stream), (uint64_t)us * 100u);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ok() : hip_fail(e, "spin launch");
}

int wxo_gate_hold(uint32_t max_us, wxo_stream_t stream, uint32_t* gate) {
    if (!gate) return fail(WXO_ERR_INVALID, "gate is NULL");
    if (max_us > 1000000u) return fail(WXO_ERR_INVALID, "gate held longer than 1 s");
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    std::lock_guard<std::mutex> lock(g_gate_mu);
    if (!g_gate_host) {
        void* h = nullptr;
        hipError_t e = hipHostMalloc(&h, 64, hipHostMallocCoherent | hipHostMallocMapped | hipHostMallocPortable);
        if (e != hipSuccess) return hip_fail(e, "hipHostMalloc (gate flag)");
        void* dp = nullptr;
        e = hipHostGetDevicePointer(&dp, h, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(h);
            return hip_fail(e, "hipHostGetDevicePointer (gate flag)");
        }
        g_gate_host = static_cast<uint32_t*>(h);
        g_gate_dev = static_cast<uint32_t*>(dp);
        __atomic_store_n(g_gate_host, 0u, __ATOMIC_RELEASE);
    }
    const uint32_t gen = g_gate_next + 1u;
    hipLaunchKernelGGL(gate_kernel, dim3(1), dim3(64), 0, as_hip(stream), (const uint32_t*)g_gate_dev, gen,
                       (uint64_t)max_us * 100u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "gate launch");
    g_gate_next = gen;
    *gate = gen;
    return ok();
}

int wxo_gate_release(uint32_t gate) {
    std::lock_guard<std::mutex> lock(g_gate_mu);
    if (!g_gate_host || (int32_t)(gate - g_gate_next) > 0 || gate == 0u)
        return fail(WXO_ERR_INVALID, "gate %u was never held", gate);
    const uint32_t cur = __atomic_load_n(g_gate_host, __ATOMIC_ACQUIRE);
    if ((int32_t)(gate - cur) > 0) __atomic_store_n(g_gate_host, gate, __ATOMIC_RELEASE);
    return ok();
}

int wxo_roofline(double* bandwidth, double* compute) {
    if (!bandwidth && !compute) return fail(WXO_ERR_INVALID, "roofline: give bandwidth, compute or both");
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    double bw = 0.0, fl = 0.0;
    const hipError_t e = wxo::measure_roofline(*d, bandwidth ? &bw : nullptr, compute ? &fl : nullptr);
    if (e != hipSuccess) return hip_fail(e, "roofline measurement");
    if (bandwidth) *bandwidth = bw;
    if (compute) *compute = fl;
    return ok();
}

int wxo_roofline_matrix(double* flops) {
    if (!flops) return fail(WXO_ERR_INVALID, "roofline_matrix: flops is NULL");
    *flops = 0.0;
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    double fl = 0.0;
    const hipError_t e = wxo::measure_matrix_ceiling(*d, &fl);
    if (e != hipSuccess) return hip_fail(e, "roofline_matrix measurement");
    *flops = fl;
    return ok();
}

// ---- ops on device pointers ------------------------------------------------

int wxo_matvec_q8(const uint32_t* weight, const float* scale, const float* vector, float* output, uint32_t N,
                  uint32_t K, uint32_t M, wxo_stream_t stream) {
    WXO_TRY(validate_matvec(weight, scale, vector, output, N, K, M));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    wxo::MatvecArgs a{weight, scale, vector, output, N, K, M, (uint32_t)(((uint64_t)K + 3) / 4)};
    wxo::Variant v = N == 0 ? wxo::Variant{} : named("fill_scaled_zero", "K=0");
    hipError_t e = wxo::launch_matvec_q8(a, *d, as_hip(stream), &v);
    return launched(e, v, "matvec_q8 launch");
}

int wxo_matvec_q8_multi(const uint32_t* const* weights, const float* const* scales, float* const* outputs,
                        const uint32_t* Ns, uint32_t count, const float* vector, uint32_t K, wxo_stream_t stream) {
    if (count == 0) return ok();
    if (!weights || !scales || !outputs || !Ns) return fail(WXO_ERR_INVALID, "projection arrays are NULL");
    for (uint32_t i = 0; i < count; ++i) {
        if (validate_matvec(weights[i], scales[i], vector, outputs[i], Ns[i], K, 1) != WXO_OK) {
            char why[256];
            snprintf(why, sizeof why, "%s", g_error);
            return fail(WXO_ERR_INVALID, "projection %u: %s", i, why);
        }
    }
    // The projections run concurrently: an output that overlaps the vector,
    // another output or any projection's weight or scale would make the
    // result depend on the schedule.
    const uint64_t W = ((uint64_t)K + 3) / 4;
    const auto meet = [](const void* p, uint64_t pb, const void* q, uint64_t qb) {
        const uintptr_t p0 = (uintptr_t)p, q0 = (uintptr_t)q;
        return pb > 0 && qb > 0 && p0 < q0 + qb && q0 < p0 + pb;
    };
    for (uint32_t i = 0; i < count; ++i) {
        const uint64_t ob = (uint64_t)Ns[i] * 4u;
        if (meet(outputs[i], ob, vector, (uint64_t)K * 4u))
            return fail(WXO_ERR_INVALID, "projection %u: output overlaps the vector", i);
        for (uint32_t j = 0; j < count; ++j) {
            if (j < i && meet(outputs[i], ob, outputs[j], (uint64_t)Ns[j] * 4u))
                return fail(WXO_ERR_INVALID, "outputs of projections %u and %u overlap", j, i);
            if (meet(outputs[i], ob, weights[j], (uint64_t)Ns[j] * W * 4u) ||
                meet(outputs[i], ob, scales[j], (uint64_t)Ns[j] * 4u))
                return fail(WXO_ERR_INVALID, "projection %u: output overlaps the weight or scale of projection %u", i, j);
        }
    }
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    for (uint32_t g = 0; g < count; g += wxo::kMaxProjections) {
        wxo::Projection p[wxo::kMaxProjections];
        const uint32_t n = count - g < wxo::kMaxProjections ? count - g : wxo::kMaxProjections;
        for (uint32_t i = 0; i < n; ++i) p[i] = {weights[g + i], scales[g + i], outputs[g + i], Ns[g + i]};
        wxo::Variant v = named("fill_scaled_zero", "K=0");
        hipError_t e = wxo::launch_matvec_q8_multi(p, n, vector, K, *d, as_hip(stream), &v);
        WXO_TRY(launched(e, v, "matvec_q8_multi launch"));
    }
    return ok();
}

int wxo_matvec_q8_residual(const uint32_t* weight, const float* scale, const float* vector, const float* residual,
                           float* output, uint32_t N, uint32_t K, wxo_stream_t stream) {
    WXO_TRY(validate_matvec(weight, scale, vector, output, N, K, 1));
    WXO_TRY(check_ptr(residual, N, "residual"));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    wxo::MatvecArgs a{weight, scale, vector, output, N, K, 1, (uint32_t)(((uint64_t)K + 3) / 4)};
    a.residual = residual;
    wxo::Variant v = N == 0 ? wxo::Variant{} : named("fused_zero", "residual.K=0");
    hipError_t e = wxo::launch_matvec_q8_fused(a, wxo::kEpiResidual, *d, as_hip(stream), &v);
    return launched(e, v, "matvec_q8_residual launch");
}

int wxo_matvec_q8_ffn(const uint32_t* weight_gate, const float* scale_gate, const uint32_t* weight_up,
                      const float* scale_up, const float* vector, float* output, uint32_t N, uint32_t K,
                      wxo_stream_t stream) {
    WXO_TRY(validate_matvec(weight_gate, scale_gate, vector, output, N, K, 1));
    WXO_TRY(check_ptr(weight_up, (uint64_t)N * (((uint64_t)K + 3) / 4), "weight_up"));
    WXO_TRY(check_ptr(scale_up, N, "scale_up"));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    wxo::MatvecArgs a{weight_gate, scale_gate, vector, output, N, K, 1, (uint32_t)(((uint64_t)K + 3) / 4)};
    a.weight2 = weight_up;
    a.scale2 = scale_up;
    wxo::Variant v = N == 0 ? wxo::Variant{} : named("fused_zero", "ffn.K=0");
    hipError_t e = wxo::launch_matvec_q8_fused(a, wxo::kEpiFfn, *d, as_hip(stream), &v);
    return launched(e, v, "matvec_q8_ffn launch");
}

int wxo_quantize(const float* input, uint32_t N, uint32_t D, int32_t* output, float* scales, wxo_stream_t stream) {
    WXO_TRY(validate_rows(input, N, D, "input"));
    WXO_TRY(check_ptr(output, (uint64_t)N * D, "output"));
    WXO_TRY(check_ptr(scales, N, "scales"));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    wxo::Variant v;
    hipError_t e = wxo::launch_quantize_rows(input, N, D, output, nullptr, scales, *d, as_hip(stream), &v);
    return launched(e, v, "quantize launch");
}

int wxo_pack_q8(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed, wxo_stream_t stream) {
    WXO_TRY(validate_rows(codes, N, K, "codes"));
    WXO_TRY(check_ptr(packed, (uint64_t)N * (((uint64_t)K + 3) / 4), "packed"));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipError_t e = wxo::launch_pack_q8(codes, N, K, packed, *d, as_hip(stream));
    return launched(e, N && K ? named("pack_q8") : wxo::Variant{}, "pack_q8 launch");
}

int wxo_pack_int8_rows(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed, wxo_stream_t stream) {
    WXO_TRY(validate_rows(codes, N, K, "codes"));
    WXO_TRY(check_ptr(packed, (uint64_t)N * (((uint64_t)K + 3) / 4), "packed"));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipError_t e = wxo::launch_pack_int8_rows(codes, N, K, packed, *d, as_hip(stream));
    return launched(e, N && K ? named("pack_int8_rows") : wxo::Variant{}, "pack_int8_rows launch");
}

int wxo_quantize_pack_q8(const float* input, uint32_t N, uint32_t K, uint32_t* packed, float* scales,
                         wxo_stream_t stream) {
    WXO_TRY(validate_rows(input, N, K, "input"));
    WXO_TRY(check_ptr(packed, (uint64_t)N * (((uint64_t)K + 3) / 4), "packed"));
    WXO_TRY(check_ptr(scales, N, "scales"));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    wxo::Variant v;
    hipError_t e = wxo::launch_quantize_rows(input, N, K, nullptr, packed, scales, *d, as_hip(stream), &v);
    return launched(e, v, "quantize_pack_q8 launch");
}

int wxo_quantize_pack_q8_multi(const float* const* inputs, const uint32_t* Ns, uint32_t* const* packed,
                               float* const* scales, uint32_t count, uint32_t K, wxo_stream_t stream) {
    if (count == 0) return ok();
    if (!inputs || !Ns || !packed || !scales) return fail(WXO_ERR_INVALID, "matrix arrays are NULL");
    const uint64_t W = ((uint64_t)K + 3) / 4;
    for (uint32_t i = 0; i < count; ++i) {
        int st = validate_rows(inputs[i], Ns[i], K, "input");
        if (st == WXO_OK) st = check_ptr(packed[i], (uint64_t)Ns[i] * W, "packed");
        if (st == WXO_OK) st = check_ptr(scales[i], Ns[i], "scales");
        if (st != WXO_OK) {
            char why[256];
            snprintf(why, sizeof why, "%s", g_error);
            return fail(st, "matrix %u: %s", i, why);
        }
    }
    // The matrices run concurrently: nothing one of them writes may overlap
    // what another reads or writes.
    struct Span {
        uintptr_t lo, hi;
    };
    const auto span = [](const void* p, uint64_t bytes) { return Span{(uintptr_t)p, (uintptr_t)p + bytes}; };
    const auto meet = [](Span a, Span b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; };
    for (uint32_t i = 0; i < count; ++i) {
        const Span outs[2] = {span(packed[i], (uint64_t)Ns[i] * W * 4), span(scales[i], (uint64_t)Ns[i] * 4)};
        if (meet(outs[0], outs[1])) return fail(WXO_ERR_INVALID, "matrix %u: packed and scales overlap", i);
        for (uint32_t j = 0; j < count; ++j) {
            const Span in = span(inputs[j], (uint64_t)Ns[j] * K * 4);
            for (const Span& o : outs) {
                if (meet(o, in)) return fail(WXO_ERR_INVALID, "outputs of matrix %u overlap the input of matrix %u", i, j);
                if (j < i && (meet(o, span(packed[j], (uint64_t)Ns[j] * W * 4)) ||
                              meet(o, span(scales[j], (uint64_t)Ns[j] * 4))))
                    return fail(WXO_ERR_INVALID, "outputs of matrices %u and %u overlap", j, i);
            }
        }
    }
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    for (uint32_t g = 0; g < count; g += wxo::kMaxQuantizeMatrices) {
        const uint32_t n = count - g < wxo::kMaxQuantizeMatrices ? count - g : wxo::kMaxQuantizeMatrices;
        hipError_t e = wxo::launch_quantize_pack_multi(inputs + g, Ns + g, packed + g, scales + g, n, K, *d,
                                                       as_hip(stream));
        WXO_TRY(launched(e, named("quantize_pack_multi"), "quantize_pack_q8_multi launch"));
    }
    return ok();
}

int wxo_matmul_q8(const float* a, const uint32_t* weight, const float* scale, float* output, uint32_t N, uint32_t M,
                  uint32_t K, wxo_stream_t stream) {
    WXO_TRY(validate_matmul(a, weight, scale, output, N, M, K));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    wxo::Variant v;
    hipError_t e = wxo::launch_matmul_q8(a, weight, scale, output, N, M, K, *d, as_hip(stream), &v);
    return launched(e, v, "matmul_q8 launch");
}

namespace {
int matmul_multi(const float* a, const uint32_t* const* weights, const float* const* scales, float* const* outputs,
                 const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K, void* workspace, size_t workspace_bytes,
                 wxo_stream_t stream) {
    if (count == 0) return ok();
    if (!weights || !scales || !outputs || !Ms) return fail(WXO_ERR_INVALID, "projection arrays are NULL");
    for (uint32_t i = 0; i < count; ++i) {
        if (validate_matmul(a, weights[i], scales[i], outputs[i], N, Ms[i], K) != WXO_OK) {
            char why[256];
            snprintf(why, sizeof why, "%s", g_error);
            return fail(WXO_ERR_INVALID, "projection %u: %s", i, why);
        }
    }
    // The projections run concurrently: an output that overlaps the
    // activations, another output or any weight or scale would make the
    // result depend on the schedule.
    const uint64_t W = ((uint64_t)K + 3) / 4;
    const auto meet = [](const void* p, uint64_t pb, const void* q, uint64_t qb) {
        const uintptr_t p0 = (uintptr_t)p, q0 = (uintptr_t)q;
        return pb > 0 && qb > 0 && p0 < q0 + qb && q0 < p0 + pb;
    };
    for (uint32_t i = 0; i < count; ++i) {
        const uint64_t ob = (uint64_t)N * Ms[i] * 4u;
        if (meet(outputs[i], ob, a, (uint64_t)N * K * 4u))
            return fail(WXO_ERR_INVALID, "projection %u: output overlaps the activations", i);
        for (uint32_t j = 0; j < count; ++j) {
            if (j < i && meet(outputs[i], ob, outputs[j], (uint64_t)N * Ms[j] * 4u))
                return fail(WXO_ERR_INVALID, "outputs of projections %u and %u overlap", j, i);
            if (meet(outputs[i], ob, weights[j], (uint64_t)Ms[j] * W * 4u) ||
                meet(outputs[i], ob, scales[j], (uint64_t)Ms[j] * 4u))
                return fail(WXO_ERR_INVALID, "projection %u: output overlaps the weight or scale of projection %u", i, j);
        }
    }
    // The workspace is written while every input is read and every output
    // written: it must touch none of them.
    if (workspace_bytes > 0 && !workspace) return fail(WXO_ERR_INVALID, "workspace is NULL with %zu bytes", workspace_bytes);
    if (workspace && ((uintptr_t)workspace & 15u)) return fail(WXO_ERR_INVALID, "workspace is not 16-byte aligned");
    if (workspace) {
        if (meet(workspace, workspace_bytes, a, (uint64_t)N * K * 4u))
            return fail(WXO_ERR_INVALID, "workspace overlaps the activations");
        for (uint32_t i = 0; i < count; ++i) {
            if (meet(workspace, workspace_bytes, outputs[i], (uint64_t)N * Ms[i] * 4u) ||
                meet(workspace, workspace_bytes, weights[i], (uint64_t)Ms[i] * W * 4u) ||
                meet(workspace, workspace_bytes, scales[i], (uint64_t)Ms[i] * 4u))
                return fail(WXO_ERR_INVALID, "workspace overlaps projection %u's weight, scale or output", i);
        }
    }
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    for (uint32_t g = 0; g < count; g += wxo::kMaxMatmulProjectionsPerLaunch) {
        wxo::MatmulProjection p[wxo::kMaxMatmulProjectionsPerLaunch];
        const uint32_t n = count - g < wxo::kMaxMatmulProjectionsPerLaunch ? count - g : wxo::kMaxMatmulProjectionsPerLaunch;
        for (uint32_t i = 0; i < n; ++i) p[i] = {weights[g + i], scales[g + i], outputs[g + i], Ms[g + i]};
        wxo::Variant v = named("matmul_q8.multi", "empty");
        hipError_t e = wxo::launch_matmul_q8_multi(a, p, n, N, K, *d, as_hip(stream), &v,
                                                   static_cast<float*>(workspace), workspace_bytes);
        WXO_TRY(launched(e, v, "matmul_q8_multi launch"));
    }
    return ok();
}
}  // namespace

int wxo_matmul_q8_multi(const float* a, const uint32_t* const* weights, const float* const* scales,
                        float* const* outputs, const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K,
                        wxo_stream_t stream) {
    return matmul_multi(a, weights, scales, outputs, Ms, count, N, K, nullptr, 0, stream);
}

int wxo_matmul_q8_multi_ws(const float* a, const uint32_t* const* weights, const float* const* scales,
                           float* const* outputs, const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K,
                           void* workspace, size_t workspace_bytes, wxo_stream_t stream) {
    return matmul_multi(a, weights, scales, outputs, Ms, count, N, K, workspace, workspace_bytes, stream);
}

int wxo_matmul_q8_multi_static(const float* a, const uint32_t* const* weights, const float* const* scales,
                               float* const* outputs, const uint32_t* Ms, uint32_t count, uint32_t N, uint32_t K,
                               wxo_stream_t stream) {
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    void* ws = g_scratch[d->ordinal];
    if (!ws) {
        return fail(WXO_ERR_DEVICE, "the library's scratch array on device %d is unavailable (hipGetSymbolAddress: %s)",
                    d->ordinal, hipGetErrorString(g_scratch_err[d->ordinal]));
    }
    return matmul_multi(a, weights, scales, outputs, Ms, count, N, K, ws, kScratchBytes, stream);
}

int wxo_matmul_q8_workspace_bytes(size_t* bytes) {
    if (!bytes) return fail(WXO_ERR_INVALID, "bytes is NULL");
    *bytes = 0;
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    *bytes = (size_t)(d->cu_count > 0 ? d->cu_count : 256) * wxo::kMatmulWorkspaceBytesPerCu;
    return ok();
}

int wxo_dequantize_packed_q8(const uint32_t* weight, const float* scale, uint32_t N, uint32_t K, float* output,
                             wxo_stream_t stream) {
    WXO_TRY(validate_dequant(weight, scale, output, N, K));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipError_t e = wxo::launch_dequantize_packed(weight, scale, N, K, output, *d, as_hip(stream));
    return launched(e, N && K ? named("dequantize_packed") : wxo::Variant{}, "dequantize_packed_q8 launch");
}

int wxo_dequant_transpose(const uint32_t* weight, const float* scale, uint32_t out_features, uint32_t in_features,
                          float* output, wxo_stream_t stream) {
    WXO_TRY(validate_dequant(weight, scale, output, out_features, in_features));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipError_t e = wxo::launch_dequant_transpose(weight, scale, out_features, in_features, output, as_hip(stream));
    return launched(e, out_features && in_features ? named("dequant_transpose") : wxo::Variant{},
                    "dequant_transpose launch");
}

int wxo_gather_dequant_rows(const int8_t* codes, const float* scale, uint32_t rows, uint32_t D,
                            const int64_t* indices, uint32_t count, float* output, wxo_stream_t stream) {
    WXO_TRY(validate_gather(codes, scale, indices, output, rows, D, count));
    const wxo::DeviceInfo* d = nullptr;
    WXO_TRY(current_device(&d));
    hipError_t e = wxo::launch_gather_dequant_rows(codes, scale, rows, D, indices, count, output, *d, as_hip(stream));
    return launched(e, count && D ? named("gather_dequant_rows") : wxo::Variant{}, "gather_dequant_rows launch");
}

// ---- host-array forms ----------------------------------------------------------

int wxo_matvec_q8_host(const uint32_t* weight, const float* scale, const float* vector, float* output, uint32_t N,
                       uint32_t K, uint32_t M) {
    WXO_TRY(validate_matvec(weight, scale, vector, output, N, K, M));
    const size_t W = ((size_t)K + 3) / 4;
    DevBuf w, s, x, y;
    WXO_TRY(w.alloc((size_t)N * W * 4));
    WXO_TRY(s.alloc((size_t)N * 4));
    WXO_TRY(x.alloc((size_t)M * K * 4));
    WXO_TRY(y.alloc((size_t)M * N * 4));
    WXO_TRY(w.upload(weight, (size_t)N * W * 4));
    WXO_TRY(s.upload(scale, (size_t)N * 4));
    WXO_TRY(x.upload(vector, (size_t)M * K * 4));
    WXO_TRY(wxo_matvec_q8((const uint32_t*)w.p, (const float*)s.p, (const float*)x.p, (float*)y.p, N, K, M, nullptr));
    return y.download(output, (size_t)M * N * 4) == WXO_OK ? ok() : WXO_ERR_DEVICE;
}

int wxo_matvec_q8_residual_host(const uint32_t* weight, const float* scale, const float* vector, const float* residual,
                                float* output, uint32_t N, uint32_t K) {
    WXO_TRY(validate_matvec(weight, scale, vector, output, N, K, 1));
    WXO_TRY(check_ptr(residual, N, "residual"));
    const size_t W = ((size_t)K + 3) / 4;
    DevBuf w, s, x, r, y;
    WXO_TRY(w.alloc((size_t)N * W * 4));
    WXO_TRY(s.alloc((size_t)N * 4));
    WXO_TRY(x.alloc((size_t)K * 4));
    WXO_TRY(r.alloc((size_t)N * 4));
    WXO_TRY(y.alloc((size_t)N * 4));
    WXO_TRY(w.upload(weight, (size_t)N * W * 4));
    WXO_TRY(s.upload(scale, (size_t)N * 4));
    WXO_TRY(x.upload(vector, (size_t)K * 4));
    WXO_TRY(r.upload(residual, (size_t)N * 4));
    WXO_TRY(wxo_matvec_q8_residual((const uint32_t*)w.p, (const float*)s.p, (const float*)x.p, (const float*)r.p,
                                   (float*)y.p, N, K, nullptr));
    WXO_TRY(y.download(output, (size_t)N * 4));
    return ok();
}

int wxo_matvec_q8_ffn_host(const uint32_t* weight_gate, const float* scale_gate, const uint32_t* weight_up,
                           const float* scale_up, const float* vector, float* output, uint32_t N, uint32_t K) {
    WXO_TRY(validate_matvec(weight_gate, scale_gate, vector, output, N, K, 1));
    const size_t W = ((size_t)K + 3) / 4;
    WXO_TRY(check_ptr(weight_up, (uint64_t)N * W, "weight_up"));
    WXO_TRY(check_ptr(scale_up, N, "scale_up"));
    DevBuf wg, sg, wu, su, x, y;
    WXO_TRY(wg.alloc((size_t)N * W * 4));
    WXO_TRY(sg.alloc((size_t)N * 4));
    WXO_TRY(wu.alloc((size_t)N * W * 4));
    WXO_TRY(su.alloc((size_t)N * 4));
    WXO_TRY(x.alloc((size_t)K * 4));
    WXO_TRY(y.alloc((size_t)N * 4));
    WXO_TRY(wg.upload(weight_gate, (size_t)N * W * 4));
    WXO_TRY(sg.upload(scale_gate, (size_t)N * 4));
    WXO_TRY(wu.upload(weight_up, (size_t)N * W * 4));
    WXO_TRY(su.upload(scale_up, (size_t)N * 4));
    WXO_TRY(x.upload(vector, (size_t)K * 4));
    WXO_TRY(wxo_matvec_q8_ffn((const uint32_t*)wg.p, (const float*)sg.p, (const uint32_t*)wu.p, (const float*)su.p,
                              (const float*)x.p, (float*)y.p, N, K, nullptr));
    WXO_TRY(y.download(output, (size_t)N * 4));
    return ok();
}

int wxo_quantize_host(const float* input, uint32_t N, uint32_t D, int32_t* output, float* scales) {
    WXO_TRY(validate_rows(input, N, D, "input"));
    WXO_TRY(check_ptr(output, (uint64_t)N * D, "output"));
    WXO_TRY(check_ptr(scales, N, "scales"));
    DevBuf in, out, sc;
    WXO_TRY(in.alloc((size_t)N * D * 4));
    WXO_TRY(out.alloc((size_t)N * D * 4));
    WXO_TRY(sc.alloc((size_t)N * 4));
    WXO_TRY(in.upload(input, (size_t)N * D * 4));
    WXO_TRY(wxo_quantize((const float*)in.p, N, D, (int32_t*)out.p, (float*)sc.p, nullptr));
    WXO_TRY(out.download(output, (size_t)N * D * 4));
    WXO_TRY(sc.download(scales, (size_t)N * 4));
    return ok();
}

int wxo_pack_q8_host(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed) {
    WXO_TRY(validate_rows(codes, N, K, "codes"));
    const size_t W = ((size_t)K + 3) / 4;
    WXO_TRY(check_ptr(packed, (uint64_t)N * W, "packed"));
    DevBuf c, p;
    WXO_TRY(c.alloc((size_t)N * K * 4));
    WXO_TRY(p.alloc((size_t)N * W * 4));
    WXO_TRY(c.upload(codes, (size_t)N * K * 4));
    WXO_TRY(wxo_pack_q8((const int32_t*)c.p, N, K, (uint32_t*)p.p, nullptr));
    WXO_TRY(p.download(packed, (size_t)N * W * 4));
    return ok();
}

int wxo_pack_int8_rows_host(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed) {
    WXO_TRY(validate_rows(codes, N, K, "codes"));
    const size_t W = ((size_t)K + 3) / 4;
    WXO_TRY(check_ptr(packed, (uint64_t)N * W, "packed"));
    DevBuf c, p;
    WXO_TRY(c.alloc((size_t)N * K));
    WXO_TRY(p.alloc((size_t)N * W * 4));
    WXO_TRY(c.upload(codes, (size_t)N * K));
    WXO_TRY(wxo_pack_int8_rows((const int8_t*)c.p, N, K, (uint32_t*)p.p, nullptr));
    WXO_TRY(p.download(packed, (size_t)N * W * 4));
    return ok();
}

int wxo_quantize_pack_q8_host(const float* input, uint32_t N, uint32_t K, uint32_t* packed, float* scales) {
    WXO_TRY(validate_rows(input, N, K, "input"));
    const size_t W = ((size_t)K + 3) / 4;
    WXO_TRY(check_ptr(packed, (uint64_t)N * W, "packed"));
    WXO_TRY(check_ptr(scales, N, "scales"));
    DevBuf in, p, sc;
    WXO_TRY(in.alloc((size_t)N * K * 4));
    WXO_TRY(p.alloc((size_t)N * W * 4));
    WXO_TRY(sc.alloc((size_t)N * 4));
    WXO_TRY(in.upload(input, (size_t)N * K * 4));
    WXO_TRY(wxo_quantize_pack_q8((const float*)in.p, N, K, (uint32_t*)p.p, (float*)sc.p, nullptr));
    WXO_TRY(p.download(packed, (size_t)N * W * 4));
    WXO_TRY(sc.download(scales, (size_t)N * 4));
    return ok();
}

int wxo_matmul_q8_host(const float* a, const uint32_t* weight, const float* scale, float* output, uint32_t N,
                       uint32_t M, uint32_t K) {
    WXO_TRY(validate_matmul(a, weight, scale, output, N, M, K));
    const size_t W = ((size_t)K + 3) / 4;
    DevBuf da, w, s, y;
    WXO_TRY(da.alloc((size_t)N * K * 4));
    WXO_TRY(w.alloc((size_t)M * W * 4));
    WXO_TRY(s.alloc((size_t)M * 4));
    WXO_TRY(y.alloc((size_t)N * M * 4));
    WXO_TRY(da.upload(a, (size_t)N * K * 4));
    WXO_TRY(w.upload(weight, (size_t)M * W * 4));
    WXO_TRY(s.upload(scale, (size_t)M * 4));
    WXO_TRY(wxo_matmul_q8((const float*)da.p, (const uint32_t*)w.p, (const float*)s.p, (float*)y.p, N, M, K, nullptr));
    WXO_TRY(y.download(output, (size_t)N * M * 4));
    return ok();
}

int wxo_dequantize_packed_q8_host(const uint32_t* weight, const float* scale, uint32_t N, uint32_t K, float* output) {
    WXO_TRY(validate_dequant(weight, scale, output, N, K));
    const size_t W = ((size_t)K + 3) / 4;
    DevBuf w, s, y;
    WXO_TRY(w.alloc((size_t)N * W * 4));
    WXO_TRY(s.alloc((size_t)N * 4));
    WXO_TRY(y.alloc((size_t)N * K * 4));
    WXO_TRY(w.upload(weight, (size_t)N * W * 4));
    WXO_TRY(s.upload(scale, (size_t)N * 4));
    WXO_TRY(wxo_dequantize_packed_q8((const uint32_t*)w.p, (const float*)s.p, N, K, (float*)y.p, nullptr));
    WXO_TRY(y.download(output, (size_t)N * K * 4));
    return ok();
}

int wxo_dequant_transpose_host(const uint32_t* weight, const float* scale, uint32_t out_features,
                               uint32_t in_features, float* output) {
    WXO_TRY(validate_dequant(weight, scale, output, out_features, in_features));
    const size_t W = ((size_t)in_features + 3) / 4;
    DevBuf w, s, y;
    WXO_TRY(w.alloc((size_t)out_features * W * 4));
    WXO_TRY(s.alloc((size_t)out_features * 4));
    WXO_TRY(y.alloc((size_t)out_features * in_features * 4));
    WXO_TRY(w.upload(weight, (size_t)out_features * W * 4));
    WXO_TRY(s.upload(scale, (size_t)out_features * 4));
    WXO_TRY(wxo_dequant_transpose((const uint32_t*)w.p, (const float*)s.p, out_features, in_features, (float*)y.p,
                                  nullptr));
    WXO_TRY(y.download(output, (size_t)out_features * in_features * 4));
    return ok();
}

int wxo_gather_dequant_rows_host(const int8_t* codes, const float* scale, uint32_t rows, uint32_t D,
                                 const int64_t* indices, uint32_t count, float* output) {
    WXO_TRY(validate_gather(codes, scale, indices, output, rows, D, count));
    DevBuf c, s, ix, y;
    WXO_TRY(c.alloc((size_t)rows * D));
    WXO_TRY(s.alloc((size_t)rows * 4));
    WXO_TRY(ix.alloc((size_t)count * 8));
    WXO_TRY(y.alloc((size_t)count * D * 4));
    WXO_TRY(c.upload(codes, (size_t)rows * D));
    WXO_TRY(s.upload(scale, (size_t)rows * 4));
    WXO_TRY(ix.upload(indices, (size_t)count * 8));
    WXO_TRY(wxo_gather_dequant_rows((const int8_t*)c.p, (const float*)s.p, rows, D, (const int64_t*)ix.p, count,
                                    (float*)y.p, nullptr));
    WXO_TRY(y.download(output, (size_t)count * D * 4));
    return ok();
}

}  // extern "C"
