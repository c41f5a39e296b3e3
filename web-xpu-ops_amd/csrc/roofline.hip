// roofline.hip -- this device's own ceilings, measured now: the best sustained
// read bandwidth from HBM and the best sustained f32 FMA rate.
//
// Reference method: harness/roofline.ts:162-198 (measureRoofline): fill a
// 512 MiB buffer with values that cannot be compressed (:46-68), sweep it
// exactly once per timed dispatch with the widest loads (:70-101; 512 MiB at
// :33), time FMAs out of registers in independent chains (:103-130), keep the
// fastest of a few attempts after a warm-up (:139-153).  The same method,
// built for gfx950:
//
//  * Two 512 MiB buffers, each filled by a hash of its word index, both swept
//    once before anything is timed.  A timed region sweeps them alternately,
//    so every sweep's data was last read 512 MiB earlier: twice the 256 MB
//    Infinity Cache, so no sweep is served from it, and no page is first
//    touched inside the region.
//  * The sweep: each workgroup reads one contiguous block with every load in
//    flight at once (each lane U buffer_load_dwordx4 of its own 16 bytes at a
//    1 KiB stride, like the matvec kernel's chunk loads), then folds the words
//    and stores only under a condition that never holds.  Two block sizes are
//    timed (U = 8 and 16 loads per lane) and the faster counts, as a ceiling
//    is a best case.
//  * Events around the region bracket the sweeps back to back behind a spin,
//    so the host's issue rate is not in it; each sweep's launch cost is (it is
//    part of what any kernel pays).
//  * The FMA chains: 8 independent chains per lane, 8 waves per SIMD, no
//    memory.  This build disables packed f32 instructions, so the figure is the
//    rate of one-wide v_fma_f32.
//
// The matrix cores (measure_matrix_ceiling; the reference measures no matrix
// rate): v_mfma_f32_16x16x32_bf16 on every CU, one workgroup of 8 waves per
// CU (two per SIMD, as the prefill GEMM runs), 8 independent accumulators per
// wave over operands loaded once.  The clock sags under matrix work by how
// much the operands' bits toggle, so the operands are the GEMM's own kinds:
// A holds int8 codes in bf16, B bf16 values of random sign and mantissa with
// exponents over 2^-8 .. 2^1 (an activation's split parts).  Each launch runs
// ~1 ms; the fastest of three after a warm-up counts.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"
#include "wave_ops.hpp"

namespace wxo {

namespace {

// MurmurHash3's 32-bit finaliser (fmix32) of the word index: every word
// differs from its neighbours in about half its bits.
__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
    h ^= h >> 16;
    h *= 0x85ebca6bu;
    h ^= h >> 13;
    h *= 0xc2b2ae35u;
    h ^= h >> 16;
    return h;
}

__global__ __launch_bounds__(256) void fill_hash_kernel(uint32_t* __restrict__ data, uint64_t words, uint32_t seed) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride)
        data[i] = fmix32((uint32_t)i ^ seed) ^ (uint32_t)(i >> 32);
}

// One block of 256 * 16 * U bytes per workgroup: wave w reads U consecutive
// KiB, lane l the 16 bytes at l * 16 of each.  Offsets past `bytes` read 0.
template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint32_t* __restrict__ data, uint32_t bytes,
                                                          uint32_t guard, uint32_t* sink) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(data, bytes);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = (int)(threadIdx.x & 63u);
    const int base = (int)(blockIdx.x * (256u * 16u * (uint32_t)U) + wave * (1024u * (uint32_t)U));
    u32x4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load_nt_b128(rs, lane * 16, base + u * 1024);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == guard) sink[threadIdx.x] = acc;
}

constexpr int kFmaChains = 8;

__global__ __launch_bounds__(256) void fma_chain_kernel(float seed, uint32_t iterations, float* sink) {
    float c[kFmaChains];
#pragma unroll
    for (int j = 0; j < kFmaChains; ++j) c[j] = seed + (float)j;
    const float k = seed * 0.5f + 1.0f;
#pragma unroll 4
    for (uint32_t i = 0; i < iterations; ++i) {
#pragma unroll
        for (int j = 0; j < kFmaChains; ++j) c[j] = __builtin_fmaf(c[j], k, 1.0f);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kFmaChains; ++j) s += c[j];
    if (s == seed - 999.0f) sink[threadIdx.x] = s;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kMatrixVectors = 65536;  // 16-byte operand vectors, 1 MiB
constexpr int kMatrixA = 2, kMatrixB = 4;   // a wave's operands: 8 accumulators

// Operand vector v (4 words, 8 bf16): even v codes, odd v activation parts.
__global__ __launch_bounds__(256) void fill_matrix_operands_kernel(uint32_t* __restrict__ ops, uint32_t seed) {
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < 4u * kMatrixVectors; i += gridDim.x * 256u) {
        const uint32_t h = fmix32(i * 0x9e3779b9u + seed);
        uint32_t lo, hi;
        if (((i >> 2) & 1u) == 0u) {
            lo = __float_as_uint((float)(int8_t)h) >> 16;  // exact in bf16
            hi = __float_as_uint((float)(int8_t)(h >> 8)) >> 16;
        } else {
            lo = ((h & 1u) << 15) | ((119u + ((h >> 1) & 0xffu) % 10u) << 7) | ((h >> 9) & 0x7fu);
            hi = (((h >> 16) & 1u) << 15) | ((119u + ((h >> 17) & 0xffu) % 10u) << 7) | ((h >> 25) & 0x7fu);
        }
        ops[i] = lo | (hi << 16);
    }
}

__global__ __launch_bounds__(512) void matrix_rate_kernel(const uint32_t* __restrict__ ops, uint32_t iterations,
                                                          float* sink) {
    const uint32_t t = blockIdx.x * 512u + threadIdx.x;
    const uint4* v = reinterpret_cast<const uint4*>(ops);
    bf16x8 a[kMatrixA], b[kMatrixB];
#pragma unroll
    for (int i = 0; i < kMatrixA; ++i) a[i] = __builtin_bit_cast(bf16x8, v[(2u * (t * 4u + (uint32_t)i)) % kMatrixVectors]);
#pragma unroll
    for (int j = 0; j < kMatrixB; ++j)
        b[j] = __builtin_bit_cast(bf16x8, v[(2u * (t * 4u + (uint32_t)j) + 1u) % kMatrixVectors]);
    f32x4 c[kMatrixA][kMatrixB];
#pragma unroll
    for (int i = 0; i < kMatrixA; ++i)
#pragma unroll
        for (int j = 0; j < kMatrixB; ++j) c[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t it = 0; it < iterations; ++it) {
#pragma unroll
        for (int i = 0; i < kMatrixA; ++i)
#pragma unroll
            for (int j = 0; j < kMatrixB; ++j) c[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], c[i][j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kMatrixA; ++i)
#pragma unroll
        for (int j = 0; j < kMatrixB; ++j) s += c[i][j][0] + c[i][j][1] + c[i][j][2] + c[i][j][3];
    if (s == 1234.5f) sink[threadIdx.x] = s;  // keeps the work; the sums never reach it
}

__global__ __launch_bounds__(64) void roofline_spin_kernel(uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

constexpr uint32_t kStreamBytes = 512u << 20;
constexpr int kSweepsPerRegion = 8;
constexpr int kRegions = 3;
constexpr uint32_t kNever = 4042322160u;  // a fold the hashed data does not give

struct Scope {
    hipStream_t stream = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    void* buf[2] = {nullptr, nullptr};
    uint32_t* sink = nullptr;
    ~Scope() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (void* b : buf)
            if (b) (void)hipFree(b);
        if (sink) (void)hipFree(sink);
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

#define RF_TRY(x)                           \
    do {                                    \
        const hipError_t e_ = (x);          \
        if (e_ != hipSuccess) return e_;    \
    } while (0)

template <int U>
hipError_t launch_sweep(const Scope& s, int which) {
    constexpr uint32_t block = 256u * 16u * (uint32_t)U;
    hipLaunchKernelGGL((stream_read_kernel<U>), dim3((kStreamBytes + block - 1) / block), dim3(256), 0, s.stream,
                       static_cast<const uint32_t*>(s.buf[which]), kStreamBytes, kNever, s.sink);
    return hipGetLastError();
}

// Fastest region of kSweepsPerRegion back-to-back sweeps, alternating buffers,
// queued behind a spin; seconds per sweep.
template <int U>
hipError_t time_sweeps(const Scope& s, double* seconds) {
    double best = 1e30;
    for (int r = 0; r < kRegions; ++r) {
        RF_TRY(hipStreamSynchronize(s.stream));
        hipLaunchKernelGGL(roofline_spin_kernel, dim3(1), dim3(64), 0, s.stream, (uint64_t)300u * 100u);
        RF_TRY(hipGetLastError());
        RF_TRY(launch_sweep<U>(s, 0));  // untimed lead: the region opens behind running work
        RF_TRY(hipEventRecord(s.e0, s.stream));
        for (int i = 0; i < kSweepsPerRegion; ++i) RF_TRY(launch_sweep<U>(s, (i + 1) & 1));
        RF_TRY(hipEventRecord(s.e1, s.stream));
        RF_TRY(hipEventSynchronize(s.e1));
        float ms = 0.0f;
        RF_TRY(hipEventElapsedTime(&ms, s.e0, s.e1));
        const double t = (double)ms * 1e-3 / kSweepsPerRegion;
        if (t > 0.0 && t < best) best = t;
    }
    *seconds = best;
    return hipSuccess;
}

}  // namespace

hipError_t measure_roofline(const DeviceInfo& dev, double* bandwidth, double* compute) {
    Scope s;
    RF_TRY(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
    RF_TRY(hipEventCreateWithFlags(&s.e0, hipEventDisableSystemFence));
    RF_TRY(hipEventCreateWithFlags(&s.e1, hipEventDisableSystemFence));
    RF_TRY(hipMalloc(&s.sink, 256 * sizeof(uint32_t)));
    if (bandwidth) {
        for (int b = 0; b < 2; ++b) {
            RF_TRY(hipMalloc(&s.buf[b], kStreamBytes));
            hipLaunchKernelGGL(fill_hash_kernel, dim3(2048), dim3(256), 0, s.stream, static_cast<uint32_t*>(s.buf[b]),
                               (uint64_t)kStreamBytes / 4u, 0x9e3779b9u * (uint32_t)(b + 1));
            RF_TRY(hipGetLastError());
        }
        RF_TRY(launch_sweep<16>(s, 0));  // warm-up: every page read once before timing
        RF_TRY(launch_sweep<16>(s, 1));
        double t16 = 0.0, t8 = 0.0;
        RF_TRY(time_sweeps<16>(s, &t16));
        RF_TRY(time_sweeps<8>(s, &t8));
        const double t = t16 < t8 ? t16 : t8;
        *bandwidth = (double)kStreamBytes / t;
    }
    if (compute) {
        const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
        const uint32_t groups = cus * 8u;  // 32 waves per CU: 8 per SIMD
        const uint32_t iterations = 4000;
        double best = 1e30;
        for (int r = 0; r < 1 + kRegions; ++r) {
            RF_TRY(hipStreamSynchronize(s.stream));
            RF_TRY(hipEventRecord(s.e0, s.stream));
            hipLaunchKernelGGL(fma_chain_kernel, dim3(groups), dim3(256), 0, s.stream, 1.0001f, iterations,
                               reinterpret_cast<float*>(s.sink));
            RF_TRY(hipGetLastError());
            RF_TRY(hipEventRecord(s.e1, s.stream));
            RF_TRY(hipEventSynchronize(s.e1));
            float ms = 0.0f;
            RF_TRY(hipEventElapsedTime(&ms, s.e0, s.e1));
            if (r > 0 && ms > 0.0f && ms * 1e-3 < best) best = ms * 1e-3;  // r = 0 is the warm-up
        }
        *compute = (double)groups * 256.0 * iterations * kFmaChains * 2.0 / best;
    }
    return hipStreamSynchronize(s.stream);
}

hipError_t measure_matrix_ceiling(const DeviceInfo& dev, double* flops) {
    Scope s;
    RF_TRY(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
    RF_TRY(hipEventCreateWithFlags(&s.e0, hipEventDisableSystemFence));
    RF_TRY(hipEventCreateWithFlags(&s.e1, hipEventDisableSystemFence));
    RF_TRY(hipMalloc(&s.sink, 512 * sizeof(uint32_t)));
    RF_TRY(hipMalloc(&s.buf[0], (size_t)kMatrixVectors * 16u));
    hipLaunchKernelGGL(fill_matrix_operands_kernel, dim3(1024), dim3(256), 0, s.stream,
                       static_cast<uint32_t*>(s.buf[0]), 0x51ed270bu);
    RF_TRY(hipGetLastError());
    const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    const uint32_t iterations = 6000;  // ~1 ms a launch at the sagged clock
    double best = 1e30;
    for (int r = 0; r < 1 + kRegions; ++r) {
        RF_TRY(hipStreamSynchronize(s.stream));
        RF_TRY(hipEventRecord(s.e0, s.stream));
        hipLaunchKernelGGL(matrix_rate_kernel, dim3(cus), dim3(512), 0, s.stream,
                           static_cast<const uint32_t*>(s.buf[0]), iterations, reinterpret_cast<float*>(s.sink));
        RF_TRY(hipGetLastError());
        RF_TRY(hipEventRecord(s.e1, s.stream));
        RF_TRY(hipEventSynchronize(s.e1));
        float ms = 0.0f;
        RF_TRY(hipEventElapsedTime(&ms, s.e0, s.e1));
        if (r > 0 && ms > 0.0f && ms * 1e-3 < best) best = ms * 1e-3;  // r = 0 is the warm-up
    }
    // 8 waves per workgroup, kMatrixA x kMatrixB ops per wave and iteration,
    // 16 x 16 x 32 x 2 flops per op
    *flops = (double)cus * 8.0 * iterations * (kMatrixA * kMatrixB) * 16384.0 / best;
    return hipStreamSynchronize(s.stream);
}

}  // namespace wxo
