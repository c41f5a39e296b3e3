// quantize_q8.hip -- per-row absmax int8 quantization and packQ8 for gfx950.
//
// Reference semantics (bit-exact): ops/quantize/reference.ts:13-38 (quantize)
// and ops/matvec/reference.ts:267-283 (packQ8).  JS evaluates quantize in f64:
//   absmax  = max_k |x_k|           (Math.max: NaN anywhere -> NaN)
//   scale   = absmax === 0 ? 1 : absmax / 127           -> Float32Array (RNE)
//   inverse = absmax === 0 ? 0 : 127 / absmax           (f64)
//   code    = clamp(Math.round(x_k * inverse), -127, 127) -> Int32Array (NaN -> 0)
// Math.round rounds ties toward +Infinity; floor(v) + (v - floor(v) >= 0.5) is
// the same function with no second rounding (v + 0.5 would misround
// 0.49999999999999994).  All of it is evaluated here in f64 exactly as JS
// does; the f64 divides are IEEE correctly rounded (no fast-math).
//
// One wave64 per row: lane l owns packed words l, l + 64, ... (4 codes each),
// loads them as dwordx4 of f32, takes |x| as the bit pattern x & 0x7fffffff
// (ordering non-NaN magnitudes like unsigned integers, with every NaN above
// +Inf) and reduces with a wave-wide v_max_u32 over DPP/permlane: no LDS, no
// barrier.  With the row held in VGPRs (WPL words per lane) the input is read
// once; rows too long for that are read twice (max pass, then code pass).
// The fused form writes the packed u32 words directly, never materialising
// the int32 codes: 4NK + NK + 4N bytes instead of 4NK + 4NK + 4NK + NK + 4N.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kernels.hpp"
#include "wave_ops.hpp"

namespace wxo {

// No contraction anywhere in this function: JS rounds x * inverse to f64
// before `v - floor(v)` sees it; a fused fma(x, inverse, -floor) would decide
// exact .5 ties on the unrounded product and misround them.
__device__ __forceinline__ int32_t js_quantize_code(float x, double inverse) {
#pragma clang fp contract(off)
    const double v = (double)x * inverse;
    if (!(v == v)) return 0;  // NaN (x or inverse) -> Int32Array stores 0
    const double f = floor(v);
    double r = (v - f >= 0.5) ? f + 1.0 : f;
    r = r < -127.0 ? -127.0 : (r > 127.0 ? 127.0 : r);
    return (int32_t)r;  // -0 -> 0
}

__device__ __forceinline__ uint32_t abs_bits_max(u32x4v v, uint32_t m) {
    m = max(m, v.x & 0x7fffffffu);
    m = max(m, v.y & 0x7fffffffu);
    m = max(m, v.z & 0x7fffffffu);
    m = max(m, v.w & 0x7fffffffu);
    return m;
}

// Codes of word w of a row (four values, 0 past K) to the packed word and/or
// the int32 codes.  Stores go through resources that span exactly the row's
// words / codes, so the pieces past W or K are dropped without a branch.
template <bool CODES, bool PACK>
__device__ __forceinline__ void emit_word(u32x4v v, double inverse, uint32_t w, __amdgpu_buffer_rsrc_t crs,
                                          __amdgpu_buffer_rsrc_t prs) {
    const int32_t c0 = js_quantize_code(__uint_as_float(v.x), inverse);
    const int32_t c1 = js_quantize_code(__uint_as_float(v.y), inverse);
    const int32_t c2 = js_quantize_code(__uint_as_float(v.z), inverse);
    const int32_t c3 = js_quantize_code(__uint_as_float(v.w), inverse);
    if constexpr (PACK) {
        // Pad lanes past K were loaded as 0.0 and quantize to 0 (0 * inverse
        // is 0 or NaN), so the word's unused high bytes are zero as packQ8's.
        const uint32_t word = ((uint32_t)c0 & 0xffu) | (((uint32_t)c1 & 0xffu) << 8) |
                              (((uint32_t)c2 & 0xffu) << 16) | (((uint32_t)c3 & 0xffu) << 24);
        __builtin_amdgcn_raw_buffer_store_b32(word, prs, (int)(w * 4u), 0, 0);
    }
    if constexpr (CODES) {
        __builtin_amdgcn_raw_buffer_store_b128(u32x4v{(uint32_t)c0, (uint32_t)c1, (uint32_t)c2, (uint32_t)c3}, crs,
                                               (int)(w * 16u), 0, 0);
    }
}

__device__ __forceinline__ void row_scale(uint32_t amax, float* scale, double* inverse) {
    if (amax == 0u) {
        *scale = 1.0f;
        *inverse = 0.0;
    } else if (amax > 0x7f800000u) {  // a NaN in the row: Math.max propagates it
        *scale = __uint_as_float(0x7fc00000u);
        *inverse = __builtin_nan("");
    } else {
        const double a = (double)__uint_as_float(amax);
        *scale = (float)(a / 127.0);
        *inverse = 127.0 / a;
    }
}

// One wave per row.  Every load is a raw-buffer dwordx4 through a resource
// spanning exactly the row's K floats: gfx950 clamps per dword, so entries
// past K read as 0 and there is no per-lane tail branch (such a branch makes
// the compiler join load sequences of different length and wait for each
// load in turn, one memory round trip per word).
// WPL > 0: the row's words l, l+64, ... (WPL of them) are all requested at
// once and stay in VGPRs.  WPL == 0: any K; two passes over the row, four
// words per lane in flight per pass step.
template <int WPL, bool CODES, bool PACK>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ input, uint32_t N,
                                                            uint32_t K, uint32_t W, int32_t* __restrict__ codes,
                                                            uint32_t* __restrict__ packed,
                                                            float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= N) return;  // wave-uniform; no barriers in this kernel
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(input + (size_t)row * K, K * 4u);
    const __amdgpu_buffer_rsrc_t crs = make_rsrc(CODES ? (const void*)(codes + (size_t)row * K) : nullptr,
                                                 CODES ? K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(PACK ? (const void*)(packed + (size_t)row * W) : nullptr,
                                                 PACK ? W * 4u : 0u);

    uint32_t m = 0;
    constexpr int S = WPL > 0 ? WPL : 1;
    u32x4v v[S];
    if constexpr (WPL > 0) {
#pragma unroll
        for (int i = 0; i < WPL; ++i)
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((lane + 64u * (uint32_t)i) * 16u), 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < WPL; ++i) m = abs_bits_max(v[i], m);
    } else {
        for (uint32_t w = lane; w < W; w += 256u) {
            u32x4v t[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                t[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((w + 64u * (uint32_t)i) * 16u), 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) m = abs_bits_max(t[i], m);
        }
    }
    const uint32_t amax = wave_max_u32(m);
    float scale;
    double inverse;
    row_scale(amax, &scale, &inverse);
    if (lane == 0) scales[row] = scale;

    if constexpr (WPL > 0) {
#pragma unroll
        for (int i = 0; i < WPL; ++i) emit_word<CODES, PACK>(v[i], inverse, lane + 64u * (uint32_t)i, crs, prs);
    } else {
        for (uint32_t w = lane; w < W; w += 256u) {
            u32x4v t[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                t[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((w + 64u * (uint32_t)i) * 16u), 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) emit_word<CODES, PACK>(t[i], inverse, w + 64u * (uint32_t)i, crs, prs);
        }
    }
}

// f32 fast path for one word's codes, exact by construction.  With
// inv32 = fl32(inverse), v32 = fl32(x * inv32) differs from JS's
// v = fl64(x * inverse) by at most 2^-24 |v| (product) + 2^-24 |v| (inverse)
// + 2^-53 |v| < 2^-15 for |v| <= 128, so rint(v32) is the integer nearest v,
// and equals Math.round(v), unless v32 lies within 2^-15 of a half-integer.
// Those words (any lane of the wave) are redone in f64.  The caller uses this
// only when inverse is finite in f32.
template <bool CODES, bool PACK>
__device__ __forceinline__ void emit_word_fast(u32x4v v, float inv32, double inverse, uint32_t w,
                                               __amdgpu_buffer_rsrc_t crs, __amdgpu_buffer_rsrc_t prs) {
    int32_t c[4];
    bool near = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x = __uint_as_float(v[e]);
        const float p = x * inv32;
        const float r = rintf(p);
        near |= fabsf(fabsf(p - r) - 0.5f) < 0x1p-15f;
        const int32_t ci = (int32_t)(p == p ? r : 0.0f);  // NaN -> 0 (Int32Array store), |r| <= 128
        c[e] = min(max(ci, -127), 127);
    }
    if (__builtin_amdgcn_ballot_w64(near) != 0ull) {  // wave-uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) c[e] = js_quantize_code(__uint_as_float(v[e]), inverse);
    }
    if constexpr (PACK) {
        const uint32_t word = ((uint32_t)c[0] & 0xffu) | (((uint32_t)c[1] & 0xffu) << 8) |
                              (((uint32_t)c[2] & 0xffu) << 16) | (((uint32_t)c[3] & 0xffu) << 24);
        __builtin_amdgcn_raw_buffer_store_b32(word, prs, (int)(w * 4u), 0, 0);
    }
    if constexpr (CODES) {
        __builtin_amdgcn_raw_buffer_store_b128(u32x4v{(uint32_t)c[0], (uint32_t)c[1], (uint32_t)c[2], (uint32_t)c[3]},
                                               crs, (int)(w * 16u), 0, 0);
    }
}

// One 256-thread workgroup per row: thread t owns words t, t + 256, ...
// (WPT of them, requested at once through the row's buffer resource), the
// four waves' absmax meet in LDS, and every thread derives scale and inverse
// itself.  A quarter of the codes per lane of the one-wave form keeps the
// compute left after a row's last bytes arrive short.  WPT == 0: any K, two
// passes over the row.
//
// The body is a device function of the row so that the multi-matrix kernel
// below runs it on its own rows.
template <int WPT, bool CODES, bool PACK>
__device__ __forceinline__ void quantize_row_wg(const float* __restrict__ input, uint32_t K, uint32_t W,
                                                int32_t* __restrict__ codes, uint32_t* __restrict__ packed,
                                                float* __restrict__ scales, uint32_t row) {
    __shared__ uint32_t wmax[4];
    const uint32_t t = threadIdx.x;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(input + (size_t)row * K, K * 4u);
    const __amdgpu_buffer_rsrc_t crs = make_rsrc(CODES ? (const void*)(codes + (size_t)row * K) : nullptr,
                                                 CODES ? K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(PACK ? (const void*)(packed + (size_t)row * W) : nullptr,
                                                 PACK ? W * 4u : 0u);
    uint32_t m = 0;
    constexpr int S = WPT > 0 ? WPT : 1;
    u32x4v v[S];
    if constexpr (WPT > 0) {
#pragma unroll
        for (int i = 0; i < WPT; ++i)
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((t + 256u * (uint32_t)i) * 16u), 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < WPT; ++i) m = abs_bits_max(v[i], m);
    } else {
        for (uint32_t w = t; w < W; w += 1024u) {
            u32x4v q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((w + 256u * (uint32_t)i) * 16u), 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) m = abs_bits_max(q[i], m);
        }
    }
    m = wave_max_u32(m);
    if ((t & 63u) == 0u) wmax[t >> 6] = m;
    __syncthreads();
    const uint32_t amax = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
    float scale;
    double inverse;
    row_scale(amax, &scale, &inverse);
    if (t == 0) scales[row] = scale;
    const float inv32 = (float)inverse;
    const bool fast = !isinf(inv32);  // row-uniform

    if constexpr (WPT > 0) {
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const uint32_t w = t + 256u * (uint32_t)i;
            if (fast)
                emit_word_fast<CODES, PACK>(v[i], inv32, inverse, w, crs, prs);
            else
                emit_word<CODES, PACK>(v[i], inverse, w, crs, prs);
        }
    } else {
        for (uint32_t w = t; w < W; w += 1024u) {
            u32x4v q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((w + 256u * (uint32_t)i) * 16u), 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (fast)
                    emit_word_fast<CODES, PACK>(q[i], inv32, inverse, w + 256u * (uint32_t)i, crs, prs);
                else
                    emit_word<CODES, PACK>(q[i], inverse, w + 256u * (uint32_t)i, crs, prs);
            }
        }
    }
}

template <int WPT, bool CODES, bool PACK>
__global__ __launch_bounds__(256) void quantize_row_wg_kernel(const float* __restrict__ input, uint32_t N,
                                                              uint32_t K, uint32_t W, int32_t* __restrict__ codes,
                                                              uint32_t* __restrict__ packed,
                                                              float* __restrict__ scales) {
    (void)N;
    quantize_row_wg<WPT, CODES, PACK>(input, K, W, codes, packed, scales, blockIdx.x);
}

// Several matrices with the same K in one launch (quantize + packQ8): the
// grid is their rows laid end to end, matrix i owning blocks
// [start[i], start[i + 1]); unused entries start at 0xffffffff.  A block
// finds its matrix with wave-uniform compares and runs the one-row body.
struct QuantizeSegments {
    const float* input[kMaxQuantizeMatrices];
    uint32_t* packed[kMaxQuantizeMatrices];
    float* scales[kMaxQuantizeMatrices];
    uint32_t start[kMaxQuantizeMatrices];
};

template <int WPT>
__global__ __launch_bounds__(256) void quantize_pack_multi_kernel(QuantizeSegments seg, uint32_t K, uint32_t W) {
    const uint32_t b = blockIdx.x;
    uint32_t i = 0;
#pragma unroll
    for (uint32_t j = 1; j < kMaxQuantizeMatrices; ++j)
        if (b >= seg.start[j]) i = j;
    quantize_row_wg<WPT, false, true>(seg.input[i], K, W, nullptr, seg.packed[i], seg.scales[i], b - seg.start[i]);
}

namespace {

template <int WPL, bool CODES, bool PACK>
hipError_t launch_q(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed, float* scales,
                    hipStream_t stream) {
    const uint32_t W = (K + 3u) / 4u;
    const uint32_t grid = (N + 3u) / 4u;
    hipLaunchKernelGGL((quantize_rows_kernel<WPL, CODES, PACK>), dim3(grid), dim3(256), 0, stream, input, N, K, W,
                       codes, packed, scales);
    return hipGetLastError();
}

template <int WPT, bool CODES, bool PACK>
hipError_t launch_qwg(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed, float* scales,
                      hipStream_t stream) {
    const uint32_t W = (K + 3u) / 4u;
    hipLaunchKernelGGL((quantize_row_wg_kernel<WPT, CODES, PACK>), dim3(N), dim3(256), 0, stream, input, N, K, W,
                       codes, packed, scales);
    return hipGetLastError();
}

template <bool CODES, bool PACK>
hipError_t dispatch_q(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed, float* scales,
                      hipStream_t stream, Variant* variant) {
    const uint32_t W = (K + 3u) / 4u;
    const char* form = CODES ? (PACK ? "codes+pack" : "codes") : "pack";
    // Short rows: one wave per row (a workgroup per row would leave most of
    // its lanes without a word).
    if (W <= 128u) {
        set_variant(variant, "quantize_rows", form, 4, 4, W <= 64u ? 1 : 2, 0, (N + 3u) / 4u);
        if (W <= 64u) return launch_q<1, CODES, PACK>(input, N, K, codes, packed, scales, stream);
        return launch_q<2, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    }
    const uint32_t wpt = (W + 255u) / 256u;
    set_variant(variant, "quantize_row_wg", form, 4, 1, wpt <= 8 ? (int)(wpt <= 2 ? wpt : wpt <= 4 ? 4 : wpt <= 6 ? 6 : 8) : 0,
                0, N);
    if (wpt <= 1) return launch_qwg<1, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpt <= 2) return launch_qwg<2, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpt <= 4) return launch_qwg<4, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpt <= 6) return launch_qwg<6, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpt <= 8) return launch_qwg<8, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (variant) variant->form = CODES ? (PACK ? "codes+pack.twopass" : "codes.twopass") : "pack.twopass";
    return launch_qwg<0, CODES, PACK>(input, N, K, codes, packed, scales, stream);
}

}  // namespace

namespace {

template <int WPT>
hipError_t launch_qmulti(const QuantizeSegments& seg, uint32_t blocks, uint32_t K, hipStream_t stream) {
    hipLaunchKernelGGL((quantize_pack_multi_kernel<WPT>), dim3(blocks), dim3(256), 0, stream, seg, K, (K + 3u) / 4u);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize_pack_multi(const float* const* inputs, const uint32_t* Ns, uint32_t* const* packed,
                                      float* const* scales, uint32_t count, uint32_t K, const DeviceInfo& dev,
                                      hipStream_t stream) {
    const uint32_t W = (K + 3u) / 4u;
    QuantizeSegments seg;
    uint32_t n = 0;
    uint64_t rows = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (Ns[i] == 0) continue;
        if (n == kMaxQuantizeMatrices) return hipErrorInvalidValue;
        seg.input[n] = inputs[i];
        seg.packed[n] = packed[i];
        seg.scales[n] = scales[i];
        seg.start[n] = (uint32_t)rows;
        rows += Ns[i];
        ++n;
    }
    if (n == 0) return hipSuccess;
    // Short rows (one wave per row), one matrix, or a grid past 2^31 - 1:
    // one launch per matrix.
    if (W <= 128u || n == 1 || rows >= 0x7fffffffu) {
        for (uint32_t i = 0; i < count; ++i) {
            if (Ns[i] == 0) continue;
            const hipError_t e = launch_quantize_rows(inputs[i], Ns[i], K, nullptr, packed[i], scales[i], dev, stream,
                                                      nullptr);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    for (uint32_t i = n; i < kMaxQuantizeMatrices; ++i) {
        seg.input[i] = nullptr;
        seg.packed[i] = nullptr;
        seg.scales[i] = nullptr;
        seg.start[i] = 0xffffffffu;
    }
    const uint32_t blocks = (uint32_t)rows;
    const uint32_t wpt = (W + 255u) / 256u;
    if (wpt <= 1) return launch_qmulti<1>(seg, blocks, K, stream);
    if (wpt <= 2) return launch_qmulti<2>(seg, blocks, K, stream);
    if (wpt <= 4) return launch_qmulti<4>(seg, blocks, K, stream);
    if (wpt <= 6) return launch_qmulti<6>(seg, blocks, K, stream);
    if (wpt <= 8) return launch_qmulti<8>(seg, blocks, K, stream);
    return launch_qmulti<0>(seg, blocks, K, stream);
}

hipError_t launch_quantize_rows(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed,
                                float* scales, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    (void)dev;
    if (N == 0) return hipSuccess;
    if (codes && packed) return dispatch_q<true, true>(input, N, K, codes, packed, scales, stream, variant);
    if (codes) return dispatch_q<true, false>(input, N, K, codes, packed, scales, stream, variant);
    return dispatch_q<false, true>(input, N, K, codes, packed, scales, stream, variant);
}

// ---------------------------------------------------------------------------
// packQ8 / packInt8Rows: one thread per output word, grid-stride.

__global__ __launch_bounds__(256) void pack_q8_kernel(const int32_t* __restrict__ codes, uint32_t K, uint32_t W,
                                                      size_t total, uint32_t* __restrict__ packed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t row = i / W;
        const uint32_t w = (uint32_t)(i - row * W);
        const uint32_t k = 4u * w;
        const int32_t* c = codes + row * K + k;
        uint32_t word;
        if (k + 4u <= K) {
            const i32x4_a4 q = *reinterpret_cast<const i32x4_a4*>(c);
            word = ((uint32_t)q.x & 0xffu) | (((uint32_t)q.y & 0xffu) << 8) | (((uint32_t)q.z & 0xffu) << 16) |
                   (((uint32_t)q.w & 0xffu) << 24);
        } else {
            word = 0u;
            for (uint32_t e = 0; k + e < K; ++e) word |= ((uint32_t)c[e] & 0xffu) << (8u * e);
        }
        packed[i] = word;
    }
}

__global__ __launch_bounds__(256) void pack_int8_rows_kernel(const int8_t* __restrict__ codes, uint32_t K,
                                                             uint32_t W, size_t total, uint32_t* __restrict__ packed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t row = i / W;
        const uint32_t w = (uint32_t)(i - row * W);
        const uint32_t k = 4u * w;
        const uint8_t* c = reinterpret_cast<const uint8_t*>(codes) + row * K + k;
        uint32_t word = 0u;
        const uint32_t n = K - k < 4u ? K - k : 4u;
        for (uint32_t e = 0; e < n; ++e) word |= (uint32_t)c[e] << (8u * e);
        packed[i] = word;
    }
}

// packInt8Rows as a byte stream.  The packed matrix is the int8 code stream
// with g = 4W - K (0..3) zero bytes after every row, so the output is written
// flat: lane j of a workgroup writes output bytes [o0 + 16j, +16) of its
// chunks (16-byte stores, 1 KiB per wave instruction) from one dword-aligned
// 24-byte window of the input (a dwordx4 and a dword on either side of it;
// neighbouring lanes' windows overlap, so those hit the caches).  Output byte m
// of the chunk is
//   input[S + m]       while its column col0 + m < K          (X1)
//   0                  for columns K .. 4W-1 (the row's pad)
//   input[S + m - g]   from the next row's first column on    (X2)
// with S the input byte of the chunk's first output byte; X1 and X2 are
// funnel shifts (v_alignbyte) of the window by a per-lane byte count, merged
// with byte masks.  Needs 4W >= 16 (a chunk crosses at most one row end).
// The input resource spans the bytes from the workgroup's first row on, from
// the dword that holds the first one (the codes may start at any byte) and
// rounded up to whole dwords: a buffer load clamps per dword, and the few
// bytes outside the input that the first and last dwords hold only ever land
// in bytes the masks drop.
// Buffer offsets do not wrap: the dword below offset 0 (the first lane's
// window) reads as 0, and only masked-off bytes come from it.
template <int U, int LPOL = 0, int SPOL = 0>
__global__ __launch_bounds__(256) void pack_int8_rows_stream_kernel(const int8_t* __restrict__ codes, uint32_t K,
                                                                    uint32_t W4, uint64_t in_bytes, uint64_t out_bytes,
                                                                    uint8_t* __restrict__ packed) {
    constexpr uint32_t WGB = 256u * 16u * (uint32_t)U;
    const uint64_t o0 = (uint64_t)blockIdx.x * WGB;
    uint64_t r0;
    uint32_t c0;
    if (out_bytes <= 0xffffffffull) {
        const uint32_t o = (uint32_t)o0;
        const uint32_t r = o / W4;
        r0 = r;
        c0 = o - r * W4;
    } else {
        r0 = o0 / W4;
        c0 = (uint32_t)(o0 - r0 * W4);
    }
    // the resource starts at the dword holding the workgroup's first input
    // byte (codes may sit at any byte address); `delta` bytes of the dword
    // precede it
    const uint64_t ib0 = r0 * K;
    const uintptr_t first = reinterpret_cast<uintptr_t>(codes) + ib0;
    const uint32_t delta = (uint32_t)(first & 3u);
    const uint64_t in_left = (in_bytes - ib0 + delta + 3u) & ~3ull;
    const __amdgpu_buffer_rsrc_t irs = make_rsrc(reinterpret_cast<const void*>(first - delta),
                                                 in_left < 0xfffffff0ull ? (uint32_t)in_left : 0xfffffff0u);
    const uint64_t out_left = out_bytes - o0;
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(packed + o0, out_left < WGB ? (uint32_t)out_left : WGB);
    const uint32_t g = W4 - K;
    u32x4v mid[U];
    uint32_t below[U], above[U], col[U], sv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t rel = c0 + 16u * ((uint32_t)u * 256u + threadIdx.x);
        const uint32_t dr = rel / W4;
        col[u] = rel - dr * W4;
        sv[u] = dr * K + col[u] + delta;
        const uint32_t q4 = sv[u] & ~3u;
        mid[u] = __builtin_amdgcn_raw_buffer_load_b128(irs, (int)q4, 0, LPOL);
        above[u] = __builtin_amdgcn_raw_buffer_load_b32(irs, (int)(q4 + 16u), 0, LPOL);
        // the dword before: past the resource (0) for the first dword of the range
        below[u] = __builtin_amdgcn_raw_buffer_load_b32(irs, (int)(q4 - 4u), 0, LPOL);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t D[6] = {below[u], mid[u].x, mid[u].y, mid[u].z, mid[u].w, above[u]};
        const uint32_t sh = sv[u] & 3u;
        const bool same = sh >= g;
        uint32_t E[5];
#pragma unroll
        for (int t = 0; t < 5; ++t) E[t] = same ? D[t + 1] : D[t];
        const uint32_t sh2 = (sh - g) & 3u;
        const int e1 = min(16, max(0, (int)K - (int)col[u]));
        const int e2 = min(16, (int)(W4 - col[u]));
        u32x4v out;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t x1 = __builtin_amdgcn_alignbyte(D[i + 2], D[i + 1], sh);
            const uint32_t x2 = __builtin_amdgcn_alignbyte(E[i + 1], E[i], sh2);
            const int n1 = min(4, max(0, e1 - 4 * i)), n2 = min(4, max(0, e2 - 4 * i));
            const uint32_t m1 = n1 >= 4 ? ~0u : ((1u << (8 * n1)) - 1u);
            const uint32_t m2 = n2 >= 4 ? ~0u : ((1u << (8 * n2)) - 1u);
            out[i] = (x1 & m1) | (x2 & ~m2);
        }
        __builtin_amdgcn_raw_buffer_store_b128(out, ors, (int)(16u * ((uint32_t)u * 256u + threadIdx.x)), 0, SPOL);
    }
}

namespace {
uint32_t flat_grid(size_t total, const DeviceInfo& dev) {
    const size_t want = (total + 255) / 256;
    const size_t cap = (size_t)(dev.cu_count > 0 ? dev.cu_count : 256) * 16;
    return (uint32_t)(want < cap ? want : cap);
}
}  // namespace

hipError_t launch_pack_q8(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed, const DeviceInfo& dev,
                          hipStream_t stream) {
    const uint32_t W = (K + 3u) / 4u;
    const size_t total = (size_t)N * W;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(pack_q8_kernel, dim3(flat_grid(total, dev)), dim3(256), 0, stream, codes, K, W, total, packed);
    return hipGetLastError();
}

hipError_t launch_pack_int8_rows(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed,
                                 const DeviceInfo& dev, hipStream_t stream) {
    const uint32_t W = (K + 3u) / 4u;
    const size_t total = (size_t)N * W;
    if (total == 0) return hipSuccess;
    if (4u * W >= 16u) {
        // 16 KiB of output per workgroup, non-temporal stores (the output is
        // not read back soon).  Same-process timings at 4096 x 4099 / 11008 x
        // 4096: 7.41 / 16.3 us, against 7.64 / 17.2 with plain stores, 7.5-8.0
        // / 16.8-17.8 with 8 or 32 KiB per workgroup, 8.8-9.7 / 19-21 with
        // non-temporal loads (neighbouring lanes share lines), and 8.18 / 18.8
        // for the runtime's device-to-device copy of the output's size.
        constexpr int U = 4;
        const uint64_t out_bytes = (uint64_t)total * 4u;
        const uint64_t wgs = (out_bytes + 256u * 16u * U - 1u) / (256u * 16u * U);
        hipLaunchKernelGGL((pack_int8_rows_stream_kernel<U, 0, kCachePolicyNT>), dim3((uint32_t)wgs), dim3(256), 0, stream,
                           codes, K, 4u * W, (uint64_t)N * K, out_bytes, reinterpret_cast<uint8_t*>(packed));
        return hipGetLastError();
    }
    hipLaunchKernelGGL(pack_int8_rows_kernel, dim3(flat_grid(total, dev)), dim3(256), 0, stream, codes, K, W, total,
                       packed);
    return hipGetLastError();
}

}  // namespace wxo
