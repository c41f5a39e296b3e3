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

// Four consecutive row values starting at column 4w (zero past K).
__device__ __forceinline__ f32x4_a4 load_row4(const float* __restrict__ xr, uint32_t K, uint32_t w) {
    const uint32_t k = 4u * w;
    if (k + 4u <= K) return load_f32x4(xr + k);
    f32x4_a4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (k + 0u < K) v.x = xr[k + 0];
    if (k + 1u < K) v.y = xr[k + 1];
    if (k + 2u < K) v.z = xr[k + 2];
    return v;
}

__device__ __forceinline__ uint32_t abs_bits_max(f32x4_a4 v, uint32_t m) {
    m = max(m, __float_as_uint(v.x) & 0x7fffffffu);
    m = max(m, __float_as_uint(v.y) & 0x7fffffffu);
    m = max(m, __float_as_uint(v.z) & 0x7fffffffu);
    m = max(m, __float_as_uint(v.w) & 0x7fffffffu);
    return m;
}

template <bool CODES, bool PACK>
__device__ __forceinline__ void emit_word(f32x4_a4 v, double inverse, uint32_t row, uint32_t w, uint32_t K,
                                          uint32_t W, int32_t* __restrict__ codes, uint32_t* __restrict__ packed) {
    const int32_t c0 = js_quantize_code(v.x, inverse);
    const int32_t c1 = js_quantize_code(v.y, inverse);
    const int32_t c2 = js_quantize_code(v.z, inverse);
    const int32_t c3 = js_quantize_code(v.w, inverse);
    const uint32_t k = 4u * w;
    if constexpr (PACK) {
        // Pad lanes past K were loaded as 0.0 and quantize to 0 (0 * inverse
        // is 0 or NaN), so the word's unused high bytes are zero as packQ8's.
        const uint32_t word = ((uint32_t)c0 & 0xffu) | (((uint32_t)c1 & 0xffu) << 8) |
                              (((uint32_t)c2 & 0xffu) << 16) | (((uint32_t)c3 & 0xffu) << 24);
        packed[(size_t)row * W + w] = word;
    }
    if constexpr (CODES) {
        int32_t* out = codes + (size_t)row * K + k;
        if (k + 4u <= K) {
            *reinterpret_cast<i32x4_a4*>(out) = i32x4_a4{c0, c1, c2, c3};
        } else {
            if (k + 0u < K) out[0] = c0;
            if (k + 1u < K) out[1] = c1;
            if (k + 2u < K) out[2] = c2;
        }
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

// WPL > 0: the row's words l, l+64, ... (WPL of them) stay in VGPRs.
// WPL == 0: any K; two passes over the row.
template <int WPL, bool CODES, bool PACK>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ input, uint32_t N,
                                                            uint32_t K, uint32_t W, int32_t* __restrict__ codes,
                                                            uint32_t* __restrict__ packed,
                                                            float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= N) return;  // wave-uniform; no barriers in this kernel
    const float* xr = input + (size_t)row * K;

    uint32_t m = 0;
    constexpr int S = WPL > 0 ? WPL : 1;
    f32x4_a4 v[S];
    if constexpr (WPL > 0) {
#pragma unroll
        for (int i = 0; i < WPL; ++i) {
            const uint32_t w = lane + 64u * (uint32_t)i;
            v[i] = (w < W) ? load_row4(xr, K, w) : f32x4_a4{0.0f, 0.0f, 0.0f, 0.0f};
            m = abs_bits_max(v[i], m);
        }
    } else {
        for (uint32_t w = lane; w < W; w += 64u) m = abs_bits_max(load_row4(xr, K, w), m);
    }
    const uint32_t amax = wave_max_u32(m);
    float scale;
    double inverse;
    row_scale(amax, &scale, &inverse);
    if (lane == 0) scales[row] = scale;

    if constexpr (WPL > 0) {
#pragma unroll
        for (int i = 0; i < WPL; ++i) {
            const uint32_t w = lane + 64u * (uint32_t)i;
            if (w < W) emit_word<CODES, PACK>(v[i], inverse, row, w, K, W, codes, packed);
        }
    } else {
        for (uint32_t w = lane; w < W; w += 64u)
            emit_word<CODES, PACK>(load_row4(xr, K, w), inverse, row, w, K, W, codes, packed);
    }
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

template <bool CODES, bool PACK>
hipError_t dispatch_q(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed, float* scales,
                      hipStream_t stream, const char** variant) {
    const uint32_t W = (K + 3u) / 4u;
    const uint32_t wpl = (W + 63u) / 64u;
    if (variant) *variant = "rows.reg";
    if (wpl <= 1) return launch_q<1, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpl <= 2) return launch_q<2, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpl <= 4) return launch_q<4, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpl <= 8) return launch_q<8, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpl <= 16) return launch_q<16, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (wpl <= 24) return launch_q<24, CODES, PACK>(input, N, K, codes, packed, scales, stream);
    if (variant) *variant = "rows.twopass";
    return launch_q<0, CODES, PACK>(input, N, K, codes, packed, scales, stream);
}

}  // namespace

hipError_t launch_quantize_rows(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed,
                                float* scales, const DeviceInfo& dev, hipStream_t stream, const char** variant) {
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
    hipLaunchKernelGGL(pack_int8_rows_kernel, dim3(flat_grid(total, dev)), dim3(256), 0, stream, codes, K, W, total,
                       packed);
    return hipGetLastError();
}

}  // namespace wxo
