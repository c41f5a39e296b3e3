// dequant_q8.hip -- packed int8 weights back to f32 on gfx950.
//
// Reference semantics (all bit-exact: one f32 product of an int8 code and
// its row's scale, which is what the reference's f64 product stored to a
// Float32Array rounds to):
//   dequantize_packed   llm/weights-q8.ts:161-177 (dequantizePackedQ8):
//                       out[n, k] = q[n, k] * s[n], f32 [N, K]
//   dequant_transpose   ops/dequant_transpose/reference.ts:40-59
//                       (dequantTranspose): out[k, n] = q[n, k] * s[n],
//                       f32 [inFeatures, outFeatures]
//   gather_dequant_rows llm/weights-q8.ts:207-222 (gatherDequantRows): rows
//                       of an int8 [rows, D] table in request order, indices
//                       outside [0, rows) give a row of zeros
//
// All three are HBM-bound byte work: the codes are read once and the f32
// output (4x the bytes) is written once, in 16-byte stores wherever the row
// layout allows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"
#include "wave_ops.hpp"

namespace wxo {

namespace {

__device__ __forceinline__ float dq(uint32_t word, int lane, float s) {
    // sign-extended byte `lane` of the word times the scale, one f32 rounding
    return __fmul_rn((float)(int32_t)((int32_t)(word << (24 - 8 * lane)) >> 24), s);
}

// out [N, K], K % 4 == 0: one packed word per thread per pass, consecutive
// threads on consecutive words; the output is the words' flat image, 16 bytes
// per word, so a wave stores 1 KiB contiguous.  IDX: 32-bit below 2^32 words.
template <typename IDX>
__global__ __launch_bounds__(256) void dequantize_packed_kernel(const uint32_t* __restrict__ weight,
                                                                const float* __restrict__ scale,
                                                                float* __restrict__ out, uint32_t W, IDX total) {
    for (IDX i = (IDX)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (IDX)gridDim.x * blockDim.x) {
        const IDX row = i / W;
        const uint32_t word = weight[i];
        const float s = scale[row];
        f32x4_a4 f;
        f.x = dq(word, 0, s);
        f.y = dq(word, 1, s);
        f.z = dq(word, 2, s);
        f.w = dq(word, 3, s);
        *reinterpret_cast<f32x4_a4*>(out + 4u * (size_t)i) = f;
    }
}

// out [N, K], K % 4 != 0 (rows end mid-word, the pad codes not stored): thread
// t writes the flat outputs 4t .. 4t+3 with one 16-byte store, so a wave
// still stores 1 KiB contiguous.  Output j is column j % K of row j / K, the
// code at byte j % K of that row's packed words.  Four outputs inside one row
// (K >= 4) are bytes c % 4 .. +3 of two consecutive words: two loads and one
// v_alignbyte.  Outputs that cross a row end, and every output when K < 4,
// take their codes one at a time.  IDX is the index type: 32-bit when the
// output has under 2^32 elements (the 64-bit division per thread cost ~2.4 us
// at 4096 x 4099).  4096 x 4099: 24.1 us with one packed word per thread and
// four scalar stores, 14.9 us so.
template <typename IDX>
__global__ __launch_bounds__(256) void dequantize_packed_ragged_kernel(const uint32_t* __restrict__ weight,
                                                                       const float* __restrict__ scale,
                                                                       float* __restrict__ out, uint32_t K,
                                                                       uint32_t W, IDX total) {
    for (IDX j0 = (IDX)4u * ((IDX)blockIdx.x * blockDim.x + threadIdx.x); j0 < total;
         j0 += (IDX)4u * ((IDX)gridDim.x * blockDim.x)) {
        const IDX r = j0 / K;
        const uint32_t c = (uint32_t)(j0 - r * K);
        float v[4];
        if (c + 3u < K) {
            // inside row r: words c / 4 and c / 4 + 1 (both inside the row,
            // since c + 3 < K <= 4 W - 1)
            const uint32_t* src = weight + (size_t)r * W + c / 4u;
            const uint32_t bytes = __builtin_amdgcn_alignbyte(src[1], src[0], c & 3u);
            const float s = scale[r];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = dq(bytes, e, s);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t ce = c + (uint32_t)e;
                const IDX re = r + ce / K;
                const uint32_t cc = ce % K;
                v[e] = 0.0f;
                if (j0 + (IDX)e < total)
                    v[e] = dq(weight[(size_t)re * W + cc / 4u], (int)(cc & 3u), scale[re]);
            }
        }
        if (j0 + 3u < total) {
            *reinterpret_cast<f32x4_a4*>(out + j0) = f32x4_a4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (j0 + (IDX)e < total) out[j0 + (IDX)e] = v[e];
        }
    }
}

// out [K, N] (inFeatures x outFeatures).  A workgroup transposes one tile of
// 64 rows (n) x 64 codes (k) through LDS: each thread reads 16 codes (4
// packed words, one 16-byte load) of one row, writes them dequantized and
// transposed, and after the barrier stores 4 floats of a k-row, so both the
// word reads and the f32 writes are contiguous runs.  One 16-byte load per
// thread instead of four 4-byte ones: 5632 x 2048 10.7 -> 10.2 us, 32000 x
// 2048 70.9 -> 62.1 us (same bits).
constexpr uint32_t kTrTile = 64u;

__global__ __launch_bounds__(256) void dequant_transpose_kernel(const uint32_t* __restrict__ weight,
                                                                const float* __restrict__ scale,
                                                                float* __restrict__ out, uint32_t N, uint32_t K,
                                                                uint32_t W) {
    __shared__ float tile[kTrTile][kTrTile + 1];
    const uint32_t n0 = blockIdx.x * kTrTile, k0 = blockIdx.y * kTrTile;
    const uint32_t t = threadIdx.x;
    // load: row r = t / 4, words k0 / 4 + 4 q .. +3 (q = t % 4) in one
    // 16-byte load (dword-aligned); at a row's end, only its own words, one
    // at a time (the words past W belong to the next row, or lie past the
    // weight)
    {
        const uint32_t r = t >> 2, q = t & 3u;
        const uint32_t n = n0 + r;
        const uint32_t w0 = k0 / 4u + 4u * q;
        uint32_t wd[4] = {0u, 0u, 0u, 0u};
        float s = 0.0f;
        if (n < N) {
            const uint32_t* src = weight + (size_t)n * W + w0;
            if (w0 + 3u < W) {
                const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(src);
                wd[0] = v.x;
                wd[1] = v.y;
                wd[2] = v.z;
                wd[3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (w0 + (uint32_t)i < W) wd[i] = src[i];
            }
            s = scale[n];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int l = 0; l < 4; ++l) tile[16u * q + 4u * (uint32_t)i + (uint32_t)l][r] = dq(wd[i], l, s);
    }
    __syncthreads();
    // store: k-row kr = t / 16 + 16 j, columns 4 (t % 16) .. +3
    const uint32_t c4 = (t & 15u) * 4u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t kr = (t >> 4) + 16u * (uint32_t)j;
        const uint32_t k = k0 + kr;
        if (k >= K) continue;
        float* o = out + (size_t)k * N + n0 + c4;
        if ((N & 3u) == 0u && n0 + c4 + 3u < N) {
            f32x4_a4 f;
            f.x = tile[kr][c4];
            f.y = tile[kr][c4 + 1u];
            f.z = tile[kr][c4 + 2u];
            f.w = tile[kr][c4 + 3u];
            *reinterpret_cast<f32x4_a4*>(o) = f;
        } else {
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q)
                if (n0 + c4 + q < N) o[q] = tile[kr][c4 + q];
        }
    }
}

// out [count, D]: one workgroup per requested row, 16 codes per thread per
// pass.  An index outside [0, rows) writes zeros.
__global__ __launch_bounds__(256) void gather_dequant_rows_kernel(const int8_t* __restrict__ codes,
                                                                  const float* __restrict__ scale,
                                                                  const int64_t* __restrict__ indices,
                                                                  float* __restrict__ out, uint32_t rows,
                                                                  uint32_t D, uint32_t count) {
    for (uint32_t i = blockIdx.x; i < count; i += gridDim.x) {
        const int64_t idx = indices[i];
        const bool valid = idx >= 0 && idx < (int64_t)rows;
        const float s = valid ? scale[idx] : 0.0f;
        const int8_t* src = codes + (valid ? (size_t)idx * D : 0);
        float* o = out + (size_t)i * D;
        if (valid && (D & 15u) == 0u && ((uintptr_t)src & 15u) == 0u) {
            for (uint32_t c = threadIdx.x * 16u; c < D; c += blockDim.x * 16u) {
                const u32x4v v = *reinterpret_cast<const u32x4v*>(src + c);
                const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f32x4_a4 f;
                    f.x = dq(ws[q], 0, s);
                    f.y = dq(ws[q], 1, s);
                    f.z = dq(ws[q], 2, s);
                    f.w = dq(ws[q], 3, s);
                    *reinterpret_cast<f32x4_a4*>(o + c + 4u * (uint32_t)q) = f;
                }
            }
        } else {
            for (uint32_t c = threadIdx.x; c < D; c += blockDim.x)
                o[c] = valid ? __fmul_rn((float)src[c], s) : 0.0f;
        }
    }
}

uint32_t grid_cap(uint64_t items, uint32_t per_block, const DeviceInfo& dev) {
    const uint64_t want = (items + per_block - 1) / per_block;
    const uint64_t cap = (uint64_t)(dev.cu_count > 0 ? dev.cu_count : 256) * 16u;
    return (uint32_t)(want < cap ? (want > 0 ? want : 1) : cap);
}

}  // namespace

hipError_t launch_dequantize_packed(const uint32_t* weight, const float* scale, uint32_t N, uint32_t K,
                                    float* out, const DeviceInfo& dev, hipStream_t stream) {
    if (N == 0 || K == 0) return hipSuccess;
    const uint32_t W = (uint32_t)(((uint64_t)K + 3) / 4);
    if ((K & 3u) == 0u) {
        const uint64_t items = (uint64_t)N * W;
        const dim3 grid(grid_cap(items, 256, dev));
        if (items < 0xff000000ull)
            hipLaunchKernelGGL(dequantize_packed_kernel<uint32_t>, grid, dim3(256), 0, stream, weight, scale, out, W,
                               (uint32_t)items);
        else
            hipLaunchKernelGGL(dequantize_packed_kernel<uint64_t>, grid, dim3(256), 0, stream, weight, scale, out, W,
                               items);
    } else {
        const uint64_t total = (uint64_t)N * K;
        const dim3 grid(grid_cap((total + 3u) / 4u, 256, dev));
        // the grid-stride loop's last step stays below 2^32 + 2^22 too
        if (total < 0xff000000ull)
            hipLaunchKernelGGL(dequantize_packed_ragged_kernel<uint32_t>, grid, dim3(256), 0, stream, weight, scale,
                               out, K, W, (uint32_t)total);
        else
            hipLaunchKernelGGL(dequantize_packed_ragged_kernel<uint64_t>, grid, dim3(256), 0, stream, weight, scale,
                               out, K, W, total);
    }
    return hipGetLastError();
}

hipError_t launch_dequant_transpose(const uint32_t* weight, const float* scale, uint32_t out_features,
                                    uint32_t in_features, float* out, hipStream_t stream) {
    if (out_features == 0 || in_features == 0) return hipSuccess;
    const uint32_t W = (uint32_t)(((uint64_t)in_features + 3) / 4);
    const dim3 grid((out_features + kTrTile - 1) / kTrTile, (in_features + kTrTile - 1) / kTrTile);
    hipLaunchKernelGGL(dequant_transpose_kernel, grid, dim3(256), 0, stream, weight, scale, out, out_features,
                       in_features, W);
    return hipGetLastError();
}

hipError_t launch_gather_dequant_rows(const int8_t* codes, const float* scale, uint32_t rows, uint32_t D,
                                      const int64_t* indices, uint32_t count, float* out, const DeviceInfo& dev,
                                      hipStream_t stream) {
    if (count == 0 || D == 0) return hipSuccess;
    const uint32_t cap = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256) * 8u;
    hipLaunchKernelGGL(gather_dequant_rows_kernel, dim3(count < cap ? count : cap), dim3(256), 0, stream, codes,
                       scale, indices, out, rows, D, count);
    return hipGetLastError();
}

}  // namespace wxo
