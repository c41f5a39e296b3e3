// matvec_q8.hip -- W8A32 GEMV for gfx950: y[m, n] = (sum_k q[n, k] * x[m, k]) * s[n].
//
// Reference semantics: ops/matvec/reference.ts:113-131 (matvecQ8); the WGSL
// kernel it replaces is ops/matvec/wgsl/q8.wgsl (one 256-lane workgroup per
// row, scalar u32 loads, 8-level LDS tree).  This is a different design:
//
//  * A "chunk" is 256 consecutive packed words (1 KiB) of one row: exactly one
//    wave-wide global_load_dwordx4 (64 lanes x 16 B).  Lane l of a wave always
//    owns words [4l, 4l+4) of its chunks, i.e. the 16 codes k = 1024c + 16l ..
//    +15, so the 16 vector values it needs are fetched once per wave and live
//    in VGPRs for every row the wave visits: no LDS traffic for x in the loop.
//  * A workgroup of WAVES waves splits each row's chunks round-robin between
//    its waves (chunk c -> wave c % WAVES, slot c / WAVES), and walks blocks of
//    R rows with R independent dwordx4 loads in flight per wave per chunk.
//  * Unpack is one v_cvt_f32_i32_sdwa (sign-extended byte select) per code
//    feeding one v_fmac_f32: 2 VALU ops per code, no MFMA (bandwidth-bound).
//  * R row sums are reduced across the wave with DPP/permlane halving
//    (~R+6 ops, no LDS), partials of the WAVES waves meet in a 2-slot LDS
//    buffer (one barrier per block), and the scale is applied once per row.
//  * Pad lanes past K: the vector registers for k >= K are zero, so whatever
//    the pad bytes hold contributes q * 0 = 0; words past the row end and
//    vector entries past K are never loaded.
//
// The small-M batched VALU kernel reuses every loaded word for up to 8
// vectors (one unpack per code, one FMA per vector, the vector slices in
// VGPRs); large weights with 5 or more vectors go to the matrix cores.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"
#include "wave_ops.hpp"

namespace wxo {

constexpr uint32_t kChunkWords = 256;   // one wave-wide dwordx4 load
constexpr uint32_t kChunkCodes = 1024;

__device__ __forceinline__ float fma_word(uint32_t w, float x0, float x1, float x2, float x3, float acc) {
    acc = __builtin_fmaf((float)(int8_t)(w), x0, acc);
    acc = __builtin_fmaf((float)(int8_t)(w >> 8), x1, acc);
    acc = __builtin_fmaf((float)(int8_t)(w >> 16), x2, acc);
    acc = __builtin_fmaf((float)((int32_t)w >> 24), x3, acc);
    return acc;
}

// Lane `lane`'s 16 vector values of chunk c (k = 1024c + 16 lane .. +15),
// through a buffer resource over the K floats: entries past K clamp to 0
// without a branch.
__device__ __forceinline__ void load_x16_rsrc(__amdgpu_buffer_rsrc_t xrs, uint32_t c, int lane, float (&xr)[16]) {
    const int off = (int)((c * kChunkCodes + (uint32_t)lane * 16u) * 4u);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(xrs, off + 16 * q, 0, 0);
        xr[4 * q + 0] = __uint_as_float(v.x);
        xr[4 * q + 1] = __uint_as_float(v.y);
        xr[4 * q + 2] = __uint_as_float(v.z);
        xr[4 * q + 3] = __uint_as_float(v.w);
    }
}

// silu(g) * u as the reference composes it: silu in f64 on the f32 gate,
// x / (1 + e^-x), rounded to f32, then one f32 product.
__device__ __forceinline__ float ffn_epilogue(float g, float u) {
    const double gd = (double)g;
    const float gated = (float)(gd / (1.0 + exp(-gd)));
    return __fmul_rn(gated, u);
}

// residual + projected as the reference adds them: in f64, then one rounding
// to f32.
__device__ __forceinline__ float residual_epilogue(float r, float projected) {
    return (float)((double)r + (double)projected);
}

// ---------------------------------------------------------------------------
// M = 1.  One block of R rows per workgroup; WAVES waves split each row's
// chunks (chunk c -> wave c % WAVES, slot c / WAVES).
//
// Every load is a raw-buffer dwordx4 whose resource spans exactly the data it
// may touch (the block's rows; the K-float vector).  gfx950 clamps buffer
// loads per dword against the resource size (offset = VGPR + SGPR part), so
// rows past N, words past the matrix end and vector entries past K read as 0
// with no branch: the only control flow left is wave-uniform.  That matters
// for speed as much as for safety: a per-lane tail branch makes the compiler
// join two load sequences of different length, and at the join it waits for
// every outstanding load (vmcnt(0)), i.e. for the whole block, before the
// first FMA.  Words past W inside a row's last chunk belong to the next row
// (or clamp to 0); their vector entries are past K, hence 0, so they add
// q * 0 = 0.
//
// Issue order: the vector slice first (its first touch per XCD misses L2 and
// must not queue behind the weight flood), then all R weight loads of the
// block, row offset r * 4W in an SGPR, non-temporal (streamed once).
// CPW > 0: the vector slices of CPW chunk slots are loaded once into VGPRs.
// CPW == 0: any K; one slot at a time with its vector slice.
//
// EPI selects what happens to a row's dot product d once it is complete:
//   kEpiPlain     y = d * s
//   kEpiResidual  y = residual + (d * s): d * s rounded to f32, the sum taken
//                 in f64 and rounded once, as the reference's
//                 fround(residual + fround(d * s)) (ops/matvec/reference.ts:235-243)
//   kEpiFfn       two weights streamed side by side (gate rows, then up rows:
//                 2R dot products per block); y = silu(g) * u with g = dg * sg,
//                 u = du * su, silu evaluated in f64 and rounded to f32 as
//                 ops/activation/reference.ts:91-92 does, then one f32 product
//                 (ops/matvec/reference.ts:196-207)
//
// Arguments are scalars, not a struct: the build preloads the leading kernel
// arguments into SGPRs (-amdgpu-kernarg-preload-count), which LLVM does only
// for non-aggregate arguments.  Each wave then builds its buffer resources and
// issues its first loads without waiting on a kernarg fetch from memory
// (measured 0.33 us per call at N=11008, K=4096).  `aux` is the up
// projection's scale (kEpiFfn) or the residual (kEpiResidual); the plain form
// ignores weight2 and aux.
//
// The body is a device function over row block `block` so that the
// multi-projection kernel below runs the same code on its own row blocks.
//
// MASK (rows with a partial last chunk): lanes past the row's last word get
// an offset past the buffer resource, which returns zeros without a memory
// request, instead of reading the next row's words (then multiplied by zero x).
// Same results; cfg3 (4096 x 4099) 5.02 -> 4.90 us, 4096 x 4352 4.95 -> 4.84;
// left off for whole chunks, where the extra compare costs ~2 %.
//
// TAIL (rows of WAVES whole chunks plus 1 to 4 words, e.g. K = 4097 .. 4112):
// no wave streams the partial chunk.  A lane r loads row r's last 16 bytes
// (the tail words, then the next row's first words, whose codes meet x
// entries past K, i.e. 0) and the 16 x entries from 1024 WAVES.
//   kTailWave0 (1): wave 0 does it, after its own chunk.
//   kTailExtraWave (2): one more wave (wave WAVES) issues that single load.
// Either way the tail sums wait in LDS and join each row's total after the
// chunk waves' partials, so both forms give the same bits, and a projection
// run as row chunks gives the same rows as one call, whichever form each
// call picks (the wave reduction sums every row in the same lane order for
// any R, since each pairwise add is commutative).  A wave's loads return
//     in issue order, so a 17th load on a streaming wave holds back that
//     wave's whole block; a wave of its own costs a wave slot instead, which
//     is free while every CU holds one workgroup.
// Same-process (us), wave 0 -> extra wave: 4096 x 4099 (one workgroup per CU)
// 4.86 -> 4.67, 2048 x 4099 3.76 -> 3.51, 4096 x 4112 4.91 -> 4.77, 4096 x
// 8200 7.34 -> 7.30, 11008 x 4100 9.25 -> 9.23, but 11008 x 8200 (688
// workgroups of 9 waves) 16.1 -> 17.1; no tail at all (wrong results) 4.59 at
// 4096 x 4099.  Against a masked wave streaming the partial chunk, the wave-0
// tail had taken 4096 x 4099 from 4.92 us, 4096 x 8200 from 7.83 and 11008 x
// 8200 from 18.2.
constexpr int kTailWave0 = 1;
constexpr int kTailExtraWave = 2;
template <int WAVES, int CPW, int R, int EPI, bool MASK = false, int TAIL = 0>
__device__ __forceinline__ void m1_row_block(const uint32_t* __restrict__ weight, const float* __restrict__ scale,
                                             const float* __restrict__ x, float* y, uint32_t N, uint32_t K,
                                             uint32_t W, const uint32_t* __restrict__ weight2, const float* aux,
                                             uint32_t block) {
    constexpr int NWT = EPI == kEpiFfn ? 2 : 1;  // weights streamed
    constexpr int V = R * NWT;                     // dot products per block
    constexpr int SHIFT = 6 - ilog2(V);
    constexpr int XS = CPW > 0 ? CPW : 1;
    static_assert(TAIL == 0 || (CPW == 1 && !MASK && R <= 64), "the tail forms have one whole chunk per wave");
    const int lane = (int)(threadIdx.x & 63u);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t C = TAIL ? (uint32_t)WAVES : (W + kChunkWords - 1) / kChunkWords;
    const uint32_t row0 = block * (uint32_t)R;
    const uint32_t rows = min((uint32_t)R, N - row0);  // >= 1
    const uint32_t rowbytes = W * 4u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)row0 * W, rows * rowbytes);
    const __amdgpu_buffer_rsrc_t wrs2 =
        NWT == 2 ? make_rsrc(weight2 + (size_t)row0 * W, rows * rowbytes) : wrs;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, K * 4u);

    // The tail words' per-row sums (one per streamed weight).
    __shared__ float tpart[TAIL ? NWT : 1][TAIL ? R : 1];
    if constexpr (TAIL == kTailExtraWave) {
        if (wave == (uint32_t)WAVES) {  // wave-uniform: the tail wave
            const int toff = (uint32_t)lane < rows ? (int)((uint32_t)lane * rowbytes + (uint32_t)WAVES * 1024u) : 0x40000000;
            u32x4v tw[NWT];
            float tx[16];
            tw[0] = load_nt_b128(wrs, toff, 0);
            if constexpr (NWT == 2) tw[1] = load_nt_b128(wrs2, toff, 0);
            load_x16_rsrc(xrs, (uint32_t)WAVES, 0, tx);
#pragma unroll
            for (int n = 0; n < NWT; ++n) {
                float t = fma_word(tw[n].x, tx[0], tx[1], tx[2], tx[3], 0.0f);
                t = fma_word(tw[n].y, tx[4], tx[5], tx[6], tx[7], t);
                t = fma_word(tw[n].z, tx[8], tx[9], tx[10], tx[11], t);
                t = fma_word(tw[n].w, tx[12], tx[13], tx[14], tx[15], t);
                if (lane < R) tpart[n][lane] = t;
            }
            __syncthreads();  // the block's one barrier, met by every wave
            return;
        }
    }

    float xr[XS][16];
    if constexpr (CPW > 0) {
#pragma unroll
        for (int j = 0; j < CPW; ++j) load_x16_rsrc(xrs, wave + (uint32_t)j * WAVES, lane, xr[j]);
    }
    u32x4v tw[NWT];
    float tx[16];
    if constexpr (TAIL == kTailWave0) {
        if (wave == 0u) {  // wave-uniform
            const int toff = (uint32_t)lane < rows ? (int)((uint32_t)lane * rowbytes + (uint32_t)WAVES * 1024u) : 0x40000000;
            tw[0] = load_nt_b128(wrs, toff, 0);
            if constexpr (NWT == 2) tw[1] = load_nt_b128(wrs2, toff, 0);
            load_x16_rsrc(xrs, (uint32_t)WAVES, 0, tx);
        }
    }
    // Keep the issue order as written: the scheduler would otherwise trickle
    // the weight loads in between FMAs to save VGPRs, throttling the bytes in
    // flight when the whole block should be requested at once.
    __builtin_amdgcn_sched_barrier(0);

    float acc[V];
#pragma unroll
    for (int r = 0; r < V; ++r) acc[r] = 0.0f;

    const int slots = CPW > 0 ? CPW : (int)((C + WAVES - 1) / WAVES);
#pragma unroll
    for (int j = 0; j < slots; ++j) {
        const uint32_t c = wave + (uint32_t)j * WAVES;
        if (CPW != 1 && c >= C) break;  // wave-uniform; with CPW == 1 every wave owns a chunk
        const uint32_t wi = c * kChunkWords + (uint32_t)lane * 4u;  // the lane's first word
        const int voff = (!MASK || wi < W) ? (int)(wi * 4u) : 0x40000000;
        u32x4v v[V];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = load_nt_b128(wrs, voff, (int)(r * rowbytes));
        if constexpr (NWT == 2) {
#pragma unroll
            for (int r = 0; r < R; ++r) v[R + r] = load_nt_b128(wrs2, voff, (int)(r * rowbytes));
        }
        __builtin_amdgcn_sched_barrier(0);
        float xl[16];
        if constexpr (CPW > 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) xl[i] = xr[j][i];
        } else {
            load_x16_rsrc(xrs, c, lane, xl);
        }
#pragma unroll
        for (int r = 0; r < V; ++r) {
            float a = acc[r];
            a = fma_word(v[r].x, xl[0], xl[1], xl[2], xl[3], a);
            a = fma_word(v[r].y, xl[4], xl[5], xl[6], xl[7], a);
            a = fma_word(v[r].z, xl[8], xl[9], xl[10], xl[11], a);
            a = fma_word(v[r].w, xl[12], xl[13], xl[14], xl[15], a);
            acc[r] = a;
        }
    }
    if constexpr (TAIL == kTailWave0) {
        if (wave == 0u) {
#pragma unroll
            for (int n = 0; n < NWT; ++n) {
                float t = fma_word(tw[n].x, tx[0], tx[1], tx[2], tx[3], 0.0f);
                t = fma_word(tw[n].y, tx[4], tx[5], tx[6], tx[7], t);
                t = fma_word(tw[n].z, tx[8], tx[9], tx[10], tx[11], t);
                t = fma_word(tw[n].w, tx[12], tx[13], tx[14], tx[15], t);
                if (lane < R) tpart[n][lane] = t;
            }
        }
    }

    wave_reduce_rows<V>(acc, lane);
    const bool leader = (lane & ((1 << SHIFT) - 1)) == 0;
    const uint32_t rr = (uint32_t)lane >> SHIFT;
    if constexpr (WAVES == 1 && EPI == kEpiPlain && TAIL == 0) {
        if (leader && rr < rows) y[row0 + rr] = acc[0] * scale[row0 + rr];
    } else {
        __shared__ float part[WAVES][V];
        if (leader) part[wave][rr] = acc[0];
        __syncthreads();
        if (threadIdx.x < rows) {
            const uint32_t t = threadIdx.x, row = row0 + t;
            float d = part[0][t];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) d += part[w][t];
            if constexpr (TAIL) d += tpart[0][t];
            if constexpr (EPI == kEpiPlain) {
                y[row] = d * scale[row];
            } else if constexpr (EPI == kEpiResidual) {
                y[row] = residual_epilogue(aux[row], __fmul_rn(d, scale[row]));
            } else {
                float du = part[0][R + t];
#pragma unroll
                for (int w = 1; w < WAVES; ++w) du += part[w][R + t];
                if constexpr (TAIL) du += tpart[NWT - 1][t];
                y[row] = ffn_epilogue(__fmul_rn(d, scale[row]), __fmul_rn(du, aux[row]));
            }
        }
    }
}

template <int WAVES, int CPW, int R, int EPI, bool MASK = false, int TAIL = 0>
__global__ __launch_bounds__((WAVES + (TAIL == kTailExtraWave ? 1 : 0)) * 64) void matvec_q8_m1_kernel(
    const uint32_t* __restrict__ weight, const float* __restrict__ scale, const float* __restrict__ x,
    float* y, uint32_t N, uint32_t K, uint32_t W, const uint32_t* __restrict__ weight2, const float* aux) {
    m1_row_block<WAVES, CPW, R, EPI, MASK, TAIL>(weight, scale, x, y, N, K, W, weight2, aux, blockIdx.x);
}

// ---------------------------------------------------------------------------
// A few vectors (M <= MV) on the single-vector kernel's streaming loop: the
// same chunk loads (a whole 1 KiB of one row per instruction), one code
// conversion per code and MV FMAs, the MV vector slices of each owned chunk in
// VGPRs.  Costs 1 + MV VALU operations per code, so it pays only while that
// stays under the streaming time (small MV); R * MV dot products per block
// reduce across the wave as in the single-vector kernel.
template <int WAVES, int CPW, int R, int MV>
__global__ __launch_bounds__(WAVES * 64) void matvec_q8_mv_kernel(
    const uint32_t* __restrict__ weight, const float* __restrict__ scale, const float* __restrict__ x,
    float* __restrict__ y, uint32_t N, uint32_t K, uint32_t W, uint32_t M) {
    constexpr int V = R * MV;
    constexpr int XS = CPW > 0 ? CPW : 1;
    static_assert(V <= 64, "R * MV values per lane are reduced across the wave");
    constexpr int SHIFT = 6 - ilog2(V);
    const int lane = (int)(threadIdx.x & 63u);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t C = (W + kChunkWords - 1) / kChunkWords;
    const uint32_t row0 = blockIdx.x * (uint32_t)R;
    const uint32_t rows = min((uint32_t)R, N - row0);
    const uint32_t rowbytes = W * 4u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)row0 * W, rows * rowbytes);
    // grid y: groups of MV vectors
    x += (size_t)blockIdx.y * MV * K;
    y += (size_t)blockIdx.y * MV * N;
    M -= blockIdx.y * MV;

    // vectors past M read as 0 (an empty resource)
    __amdgpu_buffer_rsrc_t xrs[MV];
#pragma unroll
    for (int m = 0; m < MV; ++m) xrs[m] = make_rsrc(x + (size_t)m * K, (uint32_t)m < M ? K * 4u : 0u);
    // CPW > 0: the slices of CPW chunk slots loaded once; CPW == 0: any K,
    // one slot at a time with its slices
    float xr[XS][MV][16];
    if constexpr (CPW > 0) {
#pragma unroll
        for (int m = 0; m < MV; ++m)
#pragma unroll
            for (int j = 0; j < CPW; ++j) load_x16_rsrc(xrs[m], wave + (uint32_t)j * WAVES, lane, xr[j][m]);
    }
    __builtin_amdgcn_sched_barrier(0);

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
    const int slots = CPW > 0 ? CPW : (int)((C + WAVES - 1) / WAVES);
#pragma unroll
    for (int j = 0; j < slots; ++j) {
        const uint32_t c = wave + (uint32_t)j * WAVES;
        if (CPW != 1 && c >= C) break;  // wave-uniform
        const int voff = (int)(c * kChunkWords * 4u + (uint32_t)lane * 16u);
        u32x4v v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = load_nt_b128(wrs, voff, (int)(r * rowbytes));
        __builtin_amdgcn_sched_barrier(0);
        const int js = CPW > 0 ? j : 0;
        if constexpr (CPW == 0) {
#pragma unroll
            for (int m = 0; m < MV; ++m) load_x16_rsrc(xrs[m], c, lane, xr[0][m]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                const uint32_t w = v[r][wd];
                const float q0 = (float)(int8_t)(w), q1 = (float)(int8_t)(w >> 8);
                const float q2 = (float)(int8_t)(w >> 16), q3 = (float)((int32_t)w >> 24);
#pragma unroll
                for (int m = 0; m < MV; ++m) {
                    float a = acc[r * MV + m];
                    a = __builtin_fmaf(q0, xr[js][m][4 * wd], a);
                    a = __builtin_fmaf(q1, xr[js][m][4 * wd + 1], a);
                    a = __builtin_fmaf(q2, xr[js][m][4 * wd + 2], a);
                    a = __builtin_fmaf(q3, xr[js][m][4 * wd + 3], a);
                    acc[r * MV + m] = a;
                }
            }
        }
    }

    wave_reduce_rows<V>(acc, lane);
    const bool leader = (lane & ((1 << SHIFT) - 1)) == 0;
    const uint32_t idx = (uint32_t)lane >> SHIFT;  // r * MV + m
    if constexpr (WAVES == 1) {
        const uint32_t r = idx / MV, m = idx % MV;
        if (leader && r < rows && m < M) y[(size_t)m * N + row0 + r] = acc[0] * scale[row0 + r];
    } else {
        __shared__ float part[WAVES][V];
        if (leader) part[wave][idx] = acc[0];
        __syncthreads();
        if (threadIdx.x < (unsigned)V) {
            const uint32_t r = threadIdx.x / MV, m = threadIdx.x % MV;
            if (r < rows && m < M) {
                float d = part[0][threadIdx.x];
#pragma unroll
                for (int w = 1; w < WAVES; ++w) d += part[w][threadIdx.x];
                y[(size_t)m * N + row0 + r] = d * scale[row0 + r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Several projections of one vector in one launch (up to kMaxProjections):
// y_p = matvecQ8(weight_p, scale_p, x, N_p, K) for each p, all with the same
// x and K.  The grid is the projections' row blocks laid end to end;
// projection p owns blocks [start_p, start_{p+1}) (start_0 = 0, an unused
// projection starts at 0xffffffff), so a block picks its projection with
// wave-uniform compares and then runs the single-vector body unchanged.  One
// launch instead of several saves each later launch's start-up and tail
// (about 1.5 us each), which is most of a small projection's time.
template <int WAVES, int CPW, int R>
__global__ __launch_bounds__(WAVES * 64) void matvec_q8_multi_kernel(
    const float* __restrict__ x, uint32_t K, uint32_t W, uint32_t start1, uint32_t start2, uint32_t start3,
    const uint32_t* w0, const float* s0, float* y0, uint32_t n0, const uint32_t* w1, const float* s1, float* y1,
    uint32_t n1, const uint32_t* w2, const float* s2, float* y2, uint32_t n2, const uint32_t* w3,
    const float* s3, float* y3, uint32_t n3) {
    const uint32_t b = blockIdx.x;
    const uint32_t* w = w0;
    const float* s = s0;
    float* y = y0;
    uint32_t n = n0, start = 0;
    if (b >= start1) { w = w1; s = s1; y = y1; n = n1; start = start1; }
    if (b >= start2) { w = w2; s = s2; y = y2; n = n2; start = start2; }
    if (b >= start3) { w = w3; s = s3; y = y3; n = n3; start = start3; }
    m1_row_block<WAVES, CPW, R, kEpiPlain>(w, s, x, y, n, K, W, nullptr, nullptr, b - start);
}

// ---------------------------------------------------------------------------
// Small-M batched on the matrix cores (M >= 2): y[m, n] for up to 16 vectors
// per tile (grid y), v_mfma_f32_16x16x32_bf16.
//
// Exactness: a code q in [-128, 127] is exact in bf16, and x is split into
// three bf16 parts by truncation, x = h + m + l exactly (8 + 8 + 8 significand
// bits; a non-finite x keeps all of itself in h so Inf/NaN propagate as IEEE
// products do).  Every product q * part is exact in f32; the matrix core sums
// them in f32.  h-products accumulate in one register set and the (2^-8 and
// 2^-16 smaller) m, l products in another, so the chain of roundings sits on
// the h sum alone.  The h sum is folded into an outer sum every 1024 codes,
// so a chain is at most 32 accumulations plus the matrix core's own 32-term
// sum and a fold per 1024 codes: under 80 roundings for the largest K that
// fits, 5e-6 of sum_k |s q x|, inside the 1e-5 bar.
//
// VALU work is the code conversion only (one v_cvt_f32_i32_sdwa per code,
// one perm per two codes): 1.5 ops per code whatever M is, against 1 + M on
// the FMA path.  The x parts for the tile's vectors live in LDS
// (3 x MC x Kp bf16, in B-operand order) and are read per 32-code block as one
// ds_read_b128 per part per lane.
//
// Operand layout (probed on gfx950): A lane l holds A[l % 16][8 (l / 16) + e],
// B lane l holds B[8 (l / 16) + e][l % 16], C lane l holds C[4 (l / 16) + v][l % 16].
// Any permutation of k serves as long as A and B use the same one: a lane of
// group g = l / 16 loads codes 64u + 16g .. 64u + 16g + 15 of row l % 16 for
// u = 0..3 of each 256-code step, so one load instruction covers 64
// contiguous bytes of each of the tile's 16 rows (the four groups side by
// side); block (u, e) of the step uses codes 8e .. 8e+7 of load u, and B is
// read with the same k order.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kMfmaLdsBytes = 160u * 1024u;  // gfx950: 160 KB of LDS per CU, all usable by one workgroup
constexpr uint32_t kMfmaMinRows = 16384;  // batched rows from which the matrix-core path pays


__device__ __forceinline__ uint32_t bf16_hi_pair(float a, float b) {
    // high halves of two f32 (exact bf16 of small integers), a in the low half
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

__device__ __forceinline__ bf16x8 codes_to_bf16(uint32_t w0, uint32_t w1) {
    u32x4v r;
    r.x = bf16_hi_pair((float)(int8_t)(w0), (float)(int8_t)(w0 >> 8));
    r.y = bf16_hi_pair((float)(int8_t)(w0 >> 16), (float)((int32_t)w0 >> 24));
    r.z = bf16_hi_pair((float)(int8_t)(w1), (float)(int8_t)(w1 >> 8));
    r.w = bf16_hi_pair((float)(int8_t)(w1 >> 16), (float)((int32_t)w1 >> 24));
    return __builtin_bit_cast(bf16x8, r);
}

// Each workgroup takes a contiguous range of 16-row tiles (ranges differ by
// at most one tile) and its four waves split that range evenly; a wave walks
// its tiles T at a time over all of K in 256-code steps, the (tile group,
// step) pairs forming one software pipeline with D - 1 pairs' loads in
// flight ahead of the one computing.  No wave waits for another after the
// prologue.  A finished tile's 16 x 16 block of sums goes through a
// per-wave LDS slot so each lane stores 16 contiguous bytes of one vector's
// output.
constexpr uint32_t kTileSlotFloats = 16u * 17u;  // one 16 x 16 block, rows skewed by a float

// The bf16 parts of one vector entry as f32 bit patterns (low 16 bits zero):
// x = h + m + l exactly for finite x.  A NaN whose payload sits in the low 16
// bits would truncate to an infinity: it becomes the canonical quiet NaN
// instead; a non-finite x is all h.
__device__ __forceinline__ void split_x_parts(float xe, uint32_t& hb, uint32_t& mb, uint32_t& lb) {
    hb = __builtin_isnan(xe) ? 0x7fc00000u : __float_as_uint(xe) & 0xffff0000u;
    mb = 0u;
    lb = 0u;
    if (isfinite(xe)) {
        const float r1 = xe - __uint_as_float(hb);  // exact
        mb = __float_as_uint(r1) & 0xffff0000u;
        lb = __float_as_uint(r1 - __uint_as_float(mb)) & 0xffff0000u;  // exact, <= 8 significant bits
    }
}

// Splits the four vector entries k .. k+3 of column m (v; entries past K count
// as 0) into bf16 parts h, m, l and stores them in B-operand order:
// [part][32-code block][lane group][column] x 8 bf16.  Code k sits in block
// (k / 256) * 8 + ((k / 64) % 4) * 2 + (k / 8) % 2, lane group (k / 16) % 4,
// element k % 8: the order in which the matrix-core kernels read them.
__device__ __forceinline__ void store_x_parts(uint16_t* xparts, uint32_t MC, uint32_t Kp, uint32_t K, uint32_t m,
                                              uint32_t k, u32x4v v) {
    uint16_t hh[4], mm[4], ll[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        // entries past K belong to the next vector (or read 0): zero them
        const float xe = (k + (uint32_t)e < K) ? __uint_as_float(v[e]) : 0.0f;
        uint32_t hb, mb, lb;
        split_x_parts(xe, hb, mb, lb);
        hh[e] = (uint16_t)(hb >> 16);
        mm[e] = (uint16_t)(mb >> 16);
        ll[e] = (uint16_t)(lb >> 16);
    }
    const uint32_t blk = (k >> 8) * 8u + ((k >> 6) & 3u) * 2u + ((k >> 3) & 1u);
    const uint32_t at = ((blk * 4u + ((k >> 4) & 3u)) * MC + m) * 8u + (k & 7u);
    typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<u16x4*>(&xparts[at]) = u16x4{hh[0], hh[1], hh[2], hh[3]};
    *reinterpret_cast<u16x4*>(&xparts[Kp * MC + at]) = u16x4{mm[0], mm[1], mm[2], mm[3]};
    *reinterpret_cast<u16x4*>(&xparts[2u * Kp * MC + at]) = u16x4{ll[0], ll[1], ll[2], ll[3]};
}

template <int T, int D>
__global__ __launch_bounds__(256) void matvec_q8_mfma_kernel(
    const uint32_t* __restrict__ weight, const float* __restrict__ scale, const float* __restrict__ x,
    float* __restrict__ y, uint32_t N, uint32_t K, uint32_t W, uint32_t M, uint32_t Kp) {
    // x parts in B-operand order: [part][32-code block][lane group g][column]
    // x 8 bf16, so the 64 lanes of one B read cover one contiguous run.
    extern __shared__ __attribute__((aligned(16))) uint16_t xparts[];  // 3 x Kp x MC bf16, then the tile slots
    const uint32_t m0 = blockIdx.y * 16u;
    const uint32_t MC = min(16u, M - m0);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t jb = min(j, MC - 1u);  // B column (lanes past MC compute columns nobody stores)
    float* slot = reinterpret_cast<float*>(xparts + 3u * MC * Kp) + wv * kTileSlotFloats;
    const uint32_t rowbytes = W * 4u;
    const uint32_t ntiles = (N + 15u) / 16u;
    const uint32_t S = Kp / 256u;  // steps per tile group
    // this workgroup's tiles, then this wave's quarter of them
    const uint32_t b0 = (uint32_t)((uint64_t)blockIdx.x * ntiles / gridDim.x);
    const uint32_t b1 = (uint32_t)((uint64_t)(blockIdx.x + 1u) * ntiles / gridDim.x);
    const uint32_t t0 = b0 + (b1 - b0) * wv / 4u, t1 = b0 + (b1 - b0) * (wv + 1u) / 4u;
    const uint32_t ngroups = (t1 - t0 + T - 1) / T;
    const uint32_t total = ngroups * S;
    const int voff = (int)(j * rowbytes + g * 16u);
    const uint32_t r_lane = (lane & 3u) * 4u;  // epilogue: rows r_lane .. r_lane + 3 of column lane / 4

    // Loads of pair i: tile group i / S, step i % S.  Past the last pair the
    // resource is empty and the loads read 0 without touching memory, so the
    // issue is unconditional (a conditional issue would make the compiler
    // join load sequences of different length and wait for all of them).
    // Codes past K in a row belong to the next row (or read 0 past the
    // group) and meet x parts that are 0.  The group's scales ride with its
    // last step (an epilogue load would wait, in issue order, for the next
    // step's prefetched weights).
    auto issue = [&](uint32_t i, u32x4v (&d)[T][4], u32x4v (&sc)[T]) {
        const uint32_t step = i % S;
        const uint32_t tile0 = i < total ? t0 + (i / S) * T : 0u;
        const uint32_t rows = i < total ? min((uint32_t)T * 16u, min(t1 * 16u, N) - tile0 * 16u) : 0u;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)tile0 * 16u * W, rows * rowbytes);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + tile0 * 16u, step == S - 1u ? rows * 4u : 0u);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int so = (int)((uint32_t)t * 16u * rowbytes + step * 256u);
#pragma unroll
            for (int u = 0; u < 4; ++u) d[t][u] = load_nt_b128(wrs, voff + 64 * u, so);
            sc[t] = __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(((uint32_t)t * 16u + r_lane) * 4u), 0, 0);
        }
    };

    // The x parts are staged from up to 16 float4 loads per thread, all issued
    // before the first weights: a wait for x then never has to wait for the
    // weight loads queued behind it (vmcnt retires in issue order).
    constexpr int XU = 16;
    const uint32_t kq4 = Kp / 4u;  // float4 groups per staged vector row
    const uint32_t n4 = MC * kq4;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x + (size_t)m0 * K, MC * K * 4u);
    u32x4v xv[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const uint32_t idx = threadIdx.x + (uint32_t)u * 256u;
        const uint32_t m = idx / kq4, k = (idx - m * kq4) * 4u;
        // past the staged range: an offset beyond the resource reads 0
        const int off = idx < n4 ? (int)((m * K + k) * 4u) : (int)0x7ffffff0;
        xv[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
    }

    u32x4v buf[D][T][4], sbuf[D][T];
#pragma unroll
    for (int q = 0; q < D - 1; ++q) issue((uint32_t)q, buf[q], sbuf[q]);

    auto split_store = [&](uint32_t idx, u32x4v v) {
        const uint32_t m = idx / kq4, k = (idx - m * kq4) * 4u;
        store_x_parts(xparts, MC, Kp, K, m, k, v);
    };
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const uint32_t idx = threadIdx.x + (uint32_t)u * 256u;
        if (idx < n4) split_store(idx, xv[u]);
    }
    for (uint32_t idx = threadIdx.x + XU * 256u; idx < n4; idx += 256u) {  // only when MC * Kp > 16384
        const uint32_t m = idx / kq4, k = (idx - m * kq4) * 4u;
        split_store(idx, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((m * K + k) * 4u), 0, 0));
    }
    __syncthreads();

    f32x4 hi[T], lo[T], hs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        hi[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        lo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        hs[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const uint16_t* xb = &xparts[(g * MC + jb) * 8u];
    const uint32_t pstride = Kp * MC;
    const uint32_t bstride = 32u * MC;  // bf16 elements per block

    auto compute = [&](uint32_t i, const u32x4v (&d)[T][4], const u32x4v (&sc)[T]) {
        const uint32_t step = i % S;
        const uint16_t* xs = xb + step * 8u * bstride;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t kb = ((uint32_t)u * 2u + (uint32_t)e) * bstride;
                const bf16x8 bh = *reinterpret_cast<const bf16x8*>(xs + kb);
                const bf16x8 bm = *reinterpret_cast<const bf16x8*>(xs + pstride + kb);
                const bf16x8 bl = *reinterpret_cast<const bf16x8*>(xs + 2u * pstride + kb);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const bf16x8 av = codes_to_bf16(d[t][u][2 * e], d[t][u][2 * e + 1]);
                    hi[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bh, hi[t], 0, 0, 0);
                    lo[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bm, lo[t], 0, 0, 0);
                    lo[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bl, lo[t], 0, 0, 0);
                }
            }
        if (step % 4u == 3u) {  // wave-uniform: fold the h chain every 1024 codes
#pragma unroll
            for (int t = 0; t < T; ++t) {
                hs[t] += hi[t];
                hi[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (step == S - 1u) {  // wave-uniform: the tile group is complete
            const uint32_t tile0 = t0 + (i / S) * T;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                // C lane (j, g) holds rows 4g .. 4g+3 of column j: transpose
                // through the slot so a lane stores 4 rows of one column.
                const f32x4 v = (hs[t] + hi[t]) + lo[t];
#pragma unroll
                for (int q = 0; q < 4; ++q) slot[j * 17u + g * 4u + (uint32_t)q] = v[q];
                hi[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                lo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                hs[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                const uint32_t c = lane >> 2;
                const uint32_t row0 = (tile0 + (uint32_t)t) * 16u;
                if (c < MC && tile0 + (uint32_t)t < t1) {
                    float* yo = y + (size_t)(m0 + c) * N + row0 + r_lane;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (row0 + r_lane + (uint32_t)q < N)
                            yo[q] = slot[c * 17u + r_lane + (uint32_t)q] * __uint_as_float(sc[t][q]);
                }
            }
        }
    };

    for (uint32_t i = 0; i < total; i += (uint32_t)D) {
#pragma unroll
        for (int q = 0; q < D; ++q) {
            issue(i + (uint32_t)(q + D - 1), buf[(q + D - 1) % D], sbuf[(q + D - 1) % D]);
            if (q == 0 || i + (uint32_t)q < total) compute(i + (uint32_t)q, buf[q], sbuf[q]);
        }
    }
}

// The same kernel with the weight tiles fetched straight into LDS
// (buffer_load_dwordx4 ... lds): one instruction moves 1 KiB of whole 128-byte
// lines (4 rows x 256 bytes, or 8 rows x 128 bytes), where the register form
// can only fetch 64 bytes of each of 16 rows.  NWV waves (4 or 8) each own D
// stages of T tiles of 16 rows x SC codes (SC = 256 or 128: a K step).  Piece
// q (16 bytes) of row j of a tile is stored at position q ^ (j mod pieces per
// row), so the lanes that read one piece of 16 different rows spread over the
// bank groups.  128-code steps halve the stages, which lets 8 waves (two per
// SIMD) share one copy of the x parts of up to 8 vectors: one wave's LDS and
// load waits then overlap the other's conversion and matrix work.
// Waits are explicit, since the compiler does not track these loads: every
// LDS read of a stage completes (lgkmcnt(0)) before the stage is refilled,
// and a stage is read only after its loads have landed (vmcnt, counting the
// loads issued after it; vector stores count there too, which can only make
// the wait longer).
constexpr uint32_t kDmaTileBytes = 16u * 256u;  // one tile at 256-code steps
// Stages per wave.  Three or four (more weight bytes in flight per wave,
// fewer workgroups per CU) measured slower at every M from 2 to 14.
constexpr int kDmaStages = 2;

template <int T, int D, int NWV = 4, int SC = 256>
__global__ __launch_bounds__(64 * NWV) void matvec_q8_mfma_dma_kernel(
    const uint32_t* __restrict__ weight, const float* __restrict__ scale, const float* __restrict__ x,
    float* __restrict__ y, uint32_t N, uint32_t K, uint32_t W, uint32_t M, uint32_t Kp) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xparts[];  // x parts, weight stages, tile slots
    const uint32_t m0 = blockIdx.y * 16u;
    const uint32_t MC = min(16u, M - m0);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t jb = min(j, MC - 1u);
    uint8_t* stages = reinterpret_cast<uint8_t*>(xparts + 3u * MC * Kp);
    static_assert(NWV == 4 || NWV == 8, "4 or 8 waves");
    static_assert(SC == 256 || SC == 128, "256- or 128-code steps");
    constexpr uint32_t TBY = 16u * (uint32_t)SC;       // bytes of one tile per step
    constexpr uint32_t PPR = (uint32_t)SC / 16u;        // 16-byte pieces per row
    constexpr uint32_t RPI = 1024u / (uint32_t)SC;      // rows per load instruction
    constexpr int LPT = SC / 64;                        // load instructions per tile
    constexpr uint32_t NT = 64u * NWV;                  // threads
    uint8_t* wst = stages + wv * ((uint32_t)D * T * TBY);
    float* slot = reinterpret_cast<float*>(stages + (uint32_t)NWV * D * T * TBY) + wv * kTileSlotFloats;
    const uint32_t rowbytes = W * 4u;
    const uint32_t ntiles = (N + 15u) / 16u;
    const uint32_t S = Kp / (uint32_t)SC;
    const uint32_t b0 = (uint32_t)((uint64_t)blockIdx.x * ntiles / gridDim.x);
    const uint32_t b1 = (uint32_t)((uint64_t)(blockIdx.x + 1u) * ntiles / gridDim.x);
    const uint32_t t0 = b0 + (b1 - b0) * wv / (uint32_t)NWV, t1 = b0 + (b1 - b0) * (wv + 1u) / (uint32_t)NWV;
    const uint32_t ngroups = (t1 - t0 + T - 1) / T;
    const uint32_t total = ngroups * S;
    const uint32_t r_lane = (lane & 3u) * 4u;
    // load instruction ii of a tile: lane -> row RPI ii + lane / PPR, stored
    // at position lane % PPR, which holds piece (lane % PPR) ^ (row % PPR)
    // (a fixed bound: a template-dependent array captured by the lambdas below
    // makes the host-side instantiation of the kernel fail)
    int voff[4];
    static_assert(LPT <= 4, "at most 4 load instructions per tile");
#pragma unroll
    for (int ii = 0; ii < LPT; ++ii) {
        const uint32_t row = RPI * (uint32_t)ii + lane / PPR;
        voff[ii] = (int)(row * rowbytes + (((lane % PPR) ^ (row % PPR)) * 16u));
    }

    auto issue = [&](uint32_t i, u32x4v (&sc)[T]) {
        const uint32_t step = i % S;
        const uint32_t tile0 = i < total ? t0 + (i / S) * T : 0u;
        const uint32_t rows = i < total ? min((uint32_t)T * 16u, min(t1 * 16u, N) - tile0 * 16u) : 0u;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)tile0 * 16u * W, rows * rowbytes);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + tile0 * 16u, step == S - 1u ? rows * 4u : 0u);
        uint8_t* sb = wst + (i % (uint32_t)D) * ((uint32_t)T * TBY);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int so = (int)((uint32_t)t * 16u * rowbytes + step * (uint32_t)SC);
#pragma unroll
            for (int ii = 0; ii < LPT; ++ii)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    wrs, (__attribute__((address_space(3))) void*)(sb + (uint32_t)t * TBY + (uint32_t)ii * 1024u),
                    16, voff[ii], so, 0, kCachePolicyNT);
            sc[t] = __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(((uint32_t)t * 16u + r_lane) * 4u), 0, 0);
        }
    };

    constexpr int XU = 64 / NWV;  // x loads per thread in the first pass (16 KiB of x per pass)
    const uint32_t kq4 = Kp / 4u;
    const uint32_t n4 = MC * kq4;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x + (size_t)m0 * K, MC * K * 4u);
    u32x4v xv[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const uint32_t idx = threadIdx.x + (uint32_t)u * NT;
        const uint32_t m = idx / kq4, k = (idx - m * kq4) * 4u;
        const int off = idx < n4 ? (int)((m * K + k) * 4u) : (int)0x7ffffff0;
        xv[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
    }
    u32x4v sbuf[D][T];
#pragma unroll
    for (int q = 0; q < D - 1; ++q) issue((uint32_t)q, sbuf[q]);
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const uint32_t idx = threadIdx.x + (uint32_t)u * NT;
        if (idx < n4) {
            const uint32_t m = idx / kq4;
            store_x_parts(xparts, MC, Kp, K, m, (idx - m * kq4) * 4u, xv[u]);
        }
    }
    for (uint32_t idx = threadIdx.x + XU * NT; idx < n4; idx += NT) {
        const uint32_t m = idx / kq4, k = (idx - m * kq4) * 4u;
        store_x_parts(xparts, MC, Kp, K, m, k, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)((m * K + k) * 4u), 0, 0));
    }
    // The x parts are this workgroup's own LDS writes: wait for them and meet
    // at a plain barrier (a fence here would also wait for the weight stages
    // already in flight).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    f32x4 hi[T], lo[T], hs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        hi[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        lo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        hs[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const uint16_t* xb = &xparts[(g * MC + jb) * 8u];
    const uint32_t pstride = Kp * MC;
    const uint32_t bstride = 32u * MC;
    const uint32_t arow = j * (uint32_t)SC;  // row j of a tile in a stage

    auto compute = [&](uint32_t i, const u32x4v (&sc)[T]) {
        const uint32_t step = i % S;
        const uint16_t* xs = xb + step * ((uint32_t)SC / 32u) * bstride;
        const uint8_t* sb = wst + (i % (uint32_t)D) * ((uint32_t)T * TBY);
#pragma unroll
        for (int u = 0; u < SC / 64; ++u) {
            u32x4v a[T];
#pragma unroll
            for (int t = 0; t < T; ++t)
                a[t] = *reinterpret_cast<const u32x4v*>(sb + (uint32_t)t * TBY + arow +
                                                        (((4u * (uint32_t)u + g) ^ (j % PPR)) * 16u));
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t kb = ((uint32_t)u * 2u + (uint32_t)e) * bstride;
                const bf16x8 bh = *reinterpret_cast<const bf16x8*>(xs + kb);
                const bf16x8 bm = *reinterpret_cast<const bf16x8*>(xs + pstride + kb);
                const bf16x8 bl = *reinterpret_cast<const bf16x8*>(xs + 2u * pstride + kb);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const bf16x8 av = codes_to_bf16(a[t][2 * e], a[t][2 * e + 1]);
                    hi[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bh, hi[t], 0, 0, 0);
                    lo[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bm, lo[t], 0, 0, 0);
                    lo[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bl, lo[t], 0, 0, 0);
                }
            }
        }
        constexpr uint32_t kFoldSteps = 1024u / (uint32_t)SC;  // fold the h sums every 1024 codes
        if (step % kFoldSteps == kFoldSteps - 1u) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                hs[t] += hi[t];
                hi[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (step == S - 1u) {
            const uint32_t tile0 = t0 + (i / S) * T;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 v = (hs[t] + hi[t]) + lo[t];
#pragma unroll
                for (int q = 0; q < 4; ++q) slot[j * 17u + g * 4u + (uint32_t)q] = v[q];
                hi[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                lo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                hs[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                const uint32_t c = lane >> 2;
                const uint32_t row0 = (tile0 + (uint32_t)t) * 16u;
                if (c < MC && tile0 + (uint32_t)t < t1) {
                    float* yo = y + (size_t)(m0 + c) * N + row0 + r_lane;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (row0 + r_lane + (uint32_t)q < N)
                            yo[q] = slot[c * 17u + r_lane + (uint32_t)q] * __uint_as_float(sc[t][q]);
                }
            }
        }
    };

    // vmcnt encoding (gfx9): low 4 bits in [3:0], high 2 bits in [15:14];
    // expcnt 7 and lgkmcnt 15 leave those counters unconstrained.
    constexpr int kAfter = (D - 1) * (LPT + 1) * T;  // loads issued after a stage's own
    constexpr int kVmWait = 0x0f70 | (kAfter & 15) | ((kAfter >> 4) << 14);
    static_assert(kAfter < 64, "vmcnt holds at most 63");
    for (uint32_t i = 0; i < total; i += (uint32_t)D) {
#pragma unroll
        for (int q = 0; q < D; ++q) {
            // the stage refilled next was read by the previous pair: its LDS
            // reads must have completed
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_sched_barrier(0);
            issue(i + (uint32_t)(q + D - 1), sbuf[(q + D - 1) % D]);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(kVmWait);  // this pair's loads have landed
            __builtin_amdgcn_sched_barrier(0);
            if (q == 0 || i + (uint32_t)q < total) compute(i + (uint32_t)q, sbuf[q]);
        }
    }
}

// ---------------------------------------------------------------------------
// Batched, K up to 2048: the row's codes split across the workgroup's 8 waves
// (wave w owns codes 128 (w + 8 s) .. +127 of step s = 0 .. SW - 1), so each
// wave's share of the x parts fits in its VGPRs (12 bf16x8 registers per
// step and B operand set) and is never read again from LDS; only the weight
// tiles pass through LDS.  A workgroup walks a contiguous range of 16-row
// tiles; for each (tile, step) pair a wave fetches its 16 rows x 128 codes
// (2 KiB, two DMA instructions of 8 rows x 128 bytes, whole lines) into one of
// kKsStages private LDS stages, kKsStages - 1 pairs ahead of the one it
// converts and multiplies.  The 8 partial 16 x 16 blocks of a tile meet in
// LDS: every kKsGroup tiles the waves pass one barrier, and tile t's partials
// are summed (in wave order) by wave t mod 8, which scales and stores them
// during the next group's first pair.
// The partial sums of a tile are written after the next pair's matrix work is
// issued, so the write does not hold the next pair's loads back.
//
// STW adds a ninth wave that only sums, scales and stores: after each
// group's barrier it reads the group's partials and writes y, with the
// workgroup's scales read into LDS once at the start.  Its y stores then
// count on its own vmcnt, not on the streaming waves', whose stage waits
// would otherwise also wait for every store issued before them (gfx9 counts
// loads and stores together, in order).  Same sums in the same order.  Same
// process at LM head N = 151936, K = 1024, us, eight waves -> nine: 16
// vectors 36.2-37.7 -> 33.1-33.2, 8 vectors 30.8-33.0 -> 29.9-30.4, 5
// vectors 29.7-30.6 -> 28.7-28.9, 4 vectors 28.7-29.6 -> 27.6-28.2.
//
// PACK sets how the x parts fill a B operand's 16 columns:
//   1: 16 vectors, one part each: h, m, l in three operands (3 matrix ops per
//      32-code block)
//   2: up to 8 vectors: h | m side by side, then l | 0 (2 ops); the m column
//      sums move to the h lanes with a DPP row rotation
//   3: up to 5 vectors: h | m | l in one operand (1 op)
// A column's parts are summed as h + (m + l), the order PACK 1 uses too.
//
// Measured on MI355X (rotating weight copies), against the matrix-core
// kernels above: LM head N = 151936, K = 1024: 16 vectors 33-34 us (45-47),
// 8 vectors 30-31 (41), 5 vectors 29-30 (41); N = 32768, K = 2048, 16
// vectors 17.7-18 us (58).  Of the 16-vector time at K = 1024: a
// workgroup's weight stream alone (loads, no matrix work) takes 25.5 us; the
// shader clock runs at 1.8-2.1 GHz while the matrix cores work against
// 2.3-2.4 GHz for the loads alone, and leaving out the codes' conversion and
// a third of the matrix ops (timing bounds) saves only 2-3 us.  Deeper
// stages (5-7) or four tiles per barrier measured no faster.
constexpr int kKsGroup = 2;   // tiles per barrier
constexpr int kKsStages = 4;  // LDS stages per wave (3 pairs in flight)
constexpr uint32_t kKsWaves = 8;

template <int CTRL>
__device__ __forceinline__ f32x4 dpp_f32x4(f32x4 v) {
    f32x4 r;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        r[q] = __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v[q]), CTRL, 0xf, 0xf, false));
    return r;
}

constexpr int ks_gcd(int a, int b) { return b == 0 ? a : ks_gcd(b, a % b); }

template <int PACK>
constexpr uint32_t ks_vectors() { return PACK == 1 ? 16u : PACK == 2 ? 8u : 5u; }

template <int SW, int PACK, bool STW = false>
__global__ __launch_bounds__(STW ? 576 : 512) void matvec_q8_ksplit_kernel(
    const uint32_t* __restrict__ weight, const float* __restrict__ scale, const float* __restrict__ x,
    float* __restrict__ y, uint32_t N, uint32_t K, uint32_t W, uint32_t M) {
    extern __shared__ __attribute__((aligned(16))) uint8_t ks_lds[];
    constexpr int G = kKsGroup, D = kKsStages;
    constexpr uint32_t SC = 128, TBY = 16u * SC;
    constexpr int GP = G * SW;                          // pairs per group
    constexpr int PER = GP / ks_gcd(GP, D) * D;         // pairs per unrolled loop body
    constexpr int NB = PACK == 1 ? 3 : PACK == 2 ? 2 : 1;
    constexpr uint32_t VPB = ks_vectors<PACK>();
    static_assert(8 % G == 0, "the reducing wave is the tile index mod 8");
    const uint32_t m0 = blockIdx.y * VPB;
    const uint32_t MC = min(VPB, M - m0);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    // B column j carries part `sel` of vector `vj`
    const uint32_t sel = PACK == 1 ? 0u : PACK == 2 ? j / 8u : j / 5u;
    const uint32_t vj = PACK == 1 ? j : PACK == 2 ? j % 8u : j % 5u;
    const bool col_ok = vj < MC && sel < (uint32_t)PACK;
    uint8_t* wst = ks_lds + wv * ((uint32_t)D * TBY);
    float* red = reinterpret_cast<float*>(ks_lds + kKsWaves * (uint32_t)D * TBY);  // [2][G][8 waves][64][4]
    const uint32_t rowbytes = W * 4u;
    const uint32_t ntiles = (N + 15u) / 16u;
    const uint32_t b0 = (uint32_t)((uint64_t)blockIdx.x * ntiles / gridDim.x);
    const uint32_t b1 = (uint32_t)((uint64_t)(blockIdx.x + 1u) * ntiles / gridDim.x);
    const uint32_t ngroups = (b1 - b0 + G - 1) / G;
    // The pair count rounded up to whole loop bodies; the loop stops at the
    // first group past the range.  Tiles past the range within the last group
    // are empty (zero-length resources) but run, so every wave passes the
    // same barriers.
    const uint32_t total = ((ngroups * (uint32_t)GP + PER - 1) / PER) * PER;

    if constexpr (STW) {
        if (wv == kKsWaves) {
            // The store wave: after each group's barrier it sums the group's
            // tiles (their 8 partials in wave order), scales and stores them,
            // while the streaming waves go on.  Its y stores count on its own
            // vmcnt, so the streaming waves' stage waits never include a
            // store.  The workgroup's scales come into LDS once, before the
            // first barrier, so no global load sits between two barriers.
            // It passes the same barriers as the streaming waves.
            float* scl = reinterpret_cast<float*>(ks_lds + kKsWaves * (uint32_t)D * TBY + 2u * (uint32_t)G * kKsWaves * 1024u);
            const uint32_t r0 = b0 * 16u, nr = min(b1 * 16u, N) - r0;
            const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + r0, nr * 4u);
            for (uint32_t o = 0; o < nr; o += 256u) {
                const u32x4v v4 = __builtin_amdgcn_raw_buffer_load_b128(srs, (int)((o + 4u * lane) * 4u), 0, 0);
                if (o + 4u * lane < nr) *reinterpret_cast<u32x4v*>(scl + o + 4u * lane) = v4;
            }
            for (uint32_t grp = 0; grp < ngroups; ++grp) {
                __builtin_amdgcn_s_waitcnt(0xc07f);  // scales in LDS (first pass), partials read (later ones)
                __builtin_amdgcn_s_barrier();
#pragma unroll
                for (int t = 0; t < G; ++t) {
                    const uint32_t tile = b0 + grp * (uint32_t)G + (uint32_t)t;
                    const float* rp = red + ((((grp & 1u) * G + (uint32_t)t) * kKsWaves) * 64u + lane) * 4u;
                    f32x4 part[kKsWaves];
#pragma unroll
                    for (int w = 0; w < (int)kKsWaves; ++w)
                        part[w] = *reinterpret_cast<const f32x4*>(rp + (uint32_t)w * 256u);
                    const uint32_t rl = (tile - b0) * 16u + 4u * g;  // row within the workgroup's range
                    const f32x4 sc = *reinterpret_cast<const f32x4*>(scl + (tile < b1 ? rl : 0u));
                    f32x4 sum = part[0];
#pragma unroll
                    for (int w = 1; w < (int)kKsWaves; ++w) sum += part[w];
                    if (tile < b1 && col_ok && sel == 0u) {
                        const uint32_t row = tile * 16u + 4u * g;
                        float* yo = y + (size_t)(m0 + vj) * N + row;
                        if (row + 3u < N) {
                            *reinterpret_cast<f32x4_a4*>(yo) = sum * sc;
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                if (row + (uint32_t)q < N) yo[q] = sum[q] * sc[q];
                        }
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(0);
            return;
        }
    }

    // DMA instruction ii of a pair: lane -> row 8 ii + lane / 8, stored at
    // position lane % 8, which holds piece (lane % 8) ^ (row % 8)
    int voff[2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const uint32_t row = 8u * (uint32_t)ii + lane / 8u;
        voff[ii] = (int)(row * rowbytes + (((lane % 8u) ^ (row % 8u)) * 16u));
    }

    // Memory operations per pair: two DMA instructions, plus the scale load
    // on a tile's last step (`i % SW` folds to a constant in the unrolled loop,
    // so the count is fixed per position and the waits below are exact).
    auto issue = [&](uint32_t i, u32x4v& sc) {
        const uint32_t ti = i / SW, s = i % SW;
        const uint32_t c0 = 128u * (wv + kKsWaves * s);
        const bool ok = b0 + ti < b1 && c0 < K;
        const uint32_t tile = ok ? b0 + ti : 0u;
        const uint32_t rows = ok ? min(16u, N - tile * 16u) : 0u;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)tile * 16u * W, rows * rowbytes);
        uint8_t* sb = wst + (i % (uint32_t)D) * TBY;
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wrs, (__attribute__((address_space(3))) void*)(sb + (uint32_t)ii * 1024u), 16, voff[ii], (int)c0, 0,
                kCachePolicyNT);
        if (!STW && s == SW - 1u) {
            const bool mine = b0 + ti < b1 && (ti & 7u) == wv;  // this wave sums and stores the tile
            const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + (size_t)(mine ? b0 + ti : 0u) * 16u,
                                                         mine ? min(16u, N - (b0 + ti) * 16u) * 4u : 0u);
            sc = __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(g * 16u), 0, 0);
        }
    };

    // This wave's x parts: lane (j, g), step s, block (u, e) holds codes
    // c0 + 64u + 16g + 8e + 0..7 of vector m0 + vj: the k order in which the
    // lane reads its A operand (piece 4u + g of row j).  Entries past K are 0
    // (they would belong to the next vector).
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x + (size_t)m0 * K, MC * K * 4u);
    u32x4v xl[SW][2][4];
#pragma unroll
    for (int s = 0; s < SW; ++s)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t c = 128u * (wv + kKsWaves * (uint32_t)s) + 64u * (uint32_t)u + 16u * g + 4u * (uint32_t)q;
                const int off = (col_ok && c < K) ? (int)((vj * K + c) * 4u) : (int)0x7ffffff0;
                xl[s][u][q] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
            }
    u32x4v sbuf[D];
#pragma unroll
    for (int q = 0; q < D - 1; ++q) issue((uint32_t)q, sbuf[q]);

    bf16x8 bx[SW][2][2][NB];
#pragma unroll
    for (int s = 0; s < SW; ++s)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                u32x4v pv[3];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    uint32_t hw[2], mw[2], lw[2];
#pragma unroll
                    for (int z = 0; z < 2; ++z) {
                        const int idx = 8 * e + 2 * p + z;
                        const uint32_t c = 128u * (wv + kKsWaves * (uint32_t)s) + 64u * (uint32_t)u + 16u * g + (uint32_t)idx;
                        const float xe = c < K ? __uint_as_float(xl[s][u][idx / 4][idx % 4]) : 0.0f;
                        split_x_parts(xe, hw[z], mw[z], lw[z]);
                    }
                    pv[0][p] = (hw[0] >> 16) | hw[1];
                    pv[1][p] = (mw[0] >> 16) | mw[1];
                    pv[2][p] = (lw[0] >> 16) | lw[1];
                }
                const u32x4v zero = {0u, 0u, 0u, 0u};
                if constexpr (PACK == 1) {
#pragma unroll
                    for (int b = 0; b < 3; ++b) bx[s][u][e][b] = __builtin_bit_cast(bf16x8, pv[b]);
                } else if constexpr (PACK == 2) {
                    bx[s][u][e][0] = __builtin_bit_cast(bf16x8, sel == 0u ? pv[0] : pv[1]);
                    bx[s][u][e][1] = __builtin_bit_cast(bf16x8, sel == 0u ? pv[2] : zero);
                } else {
                    bx[s][u][e][0] = __builtin_bit_cast(bf16x8, sel == 0u ? pv[0] : sel == 1u ? pv[1] : pv[2]);
                }
            }

    f32x4 acc[NB], pacc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = pacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4v rsc = {0u, 0u, 0u, 0u};
    const uint32_t arow = j * SC;

    auto compute = [&](uint32_t i, int s) {
        const uint8_t* sb = wst + (i % (uint32_t)D) * TBY;
        u32x4v a[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
            a[u] = *reinterpret_cast<const u32x4v*>(sb + arow + (((4u * (uint32_t)u + g) ^ (j & 7u)) * 16u));
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const bf16x8 av = codes_to_bf16(a[u][2 * e], a[u][2 * e + 1]);
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bx[s][u][e][b], acc[b], 0, 0, 0);
            }
    };
    // A lane's 4 sums (rows 4g .. 4g+3 of column j): valid where sel == 0.
    // DPP row_ror:n hands lane i the value of lane (i - n) mod 16 of its row.
    auto combine = [&](const f32x4 (&c)[NB]) -> f32x4 {
        if constexpr (PACK == 1) return c[0] + (c[1] + c[2]);
        else if constexpr (PACK == 2) return c[0] + (dpp_f32x4<0x128>(c[0]) + c[1]);
        else return c[0] + (dpp_f32x4<0x12B>(c[0]) + dpp_f32x4<0x126>(c[0]));
    };
    auto red_write = [&](uint32_t ti, const f32x4 (&c)[NB]) {
        const uint32_t grp = ti / G, t = ti % G;
        *reinterpret_cast<f32x4*>(red + ((((grp & 1u) * G + t) * kKsWaves + wv) * 64u + lane) * 4u) = combine(c);
    };
    auto finish = [&](uint32_t i, int s, bool defer, const u32x4v& sc) {
        if (s != SW - 1) return;
        const uint32_t ti = i / SW;
        if (defer) {
#pragma unroll
            for (int b = 0; b < NB; ++b) pacc[b] = acc[b];
        } else {
            red_write(ti, acc);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        if ((ti & 7u) == wv) rsc = sc;
    };
    auto reduce = [&](uint32_t grp) {
        const uint32_t t = (wv - grp * G) & 7u;
        if (t >= (uint32_t)G) return;
        const uint32_t ti = grp * G + t;
        const float* rp = red + ((((grp & 1u) * G + t) * kKsWaves) * 64u + lane) * 4u;
        // all 8 partials in flight at once (left to itself the compiler keeps
        // two, and the other waves then wait for this one at the next barrier)
        f32x4 part[kKsWaves];
#pragma unroll
        for (int w = 0; w < (int)kKsWaves; ++w) part[w] = *reinterpret_cast<const f32x4*>(rp + (uint32_t)w * 256u);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 sum = part[0];
#pragma unroll
        for (int w = 1; w < (int)kKsWaves; ++w) sum += part[w];
        const uint32_t tile = b0 + ti;
        if (tile < b1 && col_ok && sel == 0u) {
            const uint32_t row = tile * 16u + 4u * g;
            float* yo = y + (size_t)(m0 + vj) * N + row;
            if (row + 3u < N) {
                f32x4 o;
#pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = sum[q] * __uint_as_float(rsc[q]);
                *reinterpret_cast<f32x4_a4*>(yo) = o;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (row + (uint32_t)q < N) yo[q] = sum[q] * __uint_as_float(rsc[q]);
            }
        }
    };

    // vmcnt for pair i: the memory operations of the D - 1 pairs issued after
    // it (y stores issued in between only make the wait longer)
    auto after = [](int par) {
        int n = 0;
        for (int r = 1; r < D; ++r) n += 2 + (!STW && ((par + r) % SW) == SW - 1 ? 1 : 0);
        return n;
    };
    constexpr int kA0 = after(0), kA1 = SW > 1 ? after(1) : after(0);
    static_assert(kA0 < 64 && kA1 < 64, "vmcnt holds at most 63");
    constexpr int kVmWait0 = 0x0f70 | (kA0 & 15) | ((kA0 >> 4) << 14);
    constexpr int kVmWait1 = 0x0f70 | (kA1 & 15) | ((kA1 >> 4) << 14);
    uint32_t pending = ~0u;  // a group whose partials are written but not yet summed (wave-uniform)
    for (uint32_t i = 0; i < total; i += (uint32_t)PER) {
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            // groups past the range (the loop body is PER pairs long): stop at
            // the first, the same for every wave of the workgroup
            if (q % GP == 0 && i + (uint32_t)q >= ngroups * (uint32_t)GP) break;
            // the stage refilled next was read by the previous pair; if that
            // iteration ended with a deferred partial-sum write (its last LDS
            // operation), the write may still be in flight: LDS operations
            // complete in order, so lgkmcnt(1) already covers the reads
            __builtin_amdgcn_sched_barrier(0);
            if (q > 0 && ((q - 1) % GP) != 0 && ((q - 2 + GP) % SW) == SW - 1 && (q % GP) != 0)
                __builtin_amdgcn_s_waitcnt((0xc07f & ~0x0f00) | 0x0100);  // lgkmcnt(1)
            else
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_sched_barrier(0);
            issue(i + (uint32_t)(q + D - 1), sbuf[(q + D - 1) % D]);
            __builtin_amdgcn_sched_barrier(0);
            if (q % SW == 0) __builtin_amdgcn_s_waitcnt(kVmWait0);
            else __builtin_amdgcn_s_waitcnt(kVmWait1);
            __builtin_amdgcn_sched_barrier(0);
            compute(i + (uint32_t)q, q % SW);
            // the deferred write stays behind this pair's A reads (the wait above relies on it)
            __builtin_amdgcn_sched_barrier(0);
            if ((q % GP) != 0 && ((q - 1) % SW) == SW - 1) red_write((i + (uint32_t)q - 1u) / SW, pacc);
            finish(i + (uint32_t)q, q % SW, ((q + 1) % GP) != 0, sbuf[q % D]);
            if (!STW && q % GP == 0 && pending != ~0u) {
                // the previous group's sums, behind this pair's matrix work
                // (its partials sit in the half of the double buffer that the
                // next barrier protects)
                reduce(pending);
                pending = ~0u;
            }
            if ((q + 1) % GP == 0) {
                // the group's partials are in LDS: meet; its tiles' waves sum
                // them during the next group's first pair
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                pending = (i + (uint32_t)q) / GP;
            }
        }
    }
    if (!STW && pending != ~0u) reduce(pending);
    __builtin_amdgcn_s_waitcnt(0);  // no fetch into LDS outlives the workgroup
}

constexpr uint32_t kKsLdsBytes = kKsWaves * kKsStages * 16u * 128u + 2u * kKsGroup * kKsWaves * 1024u;

// ---------------------------------------------------------------------------
// Host-side dispatch.

namespace {

template <int WAVES, int CPW, int R, int EPI, bool MASK = false, int TAIL = 0>
hipError_t launch_m1_form(const MatvecArgs& a, hipStream_t stream, Variant* variant) {
    const uint32_t nblocks = (a.N + R - 1) / R;
    const float* aux = EPI == kEpiFfn ? a.scale2 : EPI == kEpiResidual ? a.residual : nullptr;
    constexpr int NW = WAVES + (TAIL == kTailExtraWave ? 1 : 0);
    hipLaunchKernelGGL((matvec_q8_m1_kernel<WAVES, CPW, R, EPI, MASK, TAIL>), dim3(nblocks), dim3(NW * 64), 0, stream,
                       a.weight, a.scale, a.vector, a.output, a.N, a.K, a.W, a.weight2, aux);
    set_variant(variant, EPI == kEpiFfn ? "matvec_q8_m1.ffn" : EPI == kEpiResidual ? "matvec_q8_m1.residual" : "matvec_q8_m1",
                CPW > 0 ? (TAIL == kTailExtraWave ? "xreg.tailwave" : TAIL ? "xreg.tail" : MASK ? "xreg.masked" : "xreg")
                        : "xstream",
                NW, R, CPW, 1, nblocks);
    return hipGetLastError();
}

// TAIL (bool): rows of whole chunks plus 1 to 4 words.  The extra tail wave
// when the grid is at most one workgroup per CU (it then takes no CU's wave
// slots from another workgroup), else the tail words on wave 0.
template <int WAVES, int CPW, int R, int EPI, bool MASK = false, bool TAIL = false>
hipError_t launch_m1(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    if constexpr (TAIL) {
        const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
        if ((a.N + R - 1) / R <= cus) return launch_m1_form<WAVES, CPW, R, EPI, MASK, kTailExtraWave>(a, stream, variant);
        return launch_m1_form<WAVES, CPW, R, EPI, MASK, kTailWave0>(a, stream, variant);
    } else {
        return launch_m1_form<WAVES, CPW, R, EPI, MASK, 0>(a, stream, variant);
    }
}

// Rows per workgroup: for whole chunks, an R whose grid is a whole multiple
// of the CU count when there is one (below); otherwise the largest R whose
// grid still gives every CU at least two workgroups (fewer, fatter blocks
// amortise the per-workgroup vector fetch; too few leave CUs idle), one
// workgroup for the tail form (cfg3,
// 4096 x 4099: 16 rows 4.55 us against 8 rows 4.92; 2048 x 4099: 8 rows 3.46
// against 4 rows 3.60; same-process).  The fused FFN streams two weights and
// takes at most a quarter of the rows (4 rows of each weight per block:
// 3-4 % faster than 8 at 5632 x 2048 and 11008 x 4096).
template <int WAVES, int CPW, int RMAX, int EPI, bool TAIL = false>
hipError_t dispatch_m1_rows(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    constexpr int RM = EPI == kEpiFfn ? RMAX / 4 : RMAX;
    const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    if constexpr (!TAIL && CPW == 1 && (WAVES == 2 || WAVES == 4)) {
        // First choice for rows of 2 or 4 chunks: the largest R whose grid is
        // a whole multiple of the CU count, so that every CU streams the same
        // bytes; at most 8 rows per block with 2 waves, whose 16-row chain is
        // too long.  Same-process, launches queued (us): 2048 x 2048 R=8 (256
        // blocks) 2.83-2.86 against R=4 2.99-3.01; 1024 x 2048 R=4 2.52
        // against R=2 2.63; 4096 x 4096 R=16 4.70-4.72 against R=8 4.83;
        // 5632 x 2048 R=2 (2816 blocks) 4.12-4.13 against R=8 (704) 4.24,
        // its FFN form 5.93-5.95 against 6.07; 4096 x 2048 keeps R=8 (3.83;
        // R=16 3.74, R=4 3.57).  11008 x 4096 has no such R and keeps R=16.
        constexpr int RW = WAVES == 2 ? (RM < 8 ? RM : 8) : RM;
        auto whole = [&](uint32_t R) { const uint32_t nb = (a.N + R - 1) / R; return nb >= cus && nb % cus == 0u; };
        if constexpr (RW >= 16) {
            if (whole(16)) return launch_m1<WAVES, CPW, 16, EPI, false, TAIL>(a, dev, stream, variant);
        }
        if constexpr (RW >= 8) {
            if (whole(8)) return launch_m1<WAVES, CPW, 8, EPI, false, TAIL>(a, dev, stream, variant);
        }
        if constexpr (RW >= 4) {
            if (whole(4)) return launch_m1<WAVES, CPW, 4, EPI, false, TAIL>(a, dev, stream, variant);
        }
        if (whole(2)) return launch_m1<WAVES, CPW, 2, EPI, false, TAIL>(a, dev, stream, variant);
    }
    const uint32_t want = (TAIL ? 1u : 2u) * cus;
    if constexpr (RM >= 16) {
        if ((a.N + 15) / 16 >= want) return launch_m1<WAVES, CPW, 16, EPI, false, TAIL>(a, dev, stream, variant);
    }
    if constexpr (RM >= 8) {
        if ((a.N + 7) / 8 >= want) return launch_m1<WAVES, CPW, 8, EPI, false, TAIL>(a, dev, stream, variant);
    }
    if constexpr (RM >= 4) {
        if ((a.N + 3) / 4 >= want) return launch_m1<WAVES, CPW, 4, EPI, false, TAIL>(a, dev, stream, variant);
    }
    return launch_m1<WAVES, CPW, 2, EPI, false, TAIL>(a, dev, stream, variant);
}

// One wave per chunk for 5 to 8 chunks (rows of 4097 .. 8192 codes): the
// chunks load side by side instead of one wave walking a second slot after
// its first (6-10 % faster from K = 4099 to 8192, same-process timings).
// Rows per block: the largest R that still gives 6 waves per CU.
template <int WAVES, int RMAX, int EPI, bool MASK, bool TAIL = false>
hipError_t dispatch_m1_wide_rows(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    constexpr int RM = EPI == kEpiFfn ? RMAX / 2 : RMAX;
    const uint64_t want = 6u * (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    auto waves = [&](uint32_t R) { return (uint64_t)((a.N + R - 1) / R) * WAVES; };
    if constexpr (RM >= 16) {
        if (waves(16) >= want) return launch_m1<WAVES, 1, 16, EPI, MASK, TAIL>(a, dev, stream, variant);
    }
    if constexpr (RM >= 8) {
        if (waves(8) >= want) return launch_m1<WAVES, 1, 8, EPI, MASK, TAIL>(a, dev, stream, variant);
    }
    if constexpr (RM >= 4) {
        if (waves(4) >= want) return launch_m1<WAVES, 1, 4, EPI, MASK, TAIL>(a, dev, stream, variant);
    }
    return launch_m1<WAVES, 1, 2, EPI, MASK, TAIL>(a, dev, stream, variant);
}

template <int WAVES, int RMAX, int EPI>
hipError_t dispatch_m1_wide(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    if (a.W % kChunkWords != 0u) return dispatch_m1_wide_rows<WAVES, RMAX, EPI, true>(a, dev, stream, variant);
    return dispatch_m1_wide_rows<WAVES, RMAX, EPI, false>(a, dev, stream, variant);
}

// 9 to 16 chunks (K up to 16384): one wave per chunk as well, at most 8 rows
// per block and the largest R that still gives every CU a workgroup (4-12 %
// faster than 4 waves of 4 chunk slots each, same-process timings from
// K = 9000 to 16384).
template <int WAVES, int EPI>
hipError_t dispatch_m1_wider(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    constexpr int RM = EPI == kEpiFfn ? 4 : 8;
    const uint32_t want = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    if constexpr (RM >= 8) {
        if ((a.N + 7) / 8 >= want) return launch_m1<WAVES, 1, 8, EPI>(a, dev, stream, variant);
    }
    if ((a.N + 3) / 4 >= want) return launch_m1<WAVES, 1, 4, EPI>(a, dev, stream, variant);
    return launch_m1<WAVES, 1, 2, EPI>(a, dev, stream, variant);
}

template <int EPI>
hipError_t dispatch_m1(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    // 1 to 8 whole chunks and 1 to 4 more words: no wave streams the partial
    // chunk; one extra wave loads its words (the tail form of m1_row_block)
    if (a.W % kChunkWords >= 1u && a.W % kChunkWords <= 4u) {
        switch (a.W / kChunkWords) {
            case 1: return dispatch_m1_rows<1, 1, 16, EPI, true>(a, dev, stream, variant);
            case 2: return dispatch_m1_rows<2, 1, 16, EPI, true>(a, dev, stream, variant);
            case 3: return dispatch_m1_rows<3, 1, 16, EPI, true>(a, dev, stream, variant);
            case 4: return dispatch_m1_rows<4, 1, 16, EPI, true>(a, dev, stream, variant);
            case 5: return dispatch_m1_wide_rows<5, 16, EPI, false, true>(a, dev, stream, variant);
            case 6: return dispatch_m1_wide_rows<6, 16, EPI, false, true>(a, dev, stream, variant);
            case 7: return dispatch_m1_wide_rows<7, 16, EPI, false, true>(a, dev, stream, variant);
            case 8: return dispatch_m1_wide_rows<8, 16, EPI, false, true>(a, dev, stream, variant);
            default: break;
        }
    }
    const uint32_t C = (a.W + kChunkWords - 1) / kChunkWords;
    if (C == 1) return dispatch_m1_rows<1, 1, 16, EPI>(a, dev, stream, variant);
    if (C == 2) return dispatch_m1_rows<2, 1, 16, EPI>(a, dev, stream, variant);
    if (C == 3) return dispatch_m1_rows<3, 1, 16, EPI>(a, dev, stream, variant);
    if (C == 4) return dispatch_m1_rows<4, 1, 16, EPI>(a, dev, stream, variant);
    if (C == 5) return dispatch_m1_wide<5, 16, EPI>(a, dev, stream, variant);
    if (C == 6) return dispatch_m1_wide<6, 16, EPI>(a, dev, stream, variant);
    if (C == 7) return dispatch_m1_wide<7, 16, EPI>(a, dev, stream, variant);
    if (C == 8) return dispatch_m1_wide<8, 16, EPI>(a, dev, stream, variant);
    switch (C) {
        case 9: return dispatch_m1_wider<9, EPI>(a, dev, stream, variant);
        case 10: return dispatch_m1_wider<10, EPI>(a, dev, stream, variant);
        case 11: return dispatch_m1_wider<11, EPI>(a, dev, stream, variant);
        case 12: return dispatch_m1_wider<12, EPI>(a, dev, stream, variant);
        case 13: return dispatch_m1_wider<13, EPI>(a, dev, stream, variant);
        case 14: return dispatch_m1_wider<14, EPI>(a, dev, stream, variant);
        case 15: return dispatch_m1_wider<15, EPI>(a, dev, stream, variant);
        case 16: return dispatch_m1_wider<16, EPI>(a, dev, stream, variant);
        default: break;
    }
    return dispatch_m1_rows<4, 0, 4, EPI>(a, dev, stream, variant);
}

template <int WAVES, int CPW, int R, int MV>
hipError_t launch_mv(const MatvecArgs& a, hipStream_t stream, Variant* variant) {
    const uint32_t nblocks = (a.N + R - 1) / R;
    // groups of MV vectors on grid y, at most 65535 per launch
    const uint32_t groups = (a.M + MV - 1) / MV;
    for (uint32_t g0 = 0; g0 < groups; g0 += 65535u) {
        const uint32_t gy = groups - g0 < 65535u ? groups - g0 : 65535u;
        const uint32_t m0 = g0 * (uint32_t)MV;
        hipLaunchKernelGGL((matvec_q8_mv_kernel<WAVES, CPW, R, MV>), dim3(nblocks, gy), dim3(WAVES * 64), 0, stream,
                           a.weight, a.scale, a.vector + (size_t)m0 * a.K, a.output + (size_t)m0 * a.N, a.N, a.K, a.W,
                           a.M - m0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    set_variant(variant, "matvec_q8_mv", "valu", WAVES, R, CPW, MV, nblocks, groups);
    return hipSuccess;
}

// One workgroup per CU (the LDS stages and partial sums take 96 KiB), each
// with a contiguous range of 16-row tiles; vector groups of ks_vectors<PACK>()
// on grid y.  STW adds the store wave (K <= 1024 only: with two steps per
// wave the x parts need more registers than nine waves per workgroup leave).
template <int SW, int PACK, bool STW = false>
hipError_t launch_ksplit(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    constexpr uint32_t VPB = ks_vectors<PACK>();
    const uint32_t ntiles = (a.N + 15u) / 16u;
    const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    const dim3 grid(ntiles < cus ? ntiles : cus, (a.M + VPB - 1u) / VPB);
    const size_t lds = kKsLdsBytes + (STW ? (size_t)((ntiles + grid.x - 1u) / grid.x + 1u) * 16u * 4u : 0u);
    hipLaunchKernelGGL((matvec_q8_ksplit_kernel<SW, PACK, STW>), grid, dim3(64 * (kKsWaves + (STW ? 1u : 0u))), lds,
                       stream,
                       a.weight, a.scale, a.vector, a.output, a.N, a.K, a.W, a.M);
    set_variant(variant, "matvec_q8_ksplit", PACK == 1 ? "x16" : PACK == 2 ? "x8" : "x5", (int)kKsWaves + (STW ? 1 : 0), 16, SW,
                (int)(a.M < VPB ? a.M : VPB), grid.x, grid.y);
    return hipGetLastError();
}

// Rows per workgroup: the largest R (up to RMAX) that still gives every SIMD
// a wave; fewer, fatter blocks load each vector slice fewer times.
template <int WAVES, int CPW, int RMAX, int MV>
hipError_t dispatch_mv_rows(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    const uint64_t want = 4u * (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    auto waves = [&](uint32_t R) { return (uint64_t)((a.N + R - 1) / R) * WAVES; };
    if constexpr (RMAX >= 16) {
        if (waves(16) >= want) return launch_mv<WAVES, CPW, 16, MV>(a, stream, variant);
    }
    if constexpr (RMAX >= 8) {
        if (waves(8) >= want) return launch_mv<WAVES, CPW, 8, MV>(a, stream, variant);
    }
    return launch_mv<WAVES, CPW, 4, MV>(a, stream, variant);
}

// Waves per workgroup and vector-slice form by the number of 1 KiB chunks per
// row, as for one vector; slices stay in VGPRs while they take at most 128
// per lane (CPW * MV * 16), otherwise each slot loads its own.
template <int MV>
hipError_t dispatch_mv(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    constexpr int RM = MV >= 8 ? 8 : 16;
    const uint32_t C = (a.W + kChunkWords - 1) / kChunkWords;
    if (C == 1) return dispatch_mv_rows<1, 1, RM, MV>(a, dev, stream, variant);
    if (C == 2) return dispatch_mv_rows<2, 1, RM, MV>(a, dev, stream, variant);
    if (C == 3) return dispatch_mv_rows<3, 1, RM, MV>(a, dev, stream, variant);
    if (C == 4) return dispatch_mv_rows<4, 1, RM, MV>(a, dev, stream, variant);
    // two or more slots per wave: at most 8 rows per block (VGPRs)
    if constexpr (MV <= 4) {
        if (C <= 8) return dispatch_mv_rows<4, 2, 8, MV>(a, dev, stream, variant);
    }
    if constexpr (MV <= 2) {
        if (C <= 16) return dispatch_mv_rows<4, 4, 8, MV>(a, dev, stream, variant);
    }
    return dispatch_mv_rows<4, 0, 8, MV>(a, dev, stream, variant);
}

}  // namespace

hipError_t launch_matvec_q8(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream,
                            Variant* variant) {
    if (a.N == 0 || a.M == 0) return hipSuccess;
    if (a.K == 0) {
        // No terms: y = 0 * s (NaN for a non-finite scale), as the reference.
        return launch_fill_scaled_zero(a.scale, a.output, a.N, a.M, stream);
    }
    if (a.M == 1) return dispatch_m1<kEpiPlain>(a, dev, stream, variant);
    // Batched, 768 < K <= 2048 on large weights: codes split across a
    // workgroup's waves, x parts in VGPRs (every wave busy from K > 896; at
    // K = 512 half of them would idle and the kernels below win).  Against
    // the kernels below (same-process, MI355X): 1.1-1.5x from 5 vectors at
    // 16384 <= N <= 151936, 2.6-3.4x at K = 2048 with 16 vectors; with 4
    // vectors it wins from N = 32768, and the VALU path keeps 2 and 3.
    // Below 16384 rows (decoder-sized weights) it wins where the VALU path's
    // M + 1 operations per code outgrow the k-split kernel's cost, about one
    // fixed pass (~10 us at K = 2048, ~6 us at K = 1024) per round of one
    // workgroup per CU.  Same-process, launches queued, VALU -> k-split (us):
    // K = 2048: 11008 rows x 5 / 16 vectors 14.4 -> 10.9 / 23.9 -> 12.8,
    // 5632 x 12 / 16 15.4 -> 9.9 / 16.2 -> 10.9, 2048 x 32 12.6 -> 10.5;
    // K = 1024: 8192 x 5 6.7 -> 6.3, 5632 x 8 6.7 -> 6.2, 4096 x 16 7.5 ->
    // 6.6.  The VALU path keeps 4096 rows at K = 2048 (9.7 against 10.7 at 16
    // vectors), 4 vectors, and two or more rounds at 4096 rows or fewer.
    const auto ksplit_small = [&]() {
        const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
        const uint32_t ntiles = (a.N + 15u) / 16u;
        const bool one_round = (uint64_t)(ntiles < cus ? ntiles : cus) * ((a.M + 15u) / 16u) <= cus;
        if (a.M >= 32u && one_round) return true;
        if (a.K > 1024u) return (a.N >= 11008u && a.M >= 5u) || (a.N >= 5632u && a.M >= 12u);
        return (a.N >= 8192u && a.M >= 5u) || (a.N >= 5632u && a.M >= 8u) ||
               (a.N >= 4096u && a.M >= 12u && a.M <= 16u);
    };
    if (a.K > 768u && a.K <= 2048u && (a.M + 15u) / 16u <= 65535u &&
        (a.N >= kMfmaMinRows ? (a.M >= 5u || (a.M == 4u && a.N >= 32768u)) : ksplit_small())) {
        if (a.K <= 1024u) {
            // The store wave holds its workgroup's scales in LDS beside the
            // 96 KiB of stages and partials: up to 1023 tiles per workgroup
            // (4.19M rows on 256 CUs); past that, the eight-wave form.
            const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
            const uint32_t ntiles = (a.N + 15u) / 16u, gx = ntiles < cus ? ntiles : cus;
            if (kKsLdsBytes + (uint64_t)((ntiles + gx - 1u) / gx + 1u) * 64u <= kMfmaLdsBytes) {
                if (a.M <= 5u) return launch_ksplit<1, 3, true>(a, dev, stream, variant);
                if (a.M <= 8u) return launch_ksplit<1, 2, true>(a, dev, stream, variant);
                return launch_ksplit<1, 1, true>(a, dev, stream, variant);
            }
            if (a.M <= 5u) return launch_ksplit<1, 3>(a, dev, stream, variant);
            if (a.M <= 8u) return launch_ksplit<1, 2>(a, dev, stream, variant);
            return launch_ksplit<1, 1>(a, dev, stream, variant);
        }
        if (a.M <= 5u) return launch_ksplit<2, 3>(a, dev, stream, variant);
        if (a.M <= 8u) return launch_ksplit<2, 2>(a, dev, stream, variant);
        return launch_ksplit<2, 1>(a, dev, stream, variant);
    }
    // Batched.  The matrix-core kernels pay a per-workgroup prologue (the x
    // parts of the whole K for their 16-vector tile, written to LDS) and a
    // 64-byte-per-row load pattern; they win only on large weights with at
    // least 5 vectors, where each workgroup streams many tiles and the VALU
    // path's 1 + M operations per code no longer hide under the streaming.
    // Everything else runs on the VALU path (up to 8 vectors per pass).
    // Measured on MI355X over N = 2048 .. 151936, K = 1024 .. 20000, M = 2 .. 16.
    {
        const uint32_t Kp = (a.K + 255u) / 256u * 256u;
        const uint32_t MC = a.M < 16u ? a.M : 16u;
        const uint64_t lds = 3ull * MC * Kp * 2u + 4ull * kTileSlotFloats * 4u;
        if (a.M >= 5u && a.N >= kMfmaMinRows && lds <= kMfmaLdsBytes && (a.M + 15u) / 16u <= 65535u) {
            const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
            const uint32_t ntiles = (a.N + 15u) / 16u;
            const uint32_t wgs = (uint32_t)(kMfmaLdsBytes / lds) < 2u ? (uint32_t)(kMfmaLdsBytes / lds) : 2u;
            const uint32_t grid = min((ntiles + 3u) / 4u, cus * wgs);
            const dim3 g(grid, (a.M + 15u) / 16u);
            // The weight tiles go straight into LDS (whole 128-byte lines per
            // load instruction) whenever the stages fit beside the x parts:
            // two tiles per step (one B read serves both) when they fit, one
            // tile per step up to 4 vectors in a tile.
            {
                const uint64_t xbytes = 3ull * MC * Kp * 2u + 4ull * kTileSlotFloats * 4u;
                const uint64_t lds1 = xbytes + 4ull * kDmaStages * 1u * kDmaTileBytes;
                const uint64_t lds2 = xbytes + 4ull * kDmaStages * 2u * kDmaTileBytes;
                const bool two = MC > 4u && lds2 <= kMfmaLdsBytes;
                const uint64_t ldsd = two ? lds2 : lds1;
                // one tile per step pays a B read per tile: from 5 vectors the
                // register form (two tiles per step) is faster than that
                if (two || (MC <= 4u && ldsd <= kMfmaLdsBytes)) {
                    const uint32_t wg2 = (uint32_t)(kMfmaLdsBytes / ldsd) < 2u ? 1u : 2u;
                    const dim3 g2(min((ntiles + 3u) / 4u, cus * wg2), (a.M + 15u) / 16u);
                    if (!two)
                        hipLaunchKernelGGL((matvec_q8_mfma_dma_kernel<1, kDmaStages>), g2, dim3(256), (size_t)ldsd, stream,
                                           a.weight, a.scale, a.vector, a.output, a.N, a.K, a.W, a.M, Kp);
                    else
                        hipLaunchKernelGGL((matvec_q8_mfma_dma_kernel<2, kDmaStages>), g2, dim3(256), (size_t)ldsd, stream,
                                           a.weight, a.scale, a.vector, a.output, a.N, a.K, a.W, a.M, Kp);
                    set_variant(variant, "matvec_q8_mfma_dma", two ? "T2.4waves.256" : "T1.4waves.256", 4, 16 * (two ? 2 : 1),
                                0, (int)MC, g2.x, g2.y);
                    return hipGetLastError();
                }
                // 13 to 16 vectors: two tiles per step no longer fit beside the
                // x parts, but one tile per step in 128-code steps does, shared
                // by 8 waves (two per SIMD): cfg5 (N = 151936, K = 1024) at
                // 16 vectors in 42.0 us against 45-46 on the register-load
                // kernel below.
                const uint64_t lds8 = 3ull * MC * Kp * 2u + 8ull * kTileSlotFloats * 4u +
                                      8ull * kDmaStages * 1u * 16u * 128u;
                if (MC > 12u && lds8 <= kMfmaLdsBytes) {
                    const dim3 g8(min((ntiles + 3u) / 4u, cus), (a.M + 15u) / 16u);
                    hipLaunchKernelGGL((matvec_q8_mfma_dma_kernel<1, kDmaStages, 8, 128>), g8, dim3(512), (size_t)lds8,
                                       stream, a.weight, a.scale, a.vector, a.output, a.N, a.K, a.W, a.M, Kp);
                    set_variant(variant, "matvec_q8_mfma_dma", "T1.8waves.128", 8, 16, 0, (int)MC, g8.x, g8.y);
                    return hipGetLastError();
                }
            }
            if (MC >= 12u)
                hipLaunchKernelGGL((matvec_q8_mfma_kernel<2, 2>), g, dim3(256), (size_t)lds, stream, a.weight, a.scale,
                                   a.vector, a.output, a.N, a.K, a.W, a.M, Kp);
            else
                hipLaunchKernelGGL((matvec_q8_mfma_kernel<1, 3>), g, dim3(256), (size_t)lds, stream, a.weight, a.scale,
                                   a.vector, a.output, a.N, a.K, a.W, a.M, Kp);
            set_variant(variant, "matvec_q8_mfma", MC >= 12u ? "T2.D2" : "T1.D3", 4, MC >= 12u ? 32 : 16, 0, (int)MC, g.x,
                        g.y);
            return hipGetLastError();
        }
    }
    if (a.M <= 2) return dispatch_mv<2>(a, dev, stream, variant);
    if (a.M <= 4) return dispatch_mv<4>(a, dev, stream, variant);
    return dispatch_mv<8>(a, dev, stream, variant);
}

hipError_t launch_matvec_q8_fused(const MatvecArgs& a, int epi, const DeviceInfo& dev, hipStream_t stream,
                                  Variant* variant) {
    if (a.N == 0) return hipSuccess;
    if (a.M != 1 || (epi != kEpiResidual && epi != kEpiFfn)) return hipErrorInvalidValue;
    if (a.K == 0) return launch_fused_zero(a, epi, stream);
    return epi == kEpiFfn ? dispatch_m1<kEpiFfn>(a, dev, stream, variant)
                          : dispatch_m1<kEpiResidual>(a, dev, stream, variant);
}

namespace {

template <int WAVES, int CPW, int R>
hipError_t launch_multi(const Projection* p, uint32_t count, const float* x, uint32_t K, hipStream_t stream,
                        Variant* variant) {
    Projection q[kMaxProjections] = {};
    uint32_t start[kMaxProjections + 1];
    start[0] = 0;
    for (uint32_t i = 0; i < kMaxProjections; ++i) {
        if (i < count) q[i] = p[i];
        start[i + 1] = start[i] + (q[i].N + R - 1) / R;
    }
    const uint32_t nblocks = start[count];
    for (uint32_t i = count; i < kMaxProjections; ++i) start[i] = 0xffffffffu;
    hipLaunchKernelGGL((matvec_q8_multi_kernel<WAVES, CPW, R>), dim3(nblocks), dim3(WAVES * 64), 0, stream, x, K,
                       (K + 3) / 4, start[1], start[2], start[3], q[0].weight, q[0].scale, q[0].output, q[0].N,
                       q[1].weight, q[1].scale, q[1].output, q[1].N, q[2].weight, q[2].scale, q[2].output, q[2].N,
                       q[3].weight, q[3].scale, q[3].output, q[3].N);
    set_variant(variant, "matvec_q8_multi", CPW > 0 ? "xreg" : "xstream", WAVES, R, CPW, 1, nblocks);
    return hipGetLastError();
}

template <int WAVES, int CPW, int RMAX>
hipError_t dispatch_multi_rows(const Projection* p, uint32_t count, const float* x, uint32_t K,
                               const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    // The rows-per-block rule of the single-vector kernel, over the
    // projections' blocks together.
    const uint64_t want = 2u * (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    auto blocks = [&](uint32_t R) {
        uint64_t b = 0;
        for (uint32_t i = 0; i < count; ++i) b += (p[i].N + (uint64_t)R - 1) / R;
        return b;
    };
    if constexpr (RMAX >= 16) {
        if (blocks(16) >= want) return launch_multi<WAVES, CPW, 16>(p, count, x, K, stream, variant);
    }
    if constexpr (RMAX >= 8) {
        if (blocks(8) >= want) return launch_multi<WAVES, CPW, 8>(p, count, x, K, stream, variant);
    }
    if constexpr (RMAX >= 4) {
        if (blocks(4) >= want) return launch_multi<WAVES, CPW, 4>(p, count, x, K, stream, variant);
    }
    return launch_multi<WAVES, CPW, 2>(p, count, x, K, stream, variant);
}

// 5 to 8 chunks: one wave per chunk, as for a single projection.
template <int WAVES>
hipError_t dispatch_multi_wide(const Projection* p, uint32_t count, const float* x, uint32_t K,
                               const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    const uint64_t want = 6u * (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    auto waves = [&](uint32_t R) {
        uint64_t b = 0;
        for (uint32_t i = 0; i < count; ++i) b += (p[i].N + (uint64_t)R - 1) / R;
        return b * WAVES;
    };
    if (waves(16) >= want) return launch_multi<WAVES, 1, 16>(p, count, x, K, stream, variant);
    if (waves(8) >= want) return launch_multi<WAVES, 1, 8>(p, count, x, K, stream, variant);
    if (waves(4) >= want) return launch_multi<WAVES, 1, 4>(p, count, x, K, stream, variant);
    return launch_multi<WAVES, 1, 2>(p, count, x, K, stream, variant);
}

// 9 to 16 chunks: one wave per chunk, as for a single projection.
template <int WAVES>
hipError_t dispatch_multi_wider(const Projection* p, uint32_t count, const float* x, uint32_t K,
                                const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    const uint64_t want = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    auto blocks = [&](uint32_t R) {
        uint64_t b = 0;
        for (uint32_t i = 0; i < count; ++i) b += (p[i].N + (uint64_t)R - 1) / R;
        return b;
    };
    if (blocks(8) >= want) return launch_multi<WAVES, 1, 8>(p, count, x, K, stream, variant);
    if (blocks(4) >= want) return launch_multi<WAVES, 1, 4>(p, count, x, K, stream, variant);
    return launch_multi<WAVES, 1, 2>(p, count, x, K, stream, variant);
}

}  // namespace

hipError_t launch_matvec_q8_multi(const Projection* projections, uint32_t count, const float* x, uint32_t K,
                                  const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    Projection p[kMaxProjections];
    uint32_t n = 0;
    uint64_t rows = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (projections[i].N == 0) continue;
        if (n == kMaxProjections) return hipErrorInvalidValue;
        p[n++] = projections[i];
        rows += projections[i].N;
    }
    if (n == 0) return hipSuccess;
    // One projection, no vector terms, or a grid past 2^31 - 1 blocks (the
    // blocks hold at least 2 rows each): the single-vector path per
    // projection.
    if (n == 1 || K == 0 || rows / 2 + kMaxProjections >= 0x7fffffffu) {
        for (uint32_t i = 0; i < n; ++i) {
            MatvecArgs a{p[i].weight, p[i].scale, x, p[i].output, p[i].N, K, 1, (K + 3) / 4};
            const hipError_t e = launch_matvec_q8(a, dev, stream, variant);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const uint32_t C = ((K + 3) / 4 + kChunkWords - 1) / kChunkWords;
    if (C == 1) return dispatch_multi_rows<1, 1, 16>(p, n, x, K, dev, stream, variant);
    if (C == 2) return dispatch_multi_rows<2, 1, 16>(p, n, x, K, dev, stream, variant);
    if (C == 3) return dispatch_multi_rows<3, 1, 16>(p, n, x, K, dev, stream, variant);
    if (C == 4) return dispatch_multi_rows<4, 1, 16>(p, n, x, K, dev, stream, variant);
    if (C == 5) return dispatch_multi_wide<5>(p, n, x, K, dev, stream, variant);
    if (C == 6) return dispatch_multi_wide<6>(p, n, x, K, dev, stream, variant);
    if (C == 7) return dispatch_multi_wide<7>(p, n, x, K, dev, stream, variant);
    if (C == 8) return dispatch_multi_wide<8>(p, n, x, K, dev, stream, variant);
    switch (C) {
        case 9: return dispatch_multi_wider<9>(p, n, x, K, dev, stream, variant);
        case 10: return dispatch_multi_wider<10>(p, n, x, K, dev, stream, variant);
        case 11: return dispatch_multi_wider<11>(p, n, x, K, dev, stream, variant);
        case 12: return dispatch_multi_wider<12>(p, n, x, K, dev, stream, variant);
        case 13: return dispatch_multi_wider<13>(p, n, x, K, dev, stream, variant);
        case 14: return dispatch_multi_wider<14>(p, n, x, K, dev, stream, variant);
        case 15: return dispatch_multi_wider<15>(p, n, x, K, dev, stream, variant);
        case 16: return dispatch_multi_wider<16>(p, n, x, K, dev, stream, variant);
        default: break;
    }
    return dispatch_multi_rows<4, 0, 4>(p, n, x, K, dev, stream, variant);
}

// K = 0: every dot product is 0.
__global__ void fused_zero_kernel(M1Params p, int epi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < p.N; i += gridDim.x * blockDim.x) {
        if (epi == kEpiFfn)
            p.y[i] = ffn_epilogue(0.0f * p.scale[i], 0.0f * p.scale2[i]);
        else
            p.y[i] = residual_epilogue(p.residual[i], 0.0f * p.scale[i]);
    }
}

hipError_t launch_fused_zero(const MatvecArgs& a, int epi, hipStream_t stream) {
    const M1Params p{a.weight, a.scale, a.weight2, a.scale2, a.vector, a.residual, a.output, a.N, a.K, a.W};
    const uint32_t grid = (a.N + 255) / 256 < 4096 ? (a.N + 255) / 256 : 4096;
    hipLaunchKernelGGL(fused_zero_kernel, dim3(grid), dim3(256), 0, stream, p, epi);
    return hipGetLastError();
}

__global__ void fill_scaled_zero_kernel(const float* __restrict__ scale, float* __restrict__ y, uint32_t N,
                                        uint32_t M) {
    const size_t total = (size_t)N * M;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x)
        y[i] = 0.0f * scale[i % N];
}

hipError_t launch_fill_scaled_zero(const float* scale, float* y, uint32_t N, uint32_t M, hipStream_t stream) {
    const size_t total = (size_t)N * M;
    const uint32_t grid = (uint32_t)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
    hipLaunchKernelGGL(fill_scaled_zero_kernel, dim3(grid), dim3(256), 0, stream, scale, y, N, M);
    return hipGetLastError();
}

}  // namespace wxo
