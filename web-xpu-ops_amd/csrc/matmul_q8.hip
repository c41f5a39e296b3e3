// matmul_q8.hip -- W8A32 GEMM (prefill) for gfx950 on the matrix cores:
// out[n, m] = (sum_k a[n, k] * q[m, k]) * s[m], a f32 [N, K] (tokens),
// weight [M, ceil(K/4)] packed int8 (matvecQ8's wire format), out f32 [N, M].
//
// Reference: ops/matmul/reference.ts:124-137 (matmulQ8) -- the reference
// dequantizes each weight term to f32 (fround(q * s)) and runs the f64 triple
// loop of matmul (:37-49); its own doc defines the op as "N independent
// matvecQ8 calls against the same weight" (:76-77).  This kernel computes
// that matvecQ8 form: the exact dot product of codes and activations, then
// the row scale once.  Against the reference's per-term form the two differ
// by at most one f32 rounding of each term, 2^-24 of sum |a * q * s|, far
// inside the 1e-5 bar the tests hold.
//
// Exactness on bf16 matrix cores: a code q in [-128, 127] is exact in bf16;
// each activation a is split by truncation into a = h + m + l, three bf16
// parts of 8 significant bits each (a non-finite a stays whole in h, with a
// canonical quiet NaN), so every product q * part is exact in f32 and
// v_mfma_f32_16x16x32_bf16 sums them in f32.  Each 1024-code slice of K is
// summed in the matrix-core accumulator (96 accumulations) and then folded
// into an outer f32 sum, so no rounding chain exceeds ~96 + K/1024 steps:
// for K = 11008 that is under 110 roundings, 7e-6 of sum |terms|.
//
// Tiling: a workgroup of NW = 8 waves (2 over the weight rows x 4 over the
// tokens; 4 waves, 2 x 2, also build) owns BM = 32 FB weight rows x BN = 64
// tokens and walks K in steps of 64 codes.  Each step, the threads load the
// tile's packed codes (one dwordx4 of 16 codes per chunk) and activations
// (one token's 64 / NW consecutive k per thread), convert them once (codes ->
// bf16, activations -> three bf16 parts) into LDS, and after one barrier
// every wave reads its operand fragments with ds_read_b128 and issues
// FB x (4 / (NW / 2)) x 2 x 3 matrix-core ops.  Two waves per SIMD let one
// wave's LDS and barrier waits overlap the other's work (measured: 357 ->
// 310 us for a 512-token layer against 4 waves).
// The LDS holds two stages: while a wave's matrix cores work on step i, its
// VALU converts step i + 1 into the other stage, and global loads run two
// steps ahead of their conversion in two register sets.  The non-finite handling of the split is a wave-uniform branch taken
// only by waves that hold an Inf or NaN.  Rows of 64 codes (128 bytes of bf16) are
// stored with their 16-byte pieces XOR-swizzled by row, so the 16 rows one
// fragment read touches fall in distinct bank groups.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (probed on gfx950): A lane l
// holds A[l % 16][8 (l / 16) + e], B lane l holds B[8 (l / 16) + e][l % 16],
// C lane l holds C[4 (l / 16) + v][l % 16].  A = weight rows (16 features),
// B = activations (16 tokens), so a lane's C values are 4 consecutive
// features of one token: one 16-byte store into out[token, :].
//
// Workgroups are numbered so that the 8 XCDs (which take workgroups
// round-robin) each hold a contiguous run of tiles that share activation
// tiles in that XCD's L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"
#include "wave_ops.hpp"

namespace wxo {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kBN = 64;            // tokens per workgroup
constexpr uint32_t kFoldCodes = 1024;   // fold the accumulator every 1024 codes
constexpr uint32_t kMaxMatmulProjections = 4;

// Up to four projections of the same activations in one launch: projection p
// owns weight-row tiles [mt0[p], mt0[p + 1]) of the launch's tile sequence
// (mt0[p] = 0xffffffff past the last one).  A launch whose tiles' K steps are
// split between XS workgroups writes part 0's sums into the outputs and part
// j's (j >= 1) into part + (j - 1) * partstride + partoff[p], laid out as
// the outputs are; split_sum_kernel then adds them.
struct MatmulProjections {
    const uint32_t* weight[kMaxMatmulProjections];
    const float* scale[kMaxMatmulProjections];
    float* out[kMaxMatmulProjections];
    uint32_t M[kMaxMatmulProjections];
    uint32_t mt0[kMaxMatmulProjections];
    float* part;
    uint32_t partoff[kMaxMatmulProjections];
    uint32_t partstride;
};



__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
    // upper halves of two f32 bit patterns, a in the low half
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// 16 codes (4 packed words) -> 16 bf16 in two 16-byte pieces.
__device__ __forceinline__ void codes16_to_bf16(u32x4v w, u32x4v& lo, u32x4v& hi) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t r[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float c0 = (float)(int8_t)(ws[q]);
        const float c1 = (float)(int8_t)(ws[q] >> 8);
        const float c2 = (float)(int8_t)(ws[q] >> 16);
        const float c3 = (float)((int32_t)ws[q] >> 24);
        r[2 * q] = hi_pair(__float_as_uint(c0), __float_as_uint(c1));
        r[2 * q + 1] = hi_pair(__float_as_uint(c2), __float_as_uint(c3));
    }
    lo = u32x4v{r[0], r[1], r[2], r[3]};
    hi = u32x4v{r[4], r[5], r[6], r[7]};
}

// Splits activations into bf16 parts h + m + l (bit patterns in the upper
// halves).  Finite values split exactly by truncation: h keeps the top 8
// significant bits, r = a - h is exact, m keeps r's top 8, l = r - m is exact
// with at most 8 significant bits.  A non-finite value keeps all of itself in
// h (a NaN canonicalised, so truncating its payload cannot make it Inf) and
// m = l = 0, so Inf and NaN reach the products as IEEE arithmetic has them.
__device__ __forceinline__ void split3_fast(uint32_t bits, uint32_t& h, uint32_t& m, uint32_t& l, float& r) {
    h = bits & 0xffff0000u;
    r = __uint_as_float(bits) - __uint_as_float(h);
    m = __float_as_uint(r) & 0xffff0000u;
    l = __float_as_uint(r - __uint_as_float(m));
}

__device__ __forceinline__ void split3_any(uint32_t bits, uint32_t& h, uint32_t& m, uint32_t& l) {
    const bool finite = (bits & 0x7f800000u) != 0x7f800000u;
    const bool nan = (bits & 0x7fffffffu) > 0x7f800000u;
    const uint32_t hf = bits & 0xffff0000u;
    const float r = finite ? __uint_as_float(bits) - __uint_as_float(hf) : 0.0f;
    h = finite ? hf : (nan ? 0x7fc00000u : bits);
    m = __float_as_uint(r) & 0xffff0000u;
    l = __float_as_uint(r - __uint_as_float(m));
}

// XS > 1 splits every tile's K steps between XS workgroups as well (short
// prompts, whose few tiles would leave most CUs idle): part xs takes the
// xs-th run of the steps, stores its unscaled sums (above), and the sum
// kernel adds the parts in part order and scales them.
template <int FB, int NW, int BK, int PD, int KS, int XS = 1>
__global__ __launch_bounds__(64 * NW * KS) void matmul_q8_kernel(const float* __restrict__ a, MatmulProjections P,
                                                        uint32_t N, uint32_t K, uint32_t W, uint32_t mtiles,
                                                        uint32_t ntiles) {
    constexpr uint32_t BM = 32u * FB;                 // weight rows per workgroup
    constexpr uint32_t kBK = (uint32_t)BK;            // codes per K step
    constexpr uint32_t kRowBytes = kBK * 2u;          // one LDS row: BK bf16
    constexpr uint32_t kFoldSteps = kFoldCodes / kBK;
    constexpr uint32_t CPR = kBK / 16u;               // 16-code chunks per row and step
    constexpr uint32_t AST = BM * kRowBytes;          // bytes of one A stage
    constexpr uint32_t BST = 3u * kBN * kRowBytes;    // bytes of one B stage (three parts)
    constexpr uint32_t NT = 64u * NW;                 // threads of one K group
    constexpr uint32_t ACH = BM * CPR;                // 16-code chunks of A per step
    constexpr int AL = (int)((ACH + NT - 1u) / NT);   // A loads per thread per step
    constexpr uint32_t FPT = kBK / NW;                // activations per thread per step
    constexpr int BL = (int)(FPT / 4u);               // B loads (dwordx4) per thread per step
    constexpr int TB = (int)(4u / (NW / 2u));         // 16-token blocks per wave (2 or 1)
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(BK == 64 || BK == 128, "64- or 128-code steps");
    static_assert(PD == 2 || PD == 4, "2 or 4 register sets of loads in flight");
    static_assert(kFoldSteps % (uint32_t)PD == 0u, "a fold group starts on register set 0 and stage 0");
    static_assert(KS == 1 || KS == 2, "K split over 1 or 2 groups of NW waves");
    static_assert(XS == 1 || XS == 2 || XS == 4, "K split over 1, 2 or 4 workgroups");
    constexpr uint32_t NP = (uint32_t)(KS * XS);      // parts of a tile's K steps
    // Per K group: [A0 A1 B0 B1]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    // XCD-aware tile order: workgroup i runs on XCD i % 8; give each XCD a
    // contiguous run of the (token-major) tile sequence.
    const uint32_t total = mtiles * ntiles * (uint32_t)XS;
    const uint32_t per = (total + 7u) / 8u;
    const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
    const uint32_t lin = xcd * per + slot;
    if (lin >= total) return;  // whole workgroup: no barrier is skipped by part of it
    const uint32_t tile = XS == 1 ? lin : lin / (uint32_t)XS;
    const uint32_t xs = XS == 1 ? 0u : lin - tile * (uint32_t)XS;  // which run of the K steps
    const uint32_t nt = tile / mtiles, mt = tile - nt * mtiles;
    // the projection that owns weight-row tile mt (wave-uniform)
    const uint32_t pj = (mt >= P.mt0[1] ? 1u : 0u) + (mt >= P.mt0[2] ? 1u : 0u) + (mt >= P.mt0[3] ? 1u : 0u);
    const uint32_t* __restrict__ weight = P.weight[pj];
    const float* __restrict__ scale = P.scale[pj];
    float* __restrict__ out = P.out[pj];
    const uint32_t M = P.M[pj];
    const uint32_t m0 = (mt - P.mt0[pj]) * BM, n0 = nt * kBN;

    // KS groups of NW waves share the tile and split its K steps in halves;
    // their sums meet in LDS at the end.
    const uint32_t kg = KS == 1 ? 0u : __builtin_amdgcn_readfirstlane(threadIdx.x / NT);
    const uint32_t gbase = kg * (2u * AST + 2u * BST);  // this group's stages (0 for KS = 1)
    const uint32_t t = KS == 1 ? threadIdx.x : threadIdx.x % NT;
    const uint32_t lane = t & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t wm = (wv & 1u) * (BM / 2u);            // wave's first weight row in the tile
    const uint32_t wn = (wv >> 1) * (16u * (uint32_t)TB);  // wave's first token in the tile
    const uint32_t j = lane & 15u, g = lane >> 4;

    const uint32_t mrows = min(BM, M - m0);
    const uint32_t ntok = min(kBN, N - n0);
    const uint32_t rowbytes = W * 4u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)m0 * W, mrows * rowbytes);
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(a + (size_t)n0 * K, ntok * K * 4u);

    // Global load assignment.  A: thread t, load u -> chunk t + NT u: row
    // chunk / 4, codes 16 (chunk % 4) .. +15 of the step (threads past the
    // tile's chunks load nothing; with BM = 64 and 8 waves that is waves 4-7,
    // a wave-uniform split).  B: token t / NW, k FPT (t % NW) .. +FPT-1.
    const uint32_t ac = t % CPR;
    const uint32_t ar = t / CPR;
    const uint32_t btok = t / NW;
    const uint32_t bc = t % NW;
    const int boff = (int)((btok * K + bc * FPT) * 4u);

    // PD register sets of global loads: step i's data sits in set i % PD,
    // loaded PD steps ahead of its conversion.
    u32x4v ga[PD][AL], gb[PD][BL];
    auto issue = [&](int b, uint32_t k0) {
#pragma unroll
        for (int u = 0; u < AL; ++u)
            if (ACH % NT == 0u || t + NT * (uint32_t)u < ACH)  // wave-uniform
                ga[b][u] = load_nt_b128(wrs, (int)((ar + (NT / CPR) * (uint32_t)u) * rowbytes + ac * 16u), (int)k0);
#pragma unroll
        for (int q = 0; q < BL; ++q)
            gb[b][q] = __builtin_amdgcn_raw_buffer_load_b128(ars, boff + 16 * q, (int)(k0 * 4u), 0);
    };

    // Zeroes, in register set s, the activations at k >= K of step k0 (they
    // belong to the next token).  Only the last step of a ragged K needs it;
    // the caller branches before the matrix work, so the conversion that
    // follows stays in one block with it.
    auto mask_b = [&](int s, uint32_t k0) {
        const uint32_t kb = k0 + bc * FPT;
#pragma unroll
        for (int q = 0; q < BL; ++q) {
            if (kb + 4u * (uint32_t)q >= K) gb[s][q].x = 0u;
            if (kb + 4u * (uint32_t)q + 1u >= K) gb[s][q].y = 0u;
            if (kb + 4u * (uint32_t)q + 2u >= K) gb[s][q].z = 0u;
            if (kb + 4u * (uint32_t)q + 3u >= K) gb[s][q].w = 0u;
        }
    };
    auto load_b = [&](int s, uint32_t (&v)[FPT]) {
#pragma unroll
        for (int q = 0; q < BL; ++q) {
            v[4 * q] = gb[s][q].x;
            v[4 * q + 1] = gb[s][q].y;
            v[4 * q + 2] = gb[s][q].z;
            v[4 * q + 3] = gb[s][q].w;
        }
    };
    // The three parts of the thread's FPT activations into stage s: FPT / 8
    // 16-byte pieces per part, starting at piece bc * FPT / 8 of the row.
    auto store_b = [&](int s, const uint32_t (&hp)[FPT / 2], const uint32_t (&mp)[FPT / 2],
                       const uint32_t (&lp)[FPT / 2]) {
        uint8_t* row = lds + gbase + 2u * AST + (uint32_t)s * BST + btok * kRowBytes;
#pragma unroll
        for (uint32_t q = 0; q < FPT / 8u; ++q) {
            const uint32_t pc = ((bc * (FPT / 8u) + q) ^ (btok & 7u)) * 16u;
            *reinterpret_cast<u32x4v*>(row + pc) = u32x4v{hp[4 * q], hp[4 * q + 1], hp[4 * q + 2], hp[4 * q + 3]};
            *reinterpret_cast<u32x4v*>(row + kBN * kRowBytes + pc) =
                u32x4v{mp[4 * q], mp[4 * q + 1], mp[4 * q + 2], mp[4 * q + 3]};
            *reinterpret_cast<u32x4v*>(row + 2u * kBN * kRowBytes + pc) =
                u32x4v{lp[4 * q], lp[4 * q + 1], lp[4 * q + 2], lp[4 * q + 3]};
        }
    };
    // Writes the converted step into stage s and returns the thread's
    // non-finite indicator.  Row r's 16-byte piece p sits at piece p ^ (r & 7).
    auto convert_store = [&](int s, int st) -> float {
        uint8_t* as = lds + gbase + (uint32_t)st * AST;
#pragma unroll
        for (int u = 0; u < AL; ++u) {
            if (!(ACH % NT == 0u || t + NT * (uint32_t)u < ACH)) continue;  // wave-uniform
            const uint32_t r = ar + (NT / CPR) * (uint32_t)u;
            u32x4v lo, hi;
            codes16_to_bf16(ga[s][u], lo, hi);
            const uint32_t p0 = (2u * ac) ^ (r & 7u), p1 = (2u * ac + 1u) ^ (r & 7u);
            *reinterpret_cast<u32x4v*>(as + r * kRowBytes + p0 * 16u) = lo;
            *reinterpret_cast<u32x4v*>(as + r * kRowBytes + p1 * 16u) = hi;
        }
        uint32_t v[FPT];
        load_b(s, v);
        // Split all FPT the fast way.  r = a - h is NaN exactly when a is not
        // finite, so the sum of the r's tells whether this thread needs the
        // slower split; the caller redoes the stage for a wave that does
        // (nonfinite_fixup), outside the block the scheduler interleaves with
        // the matrix work.
        uint32_t hp[FPT / 2], mp[FPT / 2], lp[FPT / 2];
        float rsum = 0.0f;
#pragma unroll
        for (int e = 0; e < (int)FPT; e += 2) {
            uint32_t h0, m0_, l0, h1, m1, l1;
            float r0, r1;
            split3_fast(v[e], h0, m0_, l0, r0);
            split3_fast(v[e + 1], h1, m1, l1, r1);
            rsum += r0 + r1;
            hp[e / 2] = hi_pair(h0, h1);
            mp[e / 2] = hi_pair(m0_, m1);
            lp[e / 2] = hi_pair(l0, l1);
        }
        store_b(st, hp, mp, lp);
        return rsum;
    };

    // The same activation conversion for every value, Inf and NaN included.
    auto nonfinite_fixup = [&](int s, int st) {
        uint32_t v[FPT];
        load_b(s, v);
        uint32_t hp[FPT / 2], mp[FPT / 2], lp[FPT / 2];
#pragma unroll
        for (int e = 0; e < (int)FPT; e += 2) {
            uint32_t h0, m0_, l0, h1, m1, l1;
            split3_any(v[e], h0, m0_, l0);
            split3_any(v[e + 1], h1, m1, l1);
            hp[e / 2] = hi_pair(h0, h1);
            mp[e / 2] = hi_pair(m0_, m1);
            lp[e / 2] = hi_pair(l0, l1);
        }
        store_b(st, hp, mp, lp);
    };

    f32x4 acc[FB][TB], sum[FB][TB];
#pragma unroll
    for (int f = 0; f < FB; ++f)
#pragma unroll
        for (int b = 0; b < TB; ++b) {
            acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
            sum[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    // Matrix work of one stage: two 32-code substeps.
    auto compute = [&](int s) {
        const uint8_t* as = lds + gbase + (uint32_t)s * AST;
        const uint8_t* bs = lds + gbase + 2u * AST + (uint32_t)s * BST;
#pragma unroll
        for (int ss = 0; ss < BK / 32; ++ss) {
            const uint32_t piece = 4u * (uint32_t)ss + g;
            bf16x8 af[FB], bf[TB][3];
#pragma unroll
            for (int f = 0; f < FB; ++f) {
                const uint32_t r = wm + 16u * (uint32_t)f + j;
                af[f] = *reinterpret_cast<const bf16x8*>(as + r * kRowBytes + ((piece ^ (r & 7u)) * 16u));
            }
#pragma unroll
            for (int b = 0; b < TB; ++b) {
                const uint32_t tk = wn + 16u * (uint32_t)b + j;
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    bf[b][p] = *reinterpret_cast<const bf16x8*>(bs + ((uint32_t)p * kBN + tk) * kRowBytes +
                                                                ((piece ^ (tk & 7u)) * 16u));
            }
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int f = 0; f < FB; ++f)
#pragma unroll
                    for (int b = 0; b < TB; ++b)
                        acc[f][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[f], bf[b][p], acc[f][b], 0, 0, 0);
        }
    };

    // Software pipeline, one barrier per step: iteration i converts step
    // i + 1 (register set (i + 1) % PD, LDS stage (i + 1) & 1) and refills
    // that set with step i + 1 + PD, then runs step i's matrix work on stage
    // i & 1.  A step's loads thus have PD iterations to arrive.  The
    // conversion (VALU) and the matrix work are independent, so a wave
    // overlaps them.  Past the last step the conversion writes a stage nobody
    // reads and the loads fall outside the buffer resources (they return 0).
    const uint32_t steps = (K + kBK - 1u) / kBK;
    const bool ragged = (K % kBK) != 0u;
    // This group's steps: [s0, s0 + gs), run xs * KS + kg of NP; every group
    // runs `iters` iterations (the same barriers), skipping the matrix work
    // past its own steps.
    const uint32_t iters = NP == 1u ? steps : (steps + NP - 1u) / NP;
    const uint32_t s0 = (xs * (uint32_t)KS + kg) * iters;
    const uint32_t gs = NP == 1u ? steps : (s0 < steps ? min(iters, steps - s0) : 0u);
    auto convert_checked = [&](int s, int st) {
        const float rsum = convert_store(s, st);
        if (__builtin_amdgcn_ballot_w64(__builtin_isnan(rsum)) != 0) nonfinite_fixup(s, st);  // uniform
    };
#pragma unroll
    for (int q = 0; q < PD; ++q) issue(q, (s0 + (uint32_t)q) * kBK);
    if (ragged && s0 + 1u == steps) mask_b(0, s0 * kBK);
    convert_checked(0, 0);
    issue(0, (s0 + (uint32_t)PD) * kBK);
    __syncthreads();
    // The matrix work comes first in program order: its LDS reads then need
    // not wait behind the conversion's LDS writes, and the scheduler can fill
    // the matrix-core latency with the conversion's VALU work.  q = i % PD.
    auto iter = [&](int q, uint32_t i) {
        const int nx = (q + 1) % PD;
        if (ragged && s0 + i + 2u == steps) mask_b(nx, (s0 + i + 1u) * kBK);  // uniform
        if (NP == 1u || i < gs) compute(q & 1);                                // uniform
        convert_checked(nx, (q + 1) & 1);
        issue(nx, (s0 + i + 1u + (uint32_t)PD) * kBK);
        __syncthreads();
    };
    // Steps run in groups of kFoldSteps (a multiple of PD, so a group starts
    // on register set 0 and stage 0); the accumulator is folded into the
    // outer sum after each group.
    for (uint32_t g0 = 0; g0 < iters; g0 += kFoldSteps) {
        const uint32_t gend = min(g0 + kFoldSteps, iters);
        uint32_t i = g0;
        for (; i + (uint32_t)PD <= gend; i += (uint32_t)PD) {
#pragma unroll
            for (int q = 0; q < PD; ++q) iter(q, i + (uint32_t)q);
        }
#pragma unroll
        for (int q = 0; q < PD - 1; ++q)
            if (i + (uint32_t)q < gend) iter(q, i + (uint32_t)q);
#pragma unroll
        for (int f = 0; f < FB; ++f)
#pragma unroll
            for (int b = 0; b < TB; ++b) {
                sum[f][b] += acc[f][b];
                acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
    }

    if constexpr (KS > 1) {
        // Group 1's sums through LDS (its stages are done) into group 0's.
        constexpr uint32_t E = (uint32_t)(FB * TB * 4);
        float* red = reinterpret_cast<float*>(lds);
        __syncthreads();
        if (kg == 1u) {
#pragma unroll
            for (int f = 0; f < FB; ++f)
#pragma unroll
                for (int b = 0; b < TB; ++b)
#pragma unroll
                    for (int v = 0; v < 4; ++v) red[((uint32_t)((f * TB + b) * 4 + v)) * NT + t] = sum[f][b][v];
        }
        __syncthreads();
        if (kg != 0u) return;  // after the last barrier
#pragma unroll
        for (int f = 0; f < FB; ++f)
#pragma unroll
            for (int b = 0; b < TB; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) sum[f][b][v] += red[((uint32_t)((f * TB + b) * 4 + v)) * NT + t];
        static_assert(E * NT * 4u <= 2u * AST + 2u * BST, "the reduction fits in group 0's stages");
    }

    // Epilogue: lane (j, g) of block (f, b) holds features m0 + wm + 16 f +
    // 4 g .. +3 of token n0 + wn + 16 b + j.  A split launch stores the
    // unscaled sums: part 0 into the output, part xs into its part buffer.
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + m0, XS == 1 ? mrows * 4u : 0u);
    float* const dst = XS == 1 || xs == 0u ? out : P.part + (size_t)(xs - 1u) * P.partstride + P.partoff[pj];
#pragma unroll
    for (int f = 0; f < FB; ++f) {
        const uint32_t fm = wm + 16u * (uint32_t)f + 4u * g;  // within the tile
        u32x4v sv = {0x3f800000u, 0x3f800000u, 0x3f800000u, 0x3f800000u};  // 1.0f
        if constexpr (XS == 1) sv = __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(fm * 4u), 0, 0);
#pragma unroll
        for (int b = 0; b < TB; ++b) {
            const uint32_t tok = wn + 16u * (uint32_t)b + j;
            if (tok >= ntok) continue;
            f32x4 y;
            if constexpr (XS == 1) {
                y[0] = sum[f][b][0] * __uint_as_float(sv.x);
                y[1] = sum[f][b][1] * __uint_as_float(sv.y);
                y[2] = sum[f][b][2] * __uint_as_float(sv.z);
                y[3] = sum[f][b][3] * __uint_as_float(sv.w);
            } else {
                y = sum[f][b];
            }
            float* o = dst + (size_t)(n0 + tok) * M + m0 + fm;
            if (fm + 3u < mrows) {
                *reinterpret_cast<f32x4_a4*>(o) = f32x4_a4{y[0], y[1], y[2], y[3]};
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (fm + (uint32_t)q < mrows) o[q] = y[q];
            }
        }
    }
}

// out = (part 0 + part 1 + ... + part parts-1) * scale, in part order, for
// every output of a split launch (grid y: projection).
__global__ __launch_bounds__(256) void split_sum_kernel(MatmulProjections P, uint32_t N, uint32_t parts) {
    const uint32_t p = blockIdx.y;
    float* __restrict__ y = P.out[p];
    const float* __restrict__ sc = P.scale[p];
    const uint32_t M = P.M[p];
    const float* part = P.part + P.partoff[p];
    const uint32_t n = N * M;
    for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < n; e += gridDim.x * blockDim.x) {
        float v = y[e];
        for (uint32_t j = 1; j < parts; ++j) v += part[(size_t)(j - 1u) * P.partstride + e];
        y[e] = v * sc[e % M];
    }
}

__global__ void fill_zero_kernel(float* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        y[i] = 0.0f;
}

// One launch over `count` (1 to 4) projections of the same activations.
// One launch over `count` (1 to 4) projections of the same activations; with
// XS > 1 a second, the sum of the parts (`part` holds (XS - 1) x the
// launch's outputs).
template <int FB, int NW, int BK, int PD, int KS = 1, int XS = 1>
hipError_t launch_fb(const float* a, const MatmulProjection* p, uint32_t count, uint32_t N, uint32_t K,
                     hipStream_t stream, float* part = nullptr) {
    constexpr uint32_t kRowBytes = (uint32_t)BK * 2u;
    constexpr uint32_t BM = 32u * FB;
    const uint32_t W = (uint32_t)(((uint64_t)K + 3) / 4);
    MatmulProjections P = {};
    uint32_t mtiles = 0, outs = 0;
    for (uint32_t i = 0; i < kMaxMatmulProjections; ++i) {
        if (i < count) {
            P.weight[i] = p[i].weight;
            P.scale[i] = p[i].scale;
            P.out[i] = p[i].output;
            P.M[i] = p[i].M;
            P.mt0[i] = mtiles;
            P.partoff[i] = outs;
            mtiles += (p[i].M + BM - 1u) / BM;
            if constexpr (XS > 1) outs += N * p[i].M;  // a split launch's outputs fit 32 bits (its tiles fit the CUs)
        } else {
            P.mt0[i] = 0xffffffffu;
        }
    }
    P.part = part;
    P.partstride = outs;
    const uint32_t ntiles = (N + kBN - 1u) / kBN;
    const uint32_t total = mtiles * ntiles * (uint32_t)XS;
    const uint32_t grid = ((total + 7u) / 8u) * 8u;
    const size_t lds = (size_t)KS * (2u * BM * kRowBytes + 2u * 3u * kBN * kRowBytes);
    hipLaunchKernelGGL((matmul_q8_kernel<FB, NW, BK, PD, KS, XS>), dim3(grid), dim3(64 * NW * KS), lds, stream, a, P, N,
                       K, W, mtiles, ntiles);
    if constexpr (XS > 1) {
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        uint32_t most = 0;
        for (uint32_t i = 0; i < count; ++i) most = most > N * p[i].M ? most : N * p[i].M;
        const uint32_t gx = (most + 255u) / 256u < 1024u ? (most + 255u) / 256u : 1024u;
        hipLaunchKernelGGL(split_sum_kernel, dim3(gx, count), dim3(256), 0, stream, P, N, (uint32_t)XS);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_matmul_q8_multi(const float* a, const MatmulProjection* projections, uint32_t count, uint32_t N,
                                  uint32_t K, const DeviceInfo& dev, hipStream_t stream, Variant* variant,
                                  float* workspace, size_t workspace_bytes) {
    static_assert(kMaxMatmulProjectionsPerLaunch == kMaxMatmulProjections, "one launch's projection table");
    MatmulProjection p[kMaxMatmulProjections];
    uint32_t n = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (projections[i].M == 0) continue;
        if (n == kMaxMatmulProjections) return hipErrorInvalidValue;
        p[n++] = projections[i];
    }
    if (N == 0 || n == 0) return hipSuccess;
    if (K == 0) {
        // matmul over an empty K: every sum is 0 (ops/matmul/reference.ts:17-18)
        for (uint32_t i = 0; i < n; ++i) {
            const size_t e = (size_t)N * p[i].M;
            const uint32_t grid = (uint32_t)((e + 255) / 256 < 65536 ? (e + 255) / 256 : 65536);
            hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, stream, p[i].output, e);
            set_variant(variant, "fill_zero", "matmul.k0", 4, 0, 0, 0, grid);
            const hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
        }
        return hipSuccess;
    }
    // Up to 32 tokens: the batched single-vector path, one token per vector
    // (out[n, m] is y[vector n][row m], the same layout), one call per
    // projection.  The GEMM walks all of K in a serial chain of steps per
    // workgroup whatever the token count (20 us for 1 token at 2048 x 2048);
    // the batched path streams the weight once per 8 or 16 tokens (3.6 us
    // for 1 token, 10.5 us for 32; the GEMM wins from about 64 tokens).
    // Both compute the matvecQ8 form.
    if (N <= 32u) {
        for (uint32_t i = 0; i < n; ++i) {
            MatvecArgs mv{p[i].weight, p[i].scale, a, p[i].output, p[i].M, K, N, (uint32_t)(((uint64_t)K + 3) / 4)};
            const hipError_t e = launch_matvec_q8(mv, dev, stream, variant);
            if (e != hipSuccess) return e;
            if (variant) variant->form = "matmul.tokens_as_vectors";
        }
        return hipSuccess;
    }
    // 128 weight rows per workgroup when that still gives every CU a tile,
    // otherwise 64 rows with four register sets of loads in flight (6-16 %
    // faster than two at 64-row tiles from K = 2048 to 11008, and faster than
    // 128-code steps; with 128-row tiles the extra registers cost more than
    // they save).  When the tiles fit in one workgroup per CU, two groups of
    // 8 waves split each tile's K steps (half the serial chain; 8-15 %
    // faster, 512 x 4096 x 11008 in 172 us against 197); with more tiles the
    // smaller one-group workgroups (two per CU) win.  Short prompts whose
    // 32-row tiles still fit one workgroup per CU take those: each tile's
    // steps move less through LDS and twice the CUs work (64 tokens, 2048 x
    // 2048: 18.5 -> 16.2 us; 2048 x 5632: 44.7 -> 38.3 us; the same sums in
    // the same order, so the same bits).  Projections in one launch count
    // their tiles together.
    const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    const uint64_t ntiles = (N + kBN - 1u) / kBN;
    uint64_t t4 = 0, t2 = 0, t1 = 0;
    for (uint32_t i = 0; i < n; ++i) {
        t4 += (uint64_t)((p[i].M + 127u) / 128u) * ntiles;
        t2 += (uint64_t)((p[i].M + 63u) / 64u) * ntiles;
        t1 += (uint64_t)((p[i].M + 31u) / 32u) * ntiles;
    }
    if (t4 >= cus) {
        set_variant(variant, n > 1 ? "matmul_q8.multi" : "matmul_q8", t4 <= cus ? "FB4.ksplit2" : "FB4",
                    t4 <= cus ? 16 : 8, 128, 0, (int)kBN, (uint32_t)((t4 + 7u) / 8u * 8u));
        return t4 <= cus ? launch_fb<4, 8, 64, 2, 2>(a, p, n, N, K, stream)
                         : launch_fb<4, 8, 64, 2, 1>(a, p, n, N, K, stream);
    }
    if (t1 <= cus) {
        // With a workspace, tiles that fill at most half (a quarter) of the
        // CUs also split their K steps between 2 (4) workgroups, each run at
        // least 4 steps per K group; the parts' sums meet in a second launch.
        uint64_t outs = 0;  // the launch's outputs
        for (uint32_t i = 0; i < n; ++i) outs += (uint64_t)N * p[i].M;
        const uint32_t steps = (uint32_t)(((uint64_t)K + 63u) / 64u);
        const char* kname = n > 1 ? "matmul_q8.multi" : "matmul_q8";
        if (workspace && 4u * t1 <= cus && steps >= 32u && 3u * outs * 4u <= workspace_bytes) {
            set_variant(variant, kname, "FB1.PD4.ksplit2.wgsplit4", 16, 32, 0, (int)kBN, (uint32_t)((4u * t1 + 7u) / 8u * 8u));
            return launch_fb<1, 8, 64, 4, 2, 4>(a, p, n, N, K, stream, workspace);
        }
        if (workspace && 2u * t1 <= cus && steps >= 16u && outs * 4u <= workspace_bytes) {
            set_variant(variant, kname, "FB1.PD4.ksplit2.wgsplit2", 16, 32, 0, (int)kBN, (uint32_t)((2u * t1 + 7u) / 8u * 8u));
            return launch_fb<1, 8, 64, 4, 2, 2>(a, p, n, N, K, stream, workspace);
        }
        set_variant(variant, kname, "FB1.PD4.ksplit2", 16, 32, 0, (int)kBN, (uint32_t)((t1 + 7u) / 8u * 8u));
        return launch_fb<1, 8, 64, 4, 2>(a, p, n, N, K, stream);
    }
    set_variant(variant, n > 1 ? "matmul_q8.multi" : "matmul_q8", t2 <= cus ? "FB2.PD4.ksplit2" : "FB2.PD4",
                t2 <= cus ? 16 : 8, 64, 0, (int)kBN, (uint32_t)((t2 + 7u) / 8u * 8u));
    return t2 <= cus ? launch_fb<2, 8, 64, 4, 2>(a, p, n, N, K, stream)
                     : launch_fb<2, 8, 64, 4, 1>(a, p, n, N, K, stream);
}

hipError_t launch_matmul_q8(const float* a, const uint32_t* weight, const float* scale, float* out, uint32_t N,
                            uint32_t M, uint32_t K, const DeviceInfo& dev, hipStream_t stream, Variant* variant) {
    const MatmulProjection p{weight, scale, out, M};
    return launch_matmul_q8_multi(a, &p, 1, N, K, dev, stream, variant, nullptr, 0);
}

}  // namespace wxo
