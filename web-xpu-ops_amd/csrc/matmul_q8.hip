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
// round-robin) each hold a contiguous run of the tile sequence, and the
// sequence walks groups of 4 weight-row tiles, each group through all its
// token tiles (tile_coords).  So an XCD's L2 holds about an eighth of the
// weight, reused by every token tile, and its resident workgroups share 4
// weight tiles and a few activation tiles.  A token-major sequence (each XCD
// one token tile and every weight row) streamed the whole weight through
// every XCD's L2: 512-token layer 215 -> 182 us, 2048 tokens 629 -> 570.
//
// With a caller's workspace, a launch may also split some tiles' K steps
// between 2, 4 or 8 workgroups (a short prompt's tiles, which would leave most
// CUs idle; the last tiles of a round that would load the CUs unevenly):
// part 0 stores its unscaled sums into the output, the other parts into
// tile-sized workspace blocks, and a second launch adds them in part order
// and scales them.  The stream order between the two launches is the only
// synchronisation, so every run gives the same bits.
//
// Long rows whose tiles make whole rounds of two per CU run one workgroup of
// 16 waves per two tiles, each group of 8 waves on a tile of its own (the
// PAIR instances); the sums are the one-group form's.
//
// Launches with enough tiles for one workgroup per CU, and short prompts'
// 256-row tiles split 4 or 8 ways, run matmul_q8_direct_kernel instead: every wave of 8 owns 16 FW weight rows and
// all 64 tokens of the tile, and loads its rows' codes straight into VGPRs
// (two dwordx2 per 16-row block and step, in the operand's k order), so only
// the activation parts pass through LDS.  That removes the codes' LDS writes
// (gfx950 writes LDS at ~75 B/clk per CU against ~200 for reads) and converts
// each code once per wave, at the matrix work.  Same sums in the same order
// as the one-group form, so the same bits; 2-7 % faster than it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"
#include "wave_ops.hpp"

namespace wxo {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

constexpr uint32_t kBN = 64;            // tokens per workgroup
constexpr uint32_t kFoldCodes = 1024;   // fold the accumulator every 1024 codes
constexpr uint32_t kMaxMatmulProjections = 4;

// Up to four projections of the same activations in one launch: projection p
// owns weight-row tiles [mt0[p], mt0[p + 1]) of the launch's tile sequence
// (mt0[p] = 0xffffffff past the last one).  A split launch runs its first
// `whole` tiles whole and splits the other `splits` tiles' K steps into
// `parts` runs, one workgroup each: part 0 stores its unscaled sums into the
// output, part j >= 1 into the workspace block (j - 1) * splits + (tile -
// whole) of BM x kBN floats ([token][row] within the tile), and
// split_sum_kernel adds the parts in part order and scales them.
struct MatmulProjections {
    const uint32_t* weight[kMaxMatmulProjections];
    const float* scale[kMaxMatmulProjections];
    float* out[kMaxMatmulProjections];
    uint32_t M[kMaxMatmulProjections];
    uint32_t mt0[kMaxMatmulProjections];
    float* part;
    uint32_t whole, splits, parts;
};



// Tile `tile` of the launch's sequence -> weight-row tile mt, token tile nt.
// The sequence takes kTileGroup row tiles at a time (fewer in the last
// group) and walks all token tiles of the group, its row tiles innermost:
// consecutive workgroups share activation tiles, and a group's weight tiles
// stay in one XCD's L2 while all token tiles use them.  Same-process sweep of
// the group size (1, 2, 4, 8, 16, all): 512-token layer 182 / 181 / 182 / 187
// / 199 / 215 us, 2048 tokens 574 / 573 / 570 / 572 / 581 / 629.
constexpr uint32_t kTileGroup = 4;
__device__ __forceinline__ void tile_coords(uint32_t tile, uint32_t mtiles, uint32_t ntiles, uint32_t& mt,
                                            uint32_t& nt) {
    const uint32_t gi = tile / (kTileGroup * ntiles), first = gi * kTileGroup;
    const uint32_t gs = min(kTileGroup, mtiles - first);
    const uint32_t r = tile - gi * (kTileGroup * ntiles);
    nt = r / gs;
    mt = first + (r - nt * gs);
}

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

// 8 codes (2 packed words) -> 8 bf16.
__device__ __forceinline__ bf16x8 codes8_to_bf16(u32x2v w) {
    const uint32_t ws[2] = {w.x, w.y};
    uint32_t r[4];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const float c0 = (float)(int8_t)(ws[q]);
        const float c1 = (float)(int8_t)(ws[q] >> 8);
        const float c2 = (float)(int8_t)(ws[q] >> 16);
        const float c3 = (float)((int32_t)ws[q] >> 24);
        r[2 * q] = hi_pair(__float_as_uint(c0), __float_as_uint(c1));
        r[2 * q + 1] = hi_pair(__float_as_uint(c2), __float_as_uint(c3));
    }
    return __builtin_bit_cast(bf16x8, u32x4v{r[0], r[1], r[2], r[3]});
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

// SPLIT instances take the split launch above: whole tiles plus split tiles
// whose K steps are shared by `parts` workgroups (a short prompt's few tiles,
// which would leave most CUs idle, or the tiles past the last whole round of
// a long prompt, which would leave some CUs with one tile more than others).
// PAIR instances (two K groups) run the first P.whole tiles two per
// workgroup, one whole tile per group, and the rest one per workgroup with
// the K steps split between the groups.  The other instances run every tile
// whole, with no branch on it.
template <int FB, int NW, int BK, int PD, int KS, bool SPLIT = false, bool PAIR = false>
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
    constexpr uint32_t WR = 2u;                        // waves over the rows
    constexpr int TB = (int)(4u * WR / NW);            // 16-token blocks per wave (2 or 1)
    constexpr int FW = (int)(BM / (16u * WR));         // 16-row blocks per wave
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(BK == 64 || BK == 128, "64- or 128-code steps");
    static_assert(PD == 2 || PD == 4, "2 or 4 register sets of loads in flight");
    static_assert(kFoldSteps % (uint32_t)PD == 0u, "a fold group starts on register set 0 and stage 0");
    static_assert(KS == 1 || KS == 2, "K split over 1 or 2 groups of NW waves");
    // Per K group: [A0 A1 B0 B1]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    // XCD-aware tile order: workgroup i runs on XCD i % 8; give each XCD a
    // contiguous run of the tile sequence (tile_coords).  A split launch
    // gives each XCD a run of the whole tiles first and then a run of the
    // split tiles' parts, so every XCD holds its share of both and the whole
    // tiles are dispatched first.  Workgroups past the end return whole (no
    // barrier is skipped by part of one).
    static_assert(!PAIR || (KS == 2 && !SPLIT), "pairs are the two K groups of a whole-tile launch");
    const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
    uint32_t tile, xs = 0u, np = (uint32_t)KS;  // np: runs of this tile's K steps
    bool pair = false;                          // this group runs a tile of its own
    if constexpr (PAIR) {
        const uint32_t pairs = P.whole / 2u, singles = mtiles * ntiles - P.whole;
        const uint32_t wpx = (pairs + 7u) / 8u;
        if (slot < wpx) {
            const uint32_t i = xcd * wpx + slot;
            if (i >= pairs) return;
            tile = 2u * i + __builtin_amdgcn_readfirstlane(threadIdx.x / (64u * NW));
            np = 1u;
            pair = true;
        } else {
            const uint32_t q = xcd * ((singles + 7u) / 8u) + (slot - wpx);
            if (q >= singles) return;
            tile = P.whole + q;
        }
    } else if constexpr (!SPLIT) {
        const uint32_t total = mtiles * ntiles;
        const uint32_t lin = xcd * ((total + 7u) / 8u) + slot;
        if (lin >= total) return;
        tile = lin;
    } else {
        const uint32_t wpx = (P.whole + 7u) / 8u;
        if (slot < wpx) {
            const uint32_t i = xcd * wpx + slot;
            if (i >= P.whole) return;
            tile = i;
        } else {
            const uint32_t np_all = P.splits * P.parts;
            const uint32_t q = xcd * ((np_all + 7u) / 8u) + (slot - wpx);
            if (q >= np_all) return;
            tile = P.whole + q / P.parts;
            xs = q % P.parts;
            np = (uint32_t)KS * P.parts;
        }
    }
    uint32_t mt, nt;
    tile_coords(tile, mtiles, ntiles, mt, nt);
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
    const uint32_t wm = (wv % WR) * (BM / WR);                  // wave's first weight row in the tile
    const uint32_t wn = (wv / WR) * (16u * (uint32_t)TB);       // wave's first token in the tile
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

    f32x4 acc[FW][TB], sum[FW][TB];
#pragma unroll
    for (int f = 0; f < FW; ++f)
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
            bf16x8 af[FW], bf[TB][3];
#pragma unroll
            for (int f = 0; f < FW; ++f) {
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
                for (int f = 0; f < FW; ++f)
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
    // This group's steps: [s0, s0 + gs), run xs * KS + kg of np; every group
    // runs `iters` iterations (the same barriers), skipping the matrix work
    // past its own steps.
    constexpr bool kOneRun = KS == 1 && !SPLIT;  // every group takes all the steps: no skip
    const uint32_t iters = kOneRun ? steps : (steps + np - 1u) / np;
    const uint32_t s0 = kOneRun || pair ? 0u : (xs * (uint32_t)KS + kg) * iters;
    const uint32_t gs = kOneRun ? steps : (s0 < steps ? min(iters, steps - s0) : 0u);
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
        if (kOneRun || i < gs) compute(q & 1);                                 // uniform
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
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (int b = 0; b < TB; ++b) {
                sum[f][b] += acc[f][b];
                acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
    }

    if constexpr (KS > 1) {
        // Group 1's sums through LDS (its stages are done) into group 0's;
        // a pair's groups each store their own tile (`pair` is
        // workgroup-uniform, and always false outside PAIR instances).
        constexpr uint32_t E = (uint32_t)(FW * TB * 4);
        static_assert(E * NT * 4u <= 2u * AST + 2u * BST, "the reduction fits in group 0's stages");
        if (!pair) {
            float* red = reinterpret_cast<float*>(lds);
            __syncthreads();
            if (kg == 1u) {
#pragma unroll
                for (int f = 0; f < FW; ++f)
#pragma unroll
                    for (int b = 0; b < TB; ++b)
#pragma unroll
                        for (int v = 0; v < 4; ++v) red[((uint32_t)((f * TB + b) * 4 + v)) * NT + t] = sum[f][b][v];
            }
            __syncthreads();
            if (kg != 0u) return;  // after the last barrier
#pragma unroll
            for (int f = 0; f < FW; ++f)
#pragma unroll
                for (int b = 0; b < TB; ++b)
#pragma unroll
                    for (int v = 0; v < 4; ++v) sum[f][b][v] += red[((uint32_t)((f * TB + b) * 4 + v)) * NT + t];
        }
    }

    // Epilogue: lane (j, g) of block (f, b) holds features m0 + wm + 16 f +
    // 4 g .. +3 of token n0 + wn + 16 b + j.  A split tile stores unscaled
    // sums: part 0 into the output, part xs into its workspace block.
    const bool split = SPLIT && tile >= P.whole;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + m0, split ? 0u : mrows * 4u);
    float* const blk = SPLIT && xs > 0u
        ? P.part + ((size_t)(xs - 1u) * P.splits + (tile - P.whole)) * (size_t)(BM * kBN) : nullptr;
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        const uint32_t fm = wm + 16u * (uint32_t)f + 4u * g;  // within the tile
        const u32x4v sv = split ? u32x4v{0x3f800000u, 0x3f800000u, 0x3f800000u, 0x3f800000u}  // 1.0f
                                : __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(fm * 4u), 0, 0);
#pragma unroll
        for (int b = 0; b < TB; ++b) {
            const uint32_t tok = wn + 16u * (uint32_t)b + j;
            if (tok >= ntok) continue;
            f32x4 y;
            y[0] = sum[f][b][0] * __uint_as_float(sv.x);
            y[1] = sum[f][b][1] * __uint_as_float(sv.y);
            y[2] = sum[f][b][2] * __uint_as_float(sv.z);
            y[3] = sum[f][b][3] * __uint_as_float(sv.w);
            float* o = blk ? blk + tok * BM + fm : out + (size_t)(n0 + tok) * M + m0 + fm;
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

// The one-group GEMM with each wave's weight codes loaded straight into
// registers.  A workgroup of 8 waves owns BM = 128 FW weight rows x 64 tokens;
// wave w owns rows 16 FW w .. +16 FW - 1 and every token of the tile, so
// nothing it converts is shared and no code passes through LDS.  Per 64-code
// step, lane (j, g) of 16-row block f loads codes 8g .. 8g+7 and 32+8g ..
// 32+8g+7 of row 16 f + j (the operand's k order for the step's two 32-code
// halves) PD steps ahead; the activations go through the same double-buffered,
// XOR-swizzled LDS stage as matmul_q8_kernel, split into three parts once per
// workgroup.  Matrix ops, their order and the fold points are the one-group
// form's, so the bits are too.  SPLIT instances split every tile's K steps
// into P.parts runs, one workgroup each (P.whole = 0): part 0 stores its
// unscaled sums into the output, part j >= 1 into workspace block
// (j - 1) * P.splits + tile, and split_sum_kernel adds them in part order and
// scales them.
template <int FW, int PD, bool SPLIT = false>
__global__ __launch_bounds__(512) void matmul_q8_direct_kernel(const float* __restrict__ a, MatmulProjections P,
                                                               uint32_t N, uint32_t K, uint32_t W, uint32_t mtiles,
                                                               uint32_t ntiles) {
    constexpr uint32_t NW = 8u, TB = 4u;
    constexpr uint32_t BM = 16u * FW * NW;
    constexpr uint32_t kRowBytes = 128u;              // one LDS row: 64 codes of bf16
    constexpr uint32_t BST = 3u * kBN * kRowBytes;    // one stage: three parts of 64 tokens
    constexpr uint32_t NT = 64u * NW;
    constexpr uint32_t FPT = kBN * 64u / NT;          // activations per thread per step
    constexpr int BL = (int)(FPT / 4u);
    constexpr uint32_t TPT = NT / kBN;                // threads per token
    constexpr uint32_t kFoldSteps = kFoldCodes / 64u;
    static_assert(TB * 16u == kBN, "a wave covers the tile's tokens");
    static_assert(FPT % 8u == 0u, "whole 16-byte pieces per part");
    static_assert(kFoldSteps % (uint32_t)PD == 0u, "a fold group starts on register set 0 and stage 0");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    // XCD-aware order as matmul_q8_kernel: each XCD a contiguous run of the
    // sequence (of tiles, or of split tiles' parts, a tile's parts adjacent)
    const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
    const uint32_t parts = SPLIT ? P.parts : 1u;
    const uint32_t units = mtiles * ntiles * parts;
    const uint32_t lin = xcd * ((units + 7u) / 8u) + slot;
    if (lin >= units) return;
    const uint32_t tile = lin / parts, xs = lin - tile * parts;
    uint32_t mt, nt;
    tile_coords(tile, mtiles, ntiles, mt, nt);
    const uint32_t pj = (mt >= P.mt0[1] ? 1u : 0u) + (mt >= P.mt0[2] ? 1u : 0u) + (mt >= P.mt0[3] ? 1u : 0u);
    const uint32_t* __restrict__ weight = P.weight[pj];
    const float* __restrict__ scale = P.scale[pj];
    float* __restrict__ out = P.out[pj];
    const uint32_t M = P.M[pj];
    const uint32_t m0 = (mt - P.mt0[pj]) * BM, n0 = nt * kBN;

    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t wm = wv * (16u * FW);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t mrows = min(BM, M - m0), ntok = min(kBN, N - n0);
    const uint32_t rowbytes = W * 4u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(weight + (size_t)m0 * W, mrows * rowbytes);
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(a + (size_t)n0 * K, ntok * K * 4u);
    const uint32_t btok = t / TPT, bc = t % TPT;
    const int boff = (int)((btok * K + bc * FPT) * 4u);

    // PD register sets each of codes (set i % PD: step i, loaded PD steps
    // before its matrix work) and activations (loaded PD steps before their
    // conversion, one step ahead of the matrix work).
    u32x2v ga[PD][FW][2];
    u32x4v gb[PD][BL];
    auto issue_a = [&](int b, uint32_t k0) {
#pragma unroll
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                ga[b][f][h] = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(
                    wrs, (int)((wm + 16u * (uint32_t)f + j) * rowbytes + 8u * g + 32u * (uint32_t)h), (int)k0, 0));
    };
    auto issue_b = [&](int b, uint32_t k0) {
#pragma unroll
        for (int q = 0; q < BL; ++q)
            gb[b][q] = __builtin_amdgcn_raw_buffer_load_b128(ars, boff + 16 * q, (int)(k0 * 4u), 0);
    };
    // activations at k >= K of step k0 belong to the next token: zero
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
    auto store_b = [&](int st, const uint32_t (&hp)[FPT / 2], const uint32_t (&mp)[FPT / 2],
                       const uint32_t (&lp)[FPT / 2]) {
        uint8_t* row = lds + (uint32_t)st * BST + btok * kRowBytes;
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
    // The three parts of register set s into stage st; a wave holding an Inf
    // or NaN (r = a - h is NaN exactly then) redoes its part with the split
    // that handles every value.
    auto convert_b = [&](int s, int st) {
        uint32_t v[FPT];
#pragma unroll
        for (int q = 0; q < BL; ++q) {
            v[4 * q] = gb[s][q].x;
            v[4 * q + 1] = gb[s][q].y;
            v[4 * q + 2] = gb[s][q].z;
            v[4 * q + 3] = gb[s][q].w;
        }
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
        if (__builtin_amdgcn_ballot_w64(__builtin_isnan(rsum)) != 0) {  // wave-uniform
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
        }
    };

    f32x4 acc[FW][TB], sum[FW][TB];
#pragma unroll
    for (int f = 0; f < FW; ++f)
#pragma unroll
        for (uint32_t b = 0; b < TB; ++b) {
            acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
            sum[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    // Matrix work of one step: activation parts from stage st, codes from
    // register set q, two 32-code halves.
    auto compute = [&](int st, int q) {
        const uint8_t* bs = lds + (uint32_t)st * BST;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t piece = 4u * (uint32_t)h + g;
            bf16x8 af[FW], bf[TB][3];
#pragma unroll
            for (uint32_t b = 0; b < TB; ++b) {
                const uint32_t tk = 16u * b + j;
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    bf[b][p] = *reinterpret_cast<const bf16x8*>(bs + ((uint32_t)p * kBN + tk) * kRowBytes +
                                                                ((piece ^ (tk & 7u)) * 16u));
            }
#pragma unroll
            for (int f = 0; f < FW; ++f) af[f] = codes8_to_bf16(ga[q][f][h]);
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int f = 0; f < FW; ++f)
#pragma unroll
                    for (uint32_t b = 0; b < TB; ++b)
                        acc[f][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[f], bf[b][p], acc[f][b], 0, 0, 0);
        }
    };

    // One barrier per step: iteration i runs step i's matrix work (stage
    // i & 1, code set i % PD), refills that code set with step i + PD,
    // converts step i + 1's activations into the other stage and refills
    // their set with step i + 1 + PD.  Loads past K fall outside the buffer
    // resources and return 0.
    // This workgroup's steps: [s0, s0 + gs) (all of them unless SPLIT).
    // Loads past the run read the next part's steps or past K (0), unused.
    const uint32_t steps = (K + 63u) / 64u;
    const bool ragged = (K % 64u) != 0u;
    const uint32_t iters = (steps + parts - 1u) / parts;
    const uint32_t s0 = xs * iters;
    const uint32_t gs = s0 < steps ? min(iters, steps - s0) : 0u;
#pragma unroll
    for (int q = 0; q < PD; ++q) {
        issue_a(q, 64u * (s0 + (uint32_t)q));
        issue_b(q, 64u * (s0 + (uint32_t)q));
    }
    if (ragged && s0 + 1u == steps) mask_b(0, 64u * s0);
    convert_b(0, 0);
    issue_b(0, 64u * (s0 + (uint32_t)PD));
    __syncthreads();
    auto iter = [&](int q, uint32_t i) {
        const int nx = (q + 1) % PD;
        if (ragged && s0 + i + 2u == steps) mask_b(nx, (s0 + i + 1u) * 64u);  // uniform
        compute(q & 1, q);
        issue_a(q, (s0 + i + (uint32_t)PD) * 64u);
        convert_b(nx, (q + 1) & 1);
        issue_b(nx, (s0 + i + 1u + (uint32_t)PD) * 64u);
        __syncthreads();
    };
    for (uint32_t g0 = 0; g0 < gs; g0 += kFoldSteps) {
        const uint32_t gend = min(g0 + kFoldSteps, gs);
        uint32_t i = g0;
        for (; i + (uint32_t)PD <= gend; i += (uint32_t)PD) {
#pragma unroll
            for (int q = 0; q < PD; ++q) iter(q, i + (uint32_t)q);
        }
#pragma unroll
        for (int q = 0; q < PD - 1; ++q)
            if (i + (uint32_t)q < gend) iter(q, i + (uint32_t)q);
#pragma unroll
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (uint32_t b = 0; b < TB; ++b) {
                sum[f][b] += acc[f][b];
                acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
    }

    // lane (j, g) of block (f, b): rows m0 + wm + 16 f + 4 g .. +3 of token
    // n0 + 16 b + j.  A split tile's parts store unscaled sums: part 0 into
    // the output, part xs into its workspace block ([token][row] in the tile).
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(scale + m0, SPLIT ? 0u : mrows * 4u);
    float* const blk = SPLIT && xs > 0u ? P.part + ((size_t)(xs - 1u) * P.splits + tile) * (size_t)(BM * kBN) : nullptr;
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        const uint32_t fm = wm + 16u * (uint32_t)f + 4u * g;
        const u32x4v sv = SPLIT ? u32x4v{0x3f800000u, 0x3f800000u, 0x3f800000u, 0x3f800000u}  // 1.0f
                                : __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(fm * 4u), 0, 0);
#pragma unroll
        for (uint32_t b = 0; b < TB; ++b) {
            const uint32_t tok = 16u * b + j;
            if (tok >= ntok) continue;
            f32x4 y;
            y[0] = sum[f][b][0] * __uint_as_float(sv.x);
            y[1] = sum[f][b][1] * __uint_as_float(sv.y);
            y[2] = sum[f][b][2] * __uint_as_float(sv.z);
            y[3] = sum[f][b][3] * __uint_as_float(sv.w);
            float* o = blk ? blk + tok * BM + fm : out + (size_t)(n0 + tok) * M + m0 + fm;
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

// out = (part 0 + part 1 + ... + part parts-1) * scale, in part order (up to
// 8 parts), for every output of the split tiles of a split launch.  Grid x: split tile;
// grid y: BM / 16 slices of it; a thread takes 4 consecutive rows of one
// token (one 16-byte group of every part), all its loads in flight at once.
template <uint32_t BM>
__global__ __launch_bounds__(256) void split_sum_kernel(MatmulProjections P, uint32_t N, uint32_t mtiles) {
    constexpr uint32_t G = BM / 4u;  // 4-row groups per token
    static_assert(kBN * G == 256u * (BM / 16u), "one group per thread");
    const uint32_t st = blockIdx.x, tile = P.whole + st;
    uint32_t mt, nt;
    tile_coords(tile, mtiles, (N + kBN - 1u) / kBN, mt, nt);
    const uint32_t pj = (mt >= P.mt0[1] ? 1u : 0u) + (mt >= P.mt0[2] ? 1u : 0u) + (mt >= P.mt0[3] ? 1u : 0u);
    const uint32_t M = P.M[pj];
    const uint32_t m0 = (mt - P.mt0[pj]) * BM, n0 = nt * kBN;
    const uint32_t mrows = min(BM, M - m0), ntok = min(kBN, N - n0);
    const uint32_t e = blockIdx.y * 256u + threadIdx.x;  // group index within the tile
    const uint32_t t = e / G, r = (e - t * G) * 4u;
    if (t >= ntok || r >= mrows) return;
    float* y = P.out[pj] + (size_t)(n0 + t) * M + m0 + r;
    const float* sc = P.scale[pj] + m0 + r;
    const uint32_t parts = P.parts;
    const size_t blk = (size_t)BM * kBN, off = (size_t)st * blk + (size_t)t * BM + r;
    if (r + 3u < mrows) {
        f32x4 v = *reinterpret_cast<const f32x4_a4*>(y);
        const f32x4 s4 = *reinterpret_cast<const f32x4_a4*>(sc);
        f32x4 q[7];
#pragma unroll
        for (uint32_t j = 1; j < 8u; ++j)
            if (j < parts) q[j - 1u] = *reinterpret_cast<const f32x4*>(P.part + (size_t)(j - 1u) * P.splits * blk + off);
#pragma unroll
        for (uint32_t j = 1; j < 8u; ++j)
            if (j < parts) v += q[j - 1u];
        *reinterpret_cast<f32x4_a4*>(y) = v * s4;
    } else {
        for (uint32_t k = 0; k < mrows - r; ++k) {
            float v = y[k];
            for (uint32_t j = 1; j < parts; ++j) v += P.part[(size_t)(j - 1u) * P.splits * blk + off + k];
            y[k] = v * sc[k];
        }
    }
}

__global__ void fill_zero_kernel(float* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        y[i] = 0.0f;
}

// The launch's projection table for BM-row tiles; returns the row tiles of
// all projections together.
uint32_t fill_projections(const MatmulProjection* p, uint32_t count, uint32_t BM, MatmulProjections& P) {
    uint32_t mtiles = 0;
    for (uint32_t i = 0; i < kMaxMatmulProjections; ++i) {
        if (i < count) {
            P.weight[i] = p[i].weight;
            P.scale[i] = p[i].scale;
            P.out[i] = p[i].output;
            P.M[i] = p[i].M;
            P.mt0[i] = mtiles;
            mtiles += (p[i].M + BM - 1u) / BM;
        } else {
            P.mt0[i] = 0xffffffffu;
        }
    }
    return mtiles;
}

// One launch of matmul_q8_direct_kernel (128 FW-row tiles, PD register sets)
// over `count` projections of the same activations.
// With parts > 1 (a SPLIT instance) every tile's K steps split into `parts`
// runs, the workspace `part` holding (parts - 1) x tiles blocks of 128 FW x
// kBN floats, and split_sum_kernel sums them in a second launch.
template <int FW, int PD, bool SPLIT = false>
hipError_t launch_direct(const float* a, const MatmulProjection* p, uint32_t count, uint32_t N, uint32_t K,
                         hipStream_t stream, float* part = nullptr, uint32_t parts = 1) {
    constexpr uint32_t BM = 128u * FW;
    const uint32_t W = (uint32_t)(((uint64_t)K + 3) / 4);
    MatmulProjections P = {};
    const uint32_t mtiles = fill_projections(p, count, BM, P);
    const uint32_t ntiles = (N + kBN - 1u) / kBN;
    const uint32_t tiles = mtiles * ntiles;
    P.part = part;
    P.whole = 0;
    P.splits = SPLIT ? tiles : 0u;
    P.parts = SPLIT ? parts : 1u;
    const uint32_t grid = ((tiles * P.parts + 7u) / 8u) * 8u;
    const size_t lds = 2u * 3u * kBN * 128u;
    hipLaunchKernelGGL((matmul_q8_direct_kernel<FW, PD, SPLIT>), dim3(grid), dim3(512), lds, stream, a, P, N, K, W,
                       mtiles, ntiles);
    if constexpr (SPLIT) {
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        hipLaunchKernelGGL(split_sum_kernel<BM>, dim3(tiles, BM / 16u), dim3(256), 0, stream, P, N, mtiles);
    }
    return hipGetLastError();
}

// One launch over `count` (1 to 4) projections of the same activations.  With
// splits > 0 (a SPLIT instance) the last `splits` tiles of the sequence have
// their K steps split into `parts` runs, with the workspace `part` holding
// (parts - 1) x splits blocks of BM x kBN floats, and a second launch sums
// them.
template <int FB, int NW, int BK, int PD, int KS = 1, bool SPLIT = false, bool PAIR = false>
hipError_t launch_fb(const float* a, const MatmulProjection* p, uint32_t count, uint32_t N, uint32_t K,
                     hipStream_t stream, float* part = nullptr, uint32_t splits = 0, uint32_t parts = 1) {
    constexpr uint32_t kRowBytes = (uint32_t)BK * 2u;
    constexpr uint32_t BM = 32u * FB;
    const uint32_t W = (uint32_t)(((uint64_t)K + 3) / 4);
    MatmulProjections P = {};
    const uint32_t mtiles = fill_projections(p, count, BM, P);
    const uint32_t ntiles = (N + kBN - 1u) / kBN;
    const uint32_t tiles = mtiles * ntiles;
    P.part = part;
    P.whole = tiles - splits;
    P.splits = splits;
    P.parts = parts;
    uint32_t grid = ((tiles + 7u) / 8u) * 8u;
    if constexpr (SPLIT) grid = 8u * ((P.whole + 7u) / 8u + (splits * parts + 7u) / 8u);
    if constexpr (PAIR) {  // `splits` here: the tiles run in pairs (even)
        P.whole = splits;
        P.splits = 0;
        grid = 8u * ((splits / 2u + 7u) / 8u + (tiles - splits + 7u) / 8u);
    }
    const size_t lds = (size_t)KS * (2u * BM * kRowBytes + 2u * 3u * kBN * kRowBytes);
    hipLaunchKernelGGL((matmul_q8_kernel<FB, NW, BK, PD, KS, SPLIT, PAIR>), dim3(grid), dim3(64 * NW * KS), lds, stream, a,
                       P, N, K, W, mtiles, ntiles);
    if constexpr (SPLIT) {
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        hipLaunchKernelGGL(split_sum_kernel<BM>, dim3(splits, BM / 16u), dim3(256), 0, stream, P, N, mtiles);
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
    // their tiles together.  Launches whose tiles take one K group and no
    // split run on matmul_q8_direct_kernel (D256, D256.PD2, D128 below).
    const uint32_t cus = (uint32_t)(dev.cu_count > 0 ? dev.cu_count : 256);
    const uint64_t ntiles = (N + kBN - 1u) / kBN;
    uint64_t t8 = 0, t4 = 0, t2 = 0, t1 = 0;
    for (uint32_t i = 0; i < n; ++i) {
        t8 += (uint64_t)((p[i].M + 255u) / 256u) * ntiles;
        t4 += (uint64_t)((p[i].M + 127u) / 128u) * ntiles;
        t2 += (uint64_t)((p[i].M + 63u) / 64u) * ntiles;
        t1 += (uint64_t)((p[i].M + 31u) / 32u) * ntiles;
    }
    const uint32_t steps = (uint32_t)(((uint64_t)K + 63u) / 64u);
    const char* kname = n > 1 ? "matmul_q8.multi" : "matmul_q8";
    // 256-row tiles on the direct kernel (8 waves of 32 rows x 64 tokens, codes
    // straight into registers, four sets in flight), one workgroup per CU,
    // when those tiles make whole rounds of the CUs or at least 2.75 of them.
    // The sums and their order are the one-group 128-row form's, so are the
    // bits.  Same process, us, against 256-row tiles through LDS (4 of 8 waves
    // over the rows, 64 x 32 each), which had replaced the 128-row one-group
    // form (1024 x 4096 x 4096 129 -> 113): 1024 x 4096 x 4096 108 -> 98,
    // 2048 x 2048 x 2048 60 -> 56, 2048 x 6144 x 2048 164 -> 155, 2048 x
    // 11264 x 2048 304 -> 289, 2048 x 2048 x 5632 145 -> 134, 2048 x 4096 x
    // 11008 502 -> 475, 4096 x 4096 x 4096 391 -> 363.
    if (t8 >= cus && (t8 % cus == 0 || 4u * t8 >= 11u * (uint64_t)cus)) {
        set_variant(variant, kname, "D256", 8, 256, 0, (int)kBN, (uint32_t)((t8 + 7u) / 8u * 8u));
        return launch_direct<2, 4>(a, p, n, N, K, stream);
    }
    if (t4 >= cus) {
        if (t4 == cus) {
            set_variant(variant, kname, "FB4.ksplit2", 16, 128, 0, (int)kBN, (uint32_t)((t4 + 7u) / 8u * 8u));
            return launch_fb<4, 8, 64, 2, 2>(a, p, n, N, K, stream);
        }
        // Two workgroups per CU.  Between cus and 2 x cus tiles, some CUs
        // take two tiles and the others one (384 tiles: half and half).  With
        // a workspace, the last S = 2 x cus - tiles tiles split their K steps
        // in two, so that whole tiles plus halves fill the 2 x cus slots and
        // every CU holds the same work (384 tiles -> 256 whole and 256 halves,
        // one of each per CU).  The halves' sum is a second launch (~5 us
        // with its launch); with more tiles the dispatch already evens the
        // CUs out over several rounds and the split no longer pays (704
        // tiles: the GEMM 90 -> 85 us, plus the sum).  Same process, 512
        // tokens: q, k, v 54.9 -> 49.3 us; at 256 tokens gate and up 51.6 ->
        // 47.1.
        const uint64_t slots = 2ull * cus;
        const uint64_t S = t4 < slots ? slots - t4 : 0u;
        const size_t blk = (size_t)128u * kBN * 4u;
        // Where the 256-row tiles fill at least two thirds of the CUs, the
        // direct kernel on those tiles (one workgroup per CU, two register
        // sets) beats both the split and the uneven round, with or without a
        // workspace.  Same process, us, split -> 256-row direct: 512 tokens q,
        // k, v (192 tiles) 51.9 -> 48.7; 256 tokens gate and up (176) 53.9 ->
        // 49.9.  With fewer (96 at 256 tokens q, k, v) it loses to the 128-row
        // forms (31.6 -> 45.0).
        if (S > 0 && 3u * t8 >= 2u * (uint64_t)cus) {
            set_variant(variant, kname, "D256.PD2", 8, 256, 0, (int)kBN, (uint32_t)((t8 + 7u) / 8u * 8u));
            return launch_direct<2, 2>(a, p, n, N, K, stream);
        }
        if (workspace && S > 0 && steps >= 8u && S * blk <= workspace_bytes) {
            set_variant(variant, kname, "FB4.balance2", 8, 128, 0, (int)kBN, (uint32_t)(t4 + S));
            return launch_fb<4, 8, 64, 2, 1, true>(a, p, n, N, K, stream, workspace, (uint32_t)S, 2u);
        }
        // Long rows whose tiles make two or more whole rounds of two per CU:
        // one workgroup of 16 waves per two consecutive tiles of the sequence,
        // one per K group.  Same process, one-group -> pairs (us, measured
        // with a token-major tile sequence): 1024 tiles
        // at K = 4096 240-245 -> 226-232, at K = 11008 645-647 -> 607-612 and
        // 334-338 -> 300-302, at K = 5632 299-317 -> 290-323; one round (512
        // tiles) even, and 5.5 rounds (2816 tiles, K = 4096) 658 -> 686-690,
        // where two workgroups per CU even out the last half round better;
        // at K = 2048 no gain.  The same sums in the same order as the
        // one-group form.
        if (K >= 4096u && t4 >= 4ull * cus && t4 % (2ull * cus) == 0) {
            set_variant(variant, kname, "FB4.pairs", 16, 128, 0, (int)kBN, (uint32_t)((t4 / 2u + 7u) / 8u * 8u));
            return launch_fb<4, 8, 64, 2, 2, false, true>(a, p, n, N, K, stream, nullptr, (uint32_t)t4, 1u);
        }
        // Otherwise the 128-row tiles on the direct kernel, two workgroups per
        // CU.  Same process, us, against the one-group form through LDS: 768
        // tokens q, k, v 86.1 -> 82.9, 1024 tokens 94.8 -> 92.4, 512 x 11008 x
        // 4096 166.6 -> 161.7.
        set_variant(variant, kname, "D128", 8, 128, 0, (int)kBN, (uint32_t)((t4 + 7u) / 8u * 8u));
        return launch_direct<1, 2>(a, p, n, N, K, stream);
    }
    // With a workspace, 256-row tiles on the direct kernel with every tile's
    // K steps split into 4 or 8 parts, one workgroup each, when that fills
    // more than 7/8 of the CUs with at least 11 steps per part (the parts
    // meet in split_sum_kernel).  Same box, us, against the two-K-group forms
    // the dispatch took before: 512 tokens down 50.0 -> 47.1 (4 parts of 22
    // steps), 256 tokens down 31.6 -> 30.2 (8 parts of 11); with 8 or 4 steps
    // per part the split's second launch costs more than it saves (o, K =
    // 2048: 24.6 -> 26.2 at 512 tokens, 19.6 -> 20.6 at 256).
    for (uint32_t xs : {4u, 8u}) {
        const size_t blk = (size_t)256u * kBN * 4u;
        if (workspace && t8 * xs <= cus && 8u * t8 * xs > 7u * cus && steps >= 11u * xs &&
            (xs - 1u) * t8 * blk <= workspace_bytes) {
            set_variant(variant, kname, xs == 4u ? "D256.split4" : "D256.split8", 8, 256, 0, (int)kBN,
                        (uint32_t)(t8 * xs));
            return launch_direct<2, 2, true>(a, p, n, N, K, stream, workspace, xs);
        }
    }
    // 128-row tiles that fill most of the CUs, one per CU with two K groups,
    // beat smaller tiles that fill them all: a 128-row tile moves ~19 bytes
    // through LDS per output and step against ~27 for 64 rows and ~45 for
    // 32.  Same process, µs: 128 tokens gate and up (176 tiles) 38.6 -> 32.0,
    // 256 tokens q, k, v (192 tiles) 38.9 -> 33.2; with 128 tiles (half the
    // CUs) they lose (512 tokens o: 29.6 -> 31.4, one box and process).
    if (5u * t4 >= 3u * cus) {
        set_variant(variant, kname, "FB4.ksplit2", 16, 128, 0, (int)kBN, (uint32_t)((t4 + 7u) / 8u * 8u));
        return launch_fb<4, 8, 64, 2, 2>(a, p, n, N, K, stream);
    }
    // With a workspace, 128-row tiles whose K steps split in 2 or 4 fill
    // (nearly) every CU, as long as each K group keeps at least 10 steps
    // (the split's second launch and every part's pipeline start cost a few
    // us): 512 tokens down 55.8 -> 49.9 us (2 parts, 22 steps per group), 256
    // tokens down 40.2 -> 31.1 (4 parts, 11 steps).  Fewer workgroups than
    // 7/8 of the CUs, or shorter runs, lose to the smaller tiles below (512
    // tokens o in 2 parts of 8 steps per group: 21.9 -> 26.0; 128 tokens q, k,
    // v in 2 parts on 3/4 of the CUs: 21.8 -> 23.9).
    for (uint32_t xs : {4u, 2u}) {
        const size_t blk = (size_t)128u * kBN * 4u;
        if (workspace && t4 * xs <= cus && 8u * t4 * xs > 7u * cus && steps >= 20u * xs &&
            (xs - 1u) * t4 * blk <= workspace_bytes) {
            set_variant(variant, kname, xs == 4u ? "FB4.ksplit2.wgsplit4" : "FB4.ksplit2.wgsplit2", 16, 128, 0, (int)kBN,
                        (uint32_t)(t4 * xs));
            return launch_fb<4, 8, 64, 2, 2, true>(a, p, n, N, K, stream, workspace, (uint32_t)t4, xs);
        }
    }
    if (t1 <= cus) {
        // With a workspace, tiles that fill at most a quarter (a half) of the
        // CUs also split their K steps between 4 (2) workgroups, each run at
        // least 4 steps per K group; the parts' sums meet in a second launch.
        const size_t blk = (size_t)32u * kBN * 4u;
        if (workspace && 4u * t1 <= cus && steps >= 32u && 3u * t1 * blk <= workspace_bytes) {
            set_variant(variant, kname, "FB1.PD4.ksplit2.wgsplit4", 16, 32, 0, (int)kBN, (uint32_t)(4u * t1));
            return launch_fb<1, 8, 64, 4, 2, true>(a, p, n, N, K, stream, workspace, (uint32_t)t1, 4u);
        }
        if (workspace && 2u * t1 <= cus && steps >= 16u && t1 * blk <= workspace_bytes) {
            set_variant(variant, kname, "FB1.PD4.ksplit2.wgsplit2", 16, 32, 0, (int)kBN, (uint32_t)(2u * t1));
            return launch_fb<1, 8, 64, 4, 2, true>(a, p, n, N, K, stream, workspace, (uint32_t)t1, 2u);
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
