// wave_ops.hpp -- wave64 building blocks for gfx950 (CDNA4).
//
// Cross-lane traffic uses DPP (quad_perm, row_mirror, row_half_mirror) inside
// each 16-lane row and gfx950's v_permlane16_swap / v_permlane32_swap across
// rows, so no reduction touches LDS or needs a barrier.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wxo {

constexpr int kWave = 64;

// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8 lanes
constexpr int kDppRowMirror = 0x140;  // lane i <-> 15-i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Value of the partner lane whose bit D differs (D in 1,2,4,8).  For D=4 and
// D=8 the partner is the mirror lane, which also differs in the lower bits;
// every reduction below only needs "an involution that flips bit D and keeps
// the bits above it", which both mirrors are.
template <int D>
__device__ __forceinline__ float partner_f32(float v) {
    if constexpr (D == 1) return dpp_f32<kDppQuadXor1>(v);
    else if constexpr (D == 2) return dpp_f32<kDppQuadXor2>(v);
    else if constexpr (D == 4) return dpp_f32<kDppHalfMirror>(v);
    else return dpp_f32<kDppRowMirror>(v);
}

template <int D>
__device__ __forceinline__ uint32_t partner_u32(uint32_t v) {
    if constexpr (D == 1) return dpp_u32<kDppQuadXor1>(v);
    else if constexpr (D == 2) return dpp_u32<kDppQuadXor2>(v);
    else if constexpr (D == 4) return dpp_u32<kDppHalfMirror>(v);
    else return dpp_u32<kDppRowMirror>(v);
}

// v_permlane32_swap: lanes 32..63 of `lo` trade places with lanes 0..31 of
// `hi`.  Afterwards lo' + hi' holds, in lanes 0..31, lo[l] + lo[l+32] and, in
// lanes 32..63, hi[l-32] + hi[l].  v_permlane16_swap does the same between odd
// rows of `lo` and even rows of `hi`.
template <int D>
__device__ __forceinline__ float swap_add(float lo, float hi) {
    static_assert(D == 16 || D == 32, "permlane swap distance");
    if constexpr (D == 32) {
        auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

// One step of a multi-row wave reduction at lane distance D: N values per lane
// become N/2 (lanes with bit D clear keep rows [0, N/2), lanes with it set keep
// rows [N/2, N)); with N == 1 it is a plain butterfly.
template <int D, int N, int R>
__device__ __forceinline__ void reduce_step(float (&a)[R], int lane) {
    if constexpr (N == 1) {
        if constexpr (D >= 16) a[0] = swap_add<D>(a[0], a[0]);
        else a[0] = a[0] + partner_f32<D>(a[0]);
    } else {
        const bool up = (lane & D) != 0;
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const float lo = a[i], hi = a[i + N / 2];
            if constexpr (D >= 16) {
                a[i] = swap_add<D>(lo, hi);
            } else {
                const float keep = up ? hi : lo;
                const float send = up ? lo : hi;
                a[i] = keep + partner_f32<D>(send);
            }
        }
    }
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

// Sums R per-lane partial values across the 64 lanes of a wave with about
// R + 6 cross-lane operations instead of 6R.  On return a[0] of lane l holds
// the full sum of row (l >> (6 - log2 R)); every lane of that group agrees.
template <int R>
__device__ __forceinline__ void wave_reduce_rows(float (&a)[R], int lane) {
    static_assert(R >= 1 && R <= 64 && (R & (R - 1)) == 0, "R must be a power of two <= 64");
    reduce_step<32, (R >= 1 ? R : 1), R>(a, lane);
    reduce_step<16, (R >= 2 ? R / 2 : 1), R>(a, lane);
    reduce_step<8, (R >= 4 ? R / 4 : 1), R>(a, lane);
    reduce_step<4, (R >= 8 ? R / 8 : 1), R>(a, lane);
    reduce_step<2, (R >= 16 ? R / 16 : 1), R>(a, lane);
    reduce_step<1, (R >= 32 ? R / 32 : 1), R>(a, lane);
}

// Wave-wide max of unsigned values (every lane receives the result).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, partner_u32<1>(v));
    v = max(v, partner_u32<2>(v));
    v = max(v, partner_u32<4>(v));
    v = max(v, partner_u32<8>(v));
    {
        auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = max(r[0], r[1]);
    }
    {
        auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = max(r[0], r[1]);
    }
    return v;
}

// Loads of 4 consecutive 32-bit words from an address that is only 4-byte
// aligned (ragged rows: row stride ceil(K/4) words).  gfx950 global loads
// accept dword-aligned dwordx4; the aligned(4) vector type tells the compiler
// exactly that, so it still emits one global_load_dwordx4.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef int32_t i32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ u32x4_a4 load_u32x4(const uint32_t* p) {
    return *reinterpret_cast<const u32x4_a4*>(p);
}
__device__ __forceinline__ f32x4_a4 load_f32x4(const float* p) {
    return *reinterpret_cast<const f32x4_a4*>(p);
}

// Raw buffer resource over [base, base + bytes) (gfx9 word 3: 32-bit untyped).
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCachePolicyNT = 2;  // "nt": streamed once, low L2 retention

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferWord3);
}

// buffer_load_dwordx4 at byte offset voffset (VGPR) + soffset (SGPR), non-temporal.
__device__ __forceinline__ u32x4v load_nt_b128(__amdgpu_buffer_rsrc_t rs, int voffset, int soffset) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, voffset, soffset, kCachePolicyNT);
}

}  // namespace wxo
