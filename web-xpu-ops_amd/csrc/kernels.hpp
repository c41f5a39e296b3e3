// kernels.hpp -- internal launch interface between the C ABI (wxo_api.hip)
// and the gfx950 kernels.  Not part of the public ABI (include/wxo_q8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace wxo {

struct DeviceInfo {
    int ordinal = -1;
    int cu_count = 0;
    size_t hbm_bytes = 0;
    char name[128] = {0};
    char arch[64] = {0};
};

struct MatvecArgs {
    const uint32_t* weight;
    const float* scale;
    const float* vector;
    float* output;
    uint32_t N, K, M;
    uint32_t W;  // ceil(K / 4) words per row
    // fused forms (M = 1): the up projection of matvecQ8Ffn, the residual of
    // matvecQ8Residual
    const uint32_t* weight2 = nullptr;
    const float* scale2 = nullptr;
    const float* residual = nullptr;
};

// Kernel arguments of the single-vector kernel (all epilogues).
struct M1Params {
    const uint32_t* weight;  // gate for the FFN form
    const float* scale;
    const uint32_t* weight2;  // up (FFN only)
    const float* scale2;
    const float* x;
    const float* residual;  // residual form only
    float* y;
    uint32_t N, K, W;
};

enum : int { kEpiPlain = 0, kEpiResidual = 1, kEpiFfn = 2 };

// The kernel instance a launcher chose, for callers that report it
// (wxo_last_variant): the kernel template, the form selected within it and
// the parameters that pick the instance.  Fields a kernel has no use for
// stay 0.
struct Variant {
    const char* kernel = "";  // kernel template name
    const char* form = "";    // selected form within it
    int waves = 0;            // waves per workgroup
    int rows = 0;             // rows (or weight-tile rows) per workgroup
    int slots = 0;            // per-lane unit count: chunk slots whose vector slices stay in
                              // VGPRs (matvec; 0 = streamed), packed words per lane (quantize)
    int vectors = 0;          // vectors per pass (batched forms)
    uint32_t grid_x = 0, grid_y = 0;
};

inline void set_variant(Variant* v, const char* kernel, const char* form, int waves, int rows, int slots,
                        int vectors, uint32_t grid_x, uint32_t grid_y = 1) {
    if (v) *v = Variant{kernel, form, waves, rows, slots, vectors, grid_x, grid_y};
}

// `variant` (optional) receives the kernel instance chosen.
hipError_t launch_matvec_q8(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream,
                            Variant* variant);
// matvecQ8Residual (epi = kEpiResidual) or matvecQ8Ffn (kEpiFfn), M = 1.
hipError_t launch_matvec_q8_fused(const MatvecArgs& a, int epi, const DeviceInfo& dev, hipStream_t stream,
                                  Variant* variant);
// Several single-vector projections of one vector x [K]: output_p =
// matvecQ8(weight_p, scale_p, x, N_p, K), count <= kMaxProjections, in one
// launch.  Outputs must be disjoint from each other and from x.
constexpr uint32_t kMaxProjections = 4;
struct Projection {
    const uint32_t* weight;
    const float* scale;
    float* output;
    uint32_t N;
};
hipError_t launch_matvec_q8_multi(const Projection* projections, uint32_t count, const float* x, uint32_t K,
                                  const DeviceInfo& dev, hipStream_t stream, Variant* variant);
hipError_t launch_fused_zero(const MatvecArgs& a, int epi, hipStream_t stream);
hipError_t launch_fill_scaled_zero(const float* scale, float* y, uint32_t N, uint32_t M, hipStream_t stream);

// quantize (codes != nullptr) and/or packQ8 (packed != nullptr) of f32 rows.
hipError_t launch_quantize_rows(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed,
                                float* scales, const DeviceInfo& dev, hipStream_t stream, Variant* variant);
// quantize + packQ8 of several matrices with the same K (count <= 8), one
// launch for rows of more than 128 words.
constexpr uint32_t kMaxQuantizeMatrices = 8;
hipError_t launch_quantize_pack_multi(const float* const* inputs, const uint32_t* Ns, uint32_t* const* packed,
                                      float* const* scales, uint32_t count, uint32_t K, const DeviceInfo& dev,
                                      hipStream_t stream);
hipError_t launch_pack_q8(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed, const DeviceInfo& dev,
                          hipStream_t stream);
hipError_t launch_pack_int8_rows(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed,
                                 const DeviceInfo& dev, hipStream_t stream);

// matmulQ8 (matmul_q8.hip): a f32 [N, K] x packed weight [M, ceil(K/4)] ->
// out f32 [N, M].  K <= 2^22.
hipError_t launch_matmul_q8(const float* a, const uint32_t* weight, const float* scale, float* out, uint32_t N,
                            uint32_t M, uint32_t K, const DeviceInfo& dev, hipStream_t stream, Variant* variant);
// Several projections of the same activations a [N, K]: output_p [N, M_p] =
// matmulQ8(a, weight_p, scale_p), count <= kMaxMatmulProjectionsPerLaunch in
// one launch.  Outputs must be disjoint from each other and from a.  With a
// workspace (device memory, disjoint from everything else), some tiles split
// their K steps between workgroups (all of a short prompt's; the last ones of
// a prompt whose tiles fill one round unevenly) and a second launch adds them;
// the workspace holds one tile of floats per extra part, at most
// kMatmulWorkspaceBytesPerCu per CU.
constexpr uint32_t kMaxMatmulProjectionsPerLaunch = 4;
struct MatmulProjection {
    const uint32_t* weight;
    const float* scale;
    float* output;
    uint32_t M;
};
// Room for every split the dispatch takes: up to 7/8 of a round of 256 x 64
// f32 tiles per CU (a short prompt's 256-row tiles in 4 or 8 parts).
constexpr size_t kMatmulWorkspaceBytesPerCu = 65536;
hipError_t launch_matmul_q8_multi(const float* a, const MatmulProjection* projections, uint32_t count, uint32_t N,
                                  uint32_t K, const DeviceInfo& dev, hipStream_t stream, Variant* variant,
                                  float* workspace = nullptr, size_t workspace_bytes = 0);

// dequant_q8.hip
hipError_t launch_dequantize_packed(const uint32_t* weight, const float* scale, uint32_t N, uint32_t K,
                                    float* out, const DeviceInfo& dev, hipStream_t stream);
hipError_t launch_dequant_transpose(const uint32_t* weight, const float* scale, uint32_t out_features,
                                    uint32_t in_features, float* out, hipStream_t stream);
hipError_t launch_gather_dequant_rows(const int8_t* codes, const float* scale, uint32_t rows, uint32_t D,
                                      const int64_t* indices, uint32_t count, float* out, const DeviceInfo& dev,
                                      hipStream_t stream);

// roofline.hip: this device's best sustained HBM read bandwidth (bytes/s) and
// one-wide f32 FMA rate (flop/s), measured now; either output may be null to
// skip that part.  Allocates (and frees) two 512 MiB buffers on its own stream.
hipError_t measure_roofline(const DeviceInfo& dev, double* bandwidth, double* compute);
// The sustained bf16 matrix-core rate (flop/s) on every CU, two waves per SIMD,
// operands like the prefill GEMM's.
hipError_t measure_matrix_ceiling(const DeviceInfo& dev, double* flops);

}  // namespace wxo
