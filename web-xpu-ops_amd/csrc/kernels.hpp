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
};

// `variant` (optional) receives a static string naming the kernel chosen.
hipError_t launch_matvec_q8(const MatvecArgs& a, const DeviceInfo& dev, hipStream_t stream,
                            const char** variant);
hipError_t launch_fill_scaled_zero(const float* scale, float* y, uint32_t N, uint32_t M, hipStream_t stream);

// quantize (codes != nullptr) and/or packQ8 (packed != nullptr) of f32 rows.
hipError_t launch_quantize_rows(const float* input, uint32_t N, uint32_t K, int32_t* codes, uint32_t* packed,
                                float* scales, const DeviceInfo& dev, hipStream_t stream, const char** variant);
hipError_t launch_pack_q8(const int32_t* codes, uint32_t N, uint32_t K, uint32_t* packed, const DeviceInfo& dev,
                          hipStream_t stream);
hipError_t launch_pack_int8_rows(const int8_t* codes, uint32_t N, uint32_t K, uint32_t* packed,
                                 const DeviceInfo& dev, hipStream_t stream);

}  // namespace wxo
