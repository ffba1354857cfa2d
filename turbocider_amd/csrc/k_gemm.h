// Launch arguments shared by the GEMM dispatcher (k_gemm.hip) and the per-variant kernel
// translation units (k_gemm_variant.hip, one object per (TYPE, SPLIT, MT)).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tc {

struct GemmArgs {
    const uint16_t *x;
    int64_t x_stride;
    int M;
    const uint8_t *w;
    int64_t w_pitch;
    int N, K;
    uint16_t *y;
    int64_t y_stride;
    const uint16_t *bias;  // bf16 [N] or null
    int tiles_m, tiles_n, splits;
    float *partials;       // SPLIT: raw fp32 accumulators of every (slice, tile)
    int grid;              // persistent workgroups
};

// One entry point per compiled variant: gemm_<type>_<split>_<mt>.
#define TC_GEMM_VARIANT_NAME(T, S, MT) gemm_##T##_##S##_##MT
#define TC_GEMM_DECLARE(T, S, MT) hipError_t TC_GEMM_VARIANT_NAME(T, S, MT)(const GemmArgs &a, hipStream_t stream);
TC_GEMM_DECLARE(12, 0, 8)
TC_GEMM_DECLARE(12, 1, 8)
TC_GEMM_DECLARE(12, 0, 4)
TC_GEMM_DECLARE(12, 1, 4)
TC_GEMM_DECLARE(12, 0, 2)
TC_GEMM_DECLARE(12, 1, 2)
TC_GEMM_DECLARE(12, 0, 1)
TC_GEMM_DECLARE(12, 1, 1)
TC_GEMM_DECLARE(14, 0, 8)
TC_GEMM_DECLARE(14, 1, 8)
TC_GEMM_DECLARE(14, 0, 4)
TC_GEMM_DECLARE(14, 1, 4)
TC_GEMM_DECLARE(14, 0, 2)
TC_GEMM_DECLARE(14, 1, 2)
TC_GEMM_DECLARE(14, 0, 1)
TC_GEMM_DECLARE(14, 1, 1)
#undef TC_GEMM_DECLARE

}  // namespace tc
