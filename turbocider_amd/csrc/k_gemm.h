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
    int act;               // output activation (kAct*, tc_kernels.h): picks the unsplit variant
};

// The second problem of a grouped launch (gemmg_* variants): another activation, weight and
// output with the first problem's type, K, activation row stride and row-block count. Its
// output tiles follow the first problem's in the work list (and in the split-K partials).
struct GemmSecond {
    const uint16_t *x;
    int M;
    const uint8_t *w;
    int N;
    uint16_t *y;
    int64_t y_stride;
    const uint16_t *bias;
    int tiles_m, tiles_n;
};

// One entry point per compiled variant: gemm_<type>_<split>_<mt>_<act>. The output
// activation (kAct*, tc_kernels.h) is a template parameter of the unsplit kernels, so that
// the variant without one compiles exactly as before it existed; split variants leave it to
// the slice reduction (act 0 only).
#define TC_GEMM_VARIANT_NAME(T, S, MT, A) gemm_##T##_##S##_##MT##_##A
#define TC_GEMM_DECLARE(T, S, MT, A) hipError_t TC_GEMM_VARIANT_NAME(T, S, MT, A)(const GemmArgs &a, hipStream_t stream);
#define TC_GEMM_DECLARE_MT(T, MT)  \
    TC_GEMM_DECLARE(T, 0, MT, 0)   \
    TC_GEMM_DECLARE(T, 0, MT, 1)   \
    TC_GEMM_DECLARE(T, 0, MT, 2)   \
    TC_GEMM_DECLARE(T, 1, MT, 0)
TC_GEMM_DECLARE_MT(12, 8)
TC_GEMM_DECLARE_MT(12, 4)
TC_GEMM_DECLARE_MT(12, 2)
TC_GEMM_DECLARE_MT(12, 1)
TC_GEMM_DECLARE_MT(13, 8)
TC_GEMM_DECLARE_MT(13, 4)
TC_GEMM_DECLARE_MT(13, 2)
TC_GEMM_DECLARE_MT(13, 1)
TC_GEMM_DECLARE_MT(14, 8)
TC_GEMM_DECLARE_MT(14, 4)
TC_GEMM_DECLARE_MT(14, 2)
TC_GEMM_DECLARE_MT(14, 1)
// kActNoneKeep (cached output stores): unsplit 128- and 256-row tiles only.
TC_GEMM_DECLARE(12, 0, 8, 3) TC_GEMM_DECLARE(12, 0, 4, 3)
TC_GEMM_DECLARE(13, 0, 8, 3) TC_GEMM_DECLARE(13, 0, 4, 3)
TC_GEMM_DECLARE(14, 0, 8, 3) TC_GEMM_DECLARE(14, 0, 4, 3)
#undef TC_GEMM_DECLARE_MT
#undef TC_GEMM_DECLARE

// Grouped variants (two problems, no output activation): gemmg_<type>_<split>_<mt>.
#define TC_GEMMG_VARIANT_NAME(T, S, MT) gemmg_##T##_##S##_##MT
#define TC_GEMMG_DECLARE(T, S, MT) \
    hipError_t TC_GEMMG_VARIANT_NAME(T, S, MT)(const GemmArgs &a, const GemmSecond &b, hipStream_t stream);
#define TC_GEMMG_DECLARE_T(T) TC_GEMMG_DECLARE(T, 0, 4) TC_GEMMG_DECLARE(T, 1, 4) TC_GEMMG_DECLARE(T, 0, 8) TC_GEMMG_DECLARE(T, 1, 8)
TC_GEMMG_DECLARE_T(12)
TC_GEMMG_DECLARE_T(13)
TC_GEMMG_DECLARE_T(14)
#undef TC_GEMMG_DECLARE_T
#undef TC_GEMMG_DECLARE

}  // namespace tc
