// One instantiation of the dequant-GEMM kernel (k_gemm_impl.h). The build compiles this file
// once per (TYPE, SPLIT, MT, ACT) with -DTC_GEMM_TYPE=12|13|14 -DTC_GEMM_SPLIT=0|1
// -DTC_GEMM_MT=1|2|4|8 -DTC_GEMM_ACT=0|1|2 (ACT 0 only for SPLIT 1; ACT 3, kActNoneKeep, for
// SPLIT 0 at MT 4 and 8), and once per grouped
// (TYPE, SPLIT, MT) with -DTC_GEMM_GROUP=1 -DTC_GEMM_MT=4|8 -DTC_GEMM_ACT=0, so that the
// variants compile in parallel; without those definitions it is empty.
#if defined(TC_GEMM_TYPE) && defined(TC_GEMM_SPLIT) && defined(TC_GEMM_MT) && defined(TC_GEMM_ACT)
#include "k_gemm_impl.h"

namespace tc {
#if defined(TC_GEMM_GROUP) && TC_GEMM_GROUP
#define TC_GEMM_DEFINE(T, S, MT, A)                                                                               \
    hipError_t TC_GEMMG_VARIANT_NAME(T, S, MT)(const GemmArgs &a, const GemmSecond &b, hipStream_t stream) { \
        return gemm_variant<T, S != 0, MT, A, true>(a, stream, b);                                               \
    }
#else
#define TC_GEMM_DEFINE(T, S, MT, A)                                                         \
    hipError_t TC_GEMM_VARIANT_NAME(T, S, MT, A)(const GemmArgs &a, hipStream_t stream) { \
        return gemm_variant<T, S != 0, MT, A>(a, stream);                                  \
    }
#endif
#define TC_GEMM_DEFINE_EXPANDED(T, S, MT, A) TC_GEMM_DEFINE(T, S, MT, A)
TC_GEMM_DEFINE_EXPANDED(TC_GEMM_TYPE, TC_GEMM_SPLIT, TC_GEMM_MT, TC_GEMM_ACT)
}  // namespace tc
#endif
