// Output activation as a pass of its own over finished projection outputs, for the routes
// whose epilogue does not apply it (runtime LoRA, the library GEMM, the forced per-row GEMV):
// y = act(pre) with the epilogues' formulas (gelu_tanh_bits / silu_glu_bits, tc_device.h), so
// a projection gives the same bits whichever route ran it, up to the route's own summation
// order. Replaces the reference's separate activation ops after the projection
// (native/models/qwen21/transformer.cpp:48-57, 973-975; native/backends/mlx.cpp:1627-1631).
#include "tc_device.h"
#include "tc_kernels.h"

namespace tc {
namespace {

// One thread per four consecutive columns of a row of pre (kActSiluGlu: two outputs).
__global__ __launch_bounds__(256) void k_act(const uint16_t *pre, int64_t pre_stride, int M, int N, uint16_t *y,
                                             int64_t y_stride, int act) {
    const int quads = (N + 3) / 4;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t)M * quads) return;
    const int m = (int)(t / quads), col = 4 * (int)(t % quads);
    const uint16_t *p = pre + (int64_t)m * pre_stride + col;
    uint32_t v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = col + c < N ? p[c] : 0u;
    store_out4(y + (int64_t)m * y_stride, col, N, v, false, act);
}

}  // namespace

hipError_t launch_act(const uint16_t *pre, int64_t pre_stride, int M, int N, uint16_t *y, int64_t y_stride, int act,
                      hipStream_t stream) {
    if (act == kActNone || M < 1 || N < 1) return hipSuccess;
    if (act == kActSiluGlu && (N & 1)) return hipErrorInvalidValue;
    const int64_t threads = (int64_t)M * ((N + 3) / 4);
    hipLaunchKernelGGL(k_act, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, pre, pre_stride, M, N, y,
                       y_stride, act);
    return hipGetLastError();
}

}  // namespace tc
