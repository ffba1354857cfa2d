// Runtime (unmerged) LoRA and bias epilogue kernels.
//
// Numerics follow the reference's runtime-LoRA sequence (native/backends/mlx.cpp:692-722,
// 957-984; tests/native/native_lora_math_test.cpp:69-107):
//   low   = f32(x) * f32(A)^T                       fp32, never narrowed before B
//   delta = f32(low * f32(B)^T)                     fp32
//   y     = bf16(f32(y) + f32(scale * delta))       one bf16 rounding per adapter
// and the bias last: y = bf16(f32(y) + f32(bias)) (mlx.cpp:687-688).
//
// Both products run on bf16 MFMA with fp32 accumulation:
//   * x and A are bf16, so every product x*A is exact in fp32;
//   * low (fp32) is split exactly into three bf16 terms low = hi + mid + lo
//     (hi = RNE(low), mid = RNE(low - hi), lo = RNE(low - hi - mid); each difference is
//     exact and three 8-bit significands cover fp32's 24), so low*B is formed from exact
//     products too, unlike the reference's opt-in Metal epilogue which narrows low to bf16
//     (native/backends/dense_gpu_lora_b.hpp:49).
#include "tc_device.h"
#include "tc_kernels.h"

namespace tc {
namespace {

// low[rows, rank]: one workgroup per 32x32 output tile, its 4 wavefronts split K and reduce
// through LDS. Lane (l32, h) feeds row l32 / K-slots 8h..8h+7 of each 16-wide K step.
__global__ __launch_bounds__(256) void k_lora_low(const uint16_t *__restrict__ x, int64_t x_stride, int rows, int K,
                                                  const uint16_t *__restrict__ a, int rank, float *__restrict__ low,
                                                  int low_stride) {
    __shared__ float part[4][32][33];
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    const int r0 = (int)blockIdx.x * 32, c0 = (int)blockIdx.y * 32;
    const uint16_t *xr = x + (int64_t)min(r0 + l32, rows - 1) * x_stride;
    const uint16_t *ar = a + (int64_t)min(c0 + l32, rank - 1) * K;
    f32x16 acc = {};
    const int steps = K / 16;
    for (int s = wave; s < steps; s += 4) {
        const bf16x8 av = *reinterpret_cast<const bf16x8 *>(xr + 16 * s + 8 * h);
        const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(ar + 16 * s + 8 * h);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) part[wave][8 * (j >> 2) + 4 * h + (j & 3)][l32] = acc[j];
    __syncthreads();
    for (int o = (int)threadIdx.x; o < 32 * 32; o += 256) {
        const int r = o >> 5, c = o & 31;
        if (r0 + r < rows && c0 + c < rank)
            low[(int64_t)(r0 + r) * low_stride + c0 + c] = part[0][r][c] + part[1][r][c] + part[2][r][c] + part[3][r][c];
    }
}

// y[r, j] for r < rows, j < n (already offset to the adapter's first row / output column).
// One workgroup per 32 rows x 128 columns (wavefront w: columns 32w..32w+31).
// `low` rows are low_stride (a multiple of 8) floats apart; `vec_b` says that B's rows
// are 16-byte aligned (rank % 8 == 0 and an aligned base), enabling 16-byte loads of B.
__global__ __launch_bounds__(256) void k_lora_apply(const float *__restrict__ low, int low_stride, int rank,
                                                    const uint16_t *__restrict__ b, bool vec_b, float scale,
                                                    uint16_t *__restrict__ y, int64_t y_stride, int rows, int n) {
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    const int r0 = (int)blockIdx.x * 32, c0 = (int)blockIdx.y * 128 + 32 * wave;
    const float *lr = low + (int64_t)min(r0 + l32, rows - 1) * low_stride;
    const uint16_t *br = b + (int64_t)min(c0 + l32, n - 1) * rank;
    f32x16 acc = {};
    for (int k0 = 0; k0 < rank; k0 += 16) {
        const int kb = k0 + 8 * h;
        float lv[8];
        uint32_t bw[4];
        if (vec_b && kb + 8 <= rank) {
            const f32x4 l0 = *reinterpret_cast<const f32x4 *>(lr + kb), l1 = *reinterpret_cast<const f32x4 *>(lr + kb + 4);
            lv[0] = l0.x; lv[1] = l0.y; lv[2] = l0.z; lv[3] = l0.w; lv[4] = l1.x; lv[5] = l1.y; lv[6] = l1.z; lv[7] = l1.w;
            const u32x4 bv = *reinterpret_cast<const u32x4 *>(br + kb);
            bw[0] = bv.x; bw[1] = bv.y; bw[2] = bv.z; bw[3] = bv.w;
        } else {
            uint16_t bh[8];
            for (int i = 0; i < 8; ++i) {
                lv[i] = kb + i < rank ? lr[kb + i] : 0.f;
                bh[i] = kb + i < rank ? br[kb + i] : (uint16_t)0;
            }
            for (int i = 0; i < 4; ++i) bw[i] = (uint32_t)bh[2 * i] | ((uint32_t)bh[2 * i + 1] << 16);
        }
        uint32_t hi[4], mid[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t hp = 0, mp = 0, lp = 0;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float v = lv[2 * i + e];
                const uint32_t hb = float_to_bf16_bits(v);
                const float r1 = v - bf16_to_float(hb);
                const uint32_t mb = float_to_bf16_bits(r1);
                const float r2 = r1 - bf16_to_float(mb);
                const uint32_t lb = float_to_bf16_bits(r2);
                hp |= hb << (16 * e);
                mp |= mb << (16 * e);
                lp |= lb << (16 * e);
            }
            hi[i] = hp; mid[i] = mp; lo[i] = lp;
        }
        const bf16x8 bv = __builtin_bit_cast(bf16x8, u32x4{bw[0], bw[1], bw[2], bw[3]});
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{hi[0], hi[1], hi[2], hi[3]}),
                                                     bv, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8, u32x4{mid[0], mid[1], mid[2], mid[3]}), bv, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], lo[2], lo[3]}),
                                                     bv, acc, 0, 0, 0);
    }
    const int c = c0 + l32;
    if (c >= n) return;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int r = r0 + 8 * (j >> 2) + 4 * h + (j & 3);
        if (r < rows) {
            uint16_t *p = y + (int64_t)r * y_stride + c;
            const float t = __fmul_rn(scale, acc[j]);
            *p = (uint16_t)float_to_bf16_bits(__fadd_rn(bf16_to_float(*p), t));
        }
    }
}

__global__ __launch_bounds__(256) void k_bias_add(uint16_t *__restrict__ y, int64_t y_stride, int M, int N,
                                                  const uint16_t *__restrict__ bias) {
    const int n = (int)(blockIdx.x * 256 + threadIdx.x), m = (int)blockIdx.y;
    if (n >= N || m >= M) return;
    uint16_t *p = y + (int64_t)m * y_stride + n;
    *p = (uint16_t)float_to_bf16_bits(bf16_to_float(*p) + bf16_to_float(bias[n]));
}

}  // namespace

hipError_t launch_lora_low(const uint16_t *x, int64_t x_stride, int rows, int K, const uint16_t *a, int rank,
                           float *low, int low_stride, hipStream_t stream) {
    hipLaunchKernelGGL(k_lora_low, dim3((unsigned)((rows + 31) / 32), (unsigned)((rank + 31) / 32)), dim3(256), 0,
                       stream, x, x_stride, rows, K, a, rank, low, low_stride);
    return hipGetLastError();
}

hipError_t launch_lora_apply(const float *low, int low_stride, int rank, const uint16_t *b, float scale, uint16_t *y,
                             int64_t y_stride, int rows, int n_begin, int n_count, hipStream_t stream) {
    const bool vec_b = rank % 8 == 0 && (reinterpret_cast<uintptr_t>(b) & 15u) == 0;
    hipLaunchKernelGGL(k_lora_apply, dim3((unsigned)((rows + 31) / 32), (unsigned)((n_count + 127) / 128)), dim3(256),
                       0, stream, low, low_stride, rank, b, vec_b, scale, y + n_begin, y_stride, rows, n_count);
    return hipGetLastError();
}

hipError_t launch_bias_add(uint16_t *y, int64_t y_stride, int M, int N, const uint16_t *bias_bf16,
                           hipStream_t stream) {
    hipLaunchKernelGGL(k_bias_add, dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256), 0, stream, y, y_stride,
                       M, N, bias_bf16);
    return hipGetLastError();
}

}  // namespace tc
