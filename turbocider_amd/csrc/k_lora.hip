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
//
// Two launches per forward call, whatever the adapter count (up to kLoraBatch per batch):
//   * k_lora_low: low of every adapter (grid z = adapter), K staged through LDS and split
//     over workgroups (partial planes added in slice order by k_lora_low_reduce);
//   * k_lora_epilogue: one read-modify-write pass over y that applies the adapters in their
//     order (each to its own rows and output columns) and then the bias, so y makes a
//     single round trip through HBM however many adapters are bound.
#include "tc_device.h"
#include "tc_kernels.h"

#include <algorithm>

namespace tc {
namespace {

// low[rows, rank] of adapter blockIdx.z, one workgroup (4 wavefronts) per 32-row x 64-rank
// tile and K slice (blockIdx.y = rank tile * ksplit + slice; slice s writes partial plane s
// of the adapter's workspace, which the epilogue sums in slice order). K is walked in
// 128-wide chunks staged through LDS: the workgroup reads a chunk's 32 x rows and 64 A rows
// with 16-byte loads on consecutive addresses (each row's 256 bytes by 16 consecutive
// lanes), one chunk ahead in registers, double-buffered in LDS; wavefront w takes K steps
// 2w, 2w + 1 of every chunk (two 32x32x16 MFMAs per step, both rank halves), and the four
// partial tiles are added through LDS in wavefront order.
constexpr int kLowKC = 128;                   // K per chunk
constexpr int kLowPitch = kLowKC * 2 + 16;    // LDS row pitch (bytes): rows 4 banks apart
constexpr int kLowXBytes = 32 * kLowPitch, kLowABytes = 64 * kLowPitch;

__global__ __launch_bounds__(256) void k_lora_low(const uint16_t *__restrict__ x, int64_t x_stride, int K,
                                                  LoraBatch batch) {
    __shared__ __attribute__((aligned(16))) uint8_t stage[2][kLowXBytes + kLowABytes];
    const LoraDesc &D = batch.d[blockIdx.z];
    const int ks = D.ksplit, slice = (int)blockIdx.y % ks;
    const int r0 = (int)blockIdx.x * 32, c0 = (int)blockIdx.y / ks * 64;
    if (r0 >= D.row_count || c0 >= D.rank) return;  // uniform: this adapter is smaller than the grid
    const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    // Loader geometry: piece e = 256 j + tid is row e / 16, 16-byte piece e % 16 of the chunk.
    const int piece = tid & 15, prow = tid >> 4;  // rows prow + 16 j
    const uint16_t *xsrc[2];
    const uint16_t *asrc[4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
        xsrc[j] = x + (int64_t)(D.row_begin + min(r0 + prow + 16 * j, D.row_count - 1)) * x_stride + 8 * piece;
#pragma unroll
    for (int j = 0; j < 4; ++j) asrc[j] = D.a + (int64_t)min(c0 + prow + 16 * j, D.rank - 1) * K + 8 * piece;
    u32x4 regs[6];
    auto load = [&](int chunk) {
        const int k0 = chunk * kLowKC;
#pragma unroll
        for (int j = 0; j < 2; ++j) regs[j] = *reinterpret_cast<const u32x4 *>(xsrc[j] + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) regs[2 + j] = *reinterpret_cast<const u32x4 *>(asrc[j] + k0);
    };
    auto store = [&](int buf) {
        uint8_t *st = stage[buf];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            *reinterpret_cast<u32x4 *>(st + (prow + 16 * j) * kLowPitch + 16 * piece) = regs[j];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u32x4 *>(st + kLowXBytes + (prow + 16 * j) * kLowPitch + 16 * piece) = regs[2 + j];
    };
    f32x16 acc0 = {}, acc1 = {};
    auto compute = [&](int buf) {
        const uint8_t *st = stage[buf];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int kb = 2 * (16 * (2 * wave + u) + 8 * h);  // byte offset of this lane's 8 K values
            const bf16x8 av = *reinterpret_cast<const bf16x8 *>(st + l32 * kLowPitch + kb);
            const bf16x8 b0 = *reinterpret_cast<const bf16x8 *>(st + kLowXBytes + l32 * kLowPitch + kb);
            const bf16x8 b1 = *reinterpret_cast<const bf16x8 *>(st + kLowXBytes + (32 + l32) * kLowPitch + kb);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b1, acc1, 0, 0, 0);
        }
    };
    const int nc_all = K / kLowKC;
    const int cb = (int)((int64_t)slice * nc_all / ks), ce = (int)((int64_t)(slice + 1) * nc_all / ks);
    if (cb < ce) {
        load(cb);
        store(0);
    }
    __syncthreads();
    for (int c = cb; c < ce; ++c) {
        if (c + 1 < ce) load(c + 1);
        compute((c - cb) & 1);
        if (c + 1 < ce) store((c - cb + 1) & 1);
        __syncthreads();
    }
    // Partial tiles through LDS (the staging buffers are free now): part[w][row][col].
    float *part = reinterpret_cast<float *>(&stage[0][0]);
    constexpr int kPartPitch = 65;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int row = 8 * (j >> 2) + 4 * h + (j & 3);
        part[(wave * 32 + row) * kPartPitch + l32] = acc0[j];
        part[(wave * 32 + row) * kPartPitch + 32 + l32] = acc1[j];
    }
    __syncthreads();
    for (int o = tid; o < 32 * 64; o += 256) {
        const int r = o >> 6, col = o & 63;
        if (r0 + r < D.row_count && c0 + col < D.rank) {
            float v = part[r * kPartPitch + col];
#pragma unroll
            for (int w = 1; w < 4; ++w) v += part[(w * 32 + r) * kPartPitch + col];
            D.low[(int64_t)slice * D.low_plane + (int64_t)(r0 + r) * D.low_stride + c0 + col] = v;
        }
    }
}

// Adds the K slices' partial planes of every adapter into plane 0, in slice order (the sum
// the epilogue reads). One thread per low element.
__global__ __launch_bounds__(256) void k_lora_low_reduce(LoraBatch batch) {
    const LoraDesc &D = batch.d[blockIdx.z];
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (D.ksplit < 2 || e >= D.low_plane) return;
    float v = D.low[e];
    for (int s = 1; s < D.ksplit; ++s) v += D.low[(int64_t)s * D.low_plane + e];
    D.low[e] = v;
}

// low = hi + mid + lo, each an exact bf16 (see the file comment), packed in MFMA operand form.
__device__ __forceinline__ void split3(const float (&lv)[8], bf16x8 &hi, bf16x8 &mid, bf16x8 &lo) {
    uint32_t hw[4], mw[4], lw[4];
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
        hw[i] = hp;
        mw[i] = mp;
        lw[i] = lp;
    }
    hi = __builtin_bit_cast(bf16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
    mid = __builtin_bit_cast(bf16x8, u32x4{mw[0], mw[1], mw[2], mw[3]});
    lo = __builtin_bit_cast(bf16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
}

// 8 consecutive B elements (k = kb .. kb + 7 of B row `row`), zero past the rank.
__device__ __forceinline__ bf16x8 load_b8(const LoraDesc &D, int row, int kb) {
    const uint16_t *br = D.b + (int64_t)row * D.rank;
    if (D.b_vec && kb + 8 <= D.rank) return *reinterpret_cast<const bf16x8 *>(br + kb);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = kb + 2 * i < D.rank ? br[kb + 2 * i] : 0u;
        const uint32_t hi = kb + 2 * i + 1 < D.rank ? br[kb + 2 * i + 1] : 0u;
        w[i] = lo | (hi << 16);
    }
    return __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
}

constexpr int kEpiRows = 32, kEpiCols = 256, kEpiPitch = kEpiCols + 8;  // pitch in bf16 elements

// One workgroup per 32 x 256 tile of y. The tile is read once (16-byte loads) into LDS; each
// wavefront then owns 64 columns (two 32 x 32 MFMA tiles t) in MFMA accumulator layout (lane
// (l32, h), value j: row 8(j/4) + 4h + (j%4), column 32t + l32), applies every adapter whose
// rows and output columns meet its part of the tile, in adapter order, then the bias, to those
// values where they lie in LDS (108 VGPRs, four wavefronts per SIMD; holding them in registers
// took 136 and three), and writes the tile back with 16-byte stores.
__global__ __launch_bounds__(256) void k_lora_epilogue(uint16_t *__restrict__ y, int64_t y_stride, int M, int N,
                                                       LoraBatch batch, const uint16_t *__restrict__ bias) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kEpiRows * kEpiPitch];
    const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int r0 = (int)blockIdx.x * kEpiRows, n0 = (int)blockIdx.y * kEpiCols;
    const bool vec_y = (y_stride % 8) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;

    // Coalesced load: pass p, thread t -> row 8p + t/32, columns 8(t%32) .. + 7.
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int row = 8 * p + (tid >> 5), col = 8 * (tid & 31), m = r0 + row, n = n0 + col;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (m < M) {
            const uint16_t *src = y + (int64_t)m * y_stride + n;
            if (vec_y && n + 8 <= N) {
                v = *reinterpret_cast<const u32x4 *>(src);
            } else {
                uint32_t e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) e[i] = n + i < N ? src[i] : 0u;
                v = u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
            }
        }
        *reinterpret_cast<u32x4 *>(&tile[row * kEpiPitch + col]) = v;
    }
    __syncthreads();

    // Lane (l32, h) of wavefront w owns the tile elements at its MFMA accumulator positions
    // (value j of tile t: row 8(j/4) + 4h + (j%4), column 64w + 32t + l32), which the adapters
    // and the bias update in place in LDS (every value is a bf16 between the steps).
    auto elem = [&](int t, int j) -> uint16_t & {
        return tile[(8 * (j >> 2) + 4 * h + (j & 3)) * kEpiPitch + 64 * wave + 32 * t + l32];
    };

    const int wcol0 = n0 + 64 * wave;  // this wavefront's first column
    for (int a = 0; a < batch.count; ++a) {
        const LoraDesc &D = batch.d[a];
        // Wave-uniform tests: the adapter's rows meet the tile's, its output columns this
        // wavefront's.
        if (r0 + kEpiRows <= D.row_begin || r0 >= D.row_begin + D.row_count) continue;
        if (wcol0 + 64 <= D.out_begin || wcol0 >= D.out_begin + D.out_count) continue;
        const float *lr = D.low + (int64_t)min(max(r0 + l32 - D.row_begin, 0), D.row_count - 1) * D.low_stride;
        const int b0 = min(max(wcol0 + l32 - D.out_begin, 0), D.out_count - 1);
        const int b1 = min(max(wcol0 + 32 + l32 - D.out_begin, 0), D.out_count - 1);
        f32x16 acc0 = {}, acc1 = {};
        for (int k0 = 0; k0 < D.rank; k0 += 16) {
            const int kb = k0 + 8 * h;
            float lv[8];
            if (kb + 8 <= D.rank) {
                const f32x4 l0 = *reinterpret_cast<const f32x4 *>(lr + kb);
                const f32x4 l1 = *reinterpret_cast<const f32x4 *>(lr + kb + 4);
                lv[0] = l0.x; lv[1] = l0.y; lv[2] = l0.z; lv[3] = l0.w;
                lv[4] = l1.x; lv[5] = l1.y; lv[6] = l1.z; lv[7] = l1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) lv[i] = kb + i < D.rank ? lr[kb + i] : 0.f;
            }
            bf16x8 hi, mid, lo;
            split3(lv, hi, mid, lo);
            const bf16x8 bv0 = load_b8(D, b0, kb), bv1 = load_b8(D, b1, kb);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, bv0, acc0, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mid, bv0, acc0, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, bv0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, bv1, acc1, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mid, bv1, acc1, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, bv1, acc1, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int n = wcol0 + 32 * t + l32;
            const bool col_in = n >= D.out_begin && n < D.out_begin + D.out_count;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int m = r0 + 8 * (j >> 2) + 4 * h + (j & 3);
                if (col_in && m >= D.row_begin && m < D.row_begin + D.row_count) {
                    const float d = __fmul_rn(D.scale, t ? acc1[j] : acc0[j]);
                    uint16_t &e = elem(t, j);
                    e = (uint16_t)float_to_bf16_bits(__fadd_rn(bf16_to_float(e), d));
                }
            }
        }
    }
    if (bias) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float b = bf16_to_float(bias[min(wcol0 + 32 * t + l32, N - 1)]);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                uint16_t &e = elem(t, j);
                e = (uint16_t)float_to_bf16_bits(bf16_to_float(e) + b);
            }
        }
    }

    __syncthreads();  // every wavefront's updates are in the tile before it is written back
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int row = 8 * p + (tid >> 5), col = 8 * (tid & 31), m = r0 + row, n = n0 + col;
        if (m >= M || n >= N) continue;
        const u32x4 val = *reinterpret_cast<const u32x4 *>(&tile[row * kEpiPitch + col]);
        uint16_t *dst = y + (int64_t)m * y_stride + n;
        if (vec_y && n + 8 <= N) {
            *reinterpret_cast<u32x4 *>(dst) = val;
        } else {
            const uint32_t e[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (n + i < N) dst[i] = (uint16_t)(e[i >> 1] >> (16 * (i & 1)));
        }
    }
}

}  // namespace

hipError_t launch_lora_low(const uint16_t *x, int64_t x_stride, int K, const LoraBatch &batch, hipStream_t stream) {
    int rows = 0, rank = 0;
    for (int a = 0; a < batch.count; ++a) {
        rows = std::max(rows, batch.d[a].row_count);
        rank = std::max(rank, batch.d[a].rank);
    }
    int ks = 1;
    for (int a = 0; a < batch.count; ++a) ks = std::max(ks, batch.d[a].ksplit);
    const dim3 grid((unsigned)((rows + 31) / 32), (unsigned)((rank + 63) / 64 * ks), (unsigned)batch.count);
    hipLaunchKernelGGL(k_lora_low, grid, dim3(256), 0, stream, x, x_stride, K, batch);
    if (ks > 1) {
        int64_t plane = 0;
        for (int a = 0; a < batch.count; ++a) plane = std::max(plane, batch.d[a].low_plane);
        hipLaunchKernelGGL(k_lora_low_reduce, dim3((unsigned)((plane + 255) / 256), 1, (unsigned)batch.count),
                           dim3(256), 0, stream, batch);
    }
    return hipGetLastError();
}

hipError_t launch_lora_epilogue(uint16_t *y, int64_t y_stride, int M, int N, const LoraBatch &batch,
                                const uint16_t *bias_bf16, hipStream_t stream) {
    const dim3 grid((unsigned)((M + kEpiRows - 1) / kEpiRows), (unsigned)((N + kEpiCols - 1) / kEpiCols));
    hipLaunchKernelGGL(k_lora_epilogue, grid, dim3(256), 0, stream, y, y_stride, M, N, batch, bias_bf16);
    return hipGetLastError();
}

}  // namespace tc
