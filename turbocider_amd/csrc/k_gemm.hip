// Fused K-quant dequant + bf16 MFMA GEMM for gfx950:  y[M,N] = bf16(x[M,K] * deq(W)^T) (+bias).
//
// Replaces the reference's Metal quantized matmul (mx::quantized_matmul affine QMM,
// native/backends/mlx.cpp:678-679, and affine_gpu::projection_shared,
// native/backends/affine_gpu_shared.hpp:41-84), decoding raw GGUF blocks instead of the
// reference's lossy affine repack (native/core/gguf_affine.cpp:147-307).
//
// Tiling (one workgroup of 4 wavefronts, one wavefront per SIMD):
//   * block tile 256 (M) x 256 (N); wavefront w owns all 256 rows of M and the 64 columns
//     [64w, 64w + 64) of N as 8 x 2 tiles of v_mfma_f32_32x32x16_bf16 (256 fp32
//     accumulators per lane), so every weight is dequantized exactly once per workgroup;
//   * the K loop walks 64-wide chunks. A chunk is one 32-byte qs segment of a Q4_K block
//     (sub-blocks 2p and 2p+1: low and high nibbles), or one ql segment of a Q6_K block
//     (sub-blocks p and p+2). Its K set is two 32-wide runs, seg0 and seg1; the MFMA K
//     order inside a chunk follows the nibble layout, which is legal because the sum over
//     K does not depend on the order in which A and B visit it;
//   * activations for the chunk (256 rows x 64 bf16) are staged through LDS (double
//     buffered, 144-byte row pitch so that the 16-byte fragment reads of 8/16 consecutive
//     lanes fall in distinct banks); the raw weight bytes go straight from global memory
//     to registers (16-byte loads), are dequantized to bf16 in registers by the lane that
//     feeds them to the MFMA, and never touch LDS.
// Dequantization is bit-exact: fp32 fma(d*sc, q, -dmin*m) (Q4_K) / (d*sc)*(q-32) (Q6_K)
// rounded once (every product is exact), then RNE to bf16 (v_cvt_pk_bf16_f32).
// Epilogue: y = RNE_bf16(acc); with a bias y = RNE_bf16(f32(y) + f32(bias_bf16))
// (bias added after the cast, native/backends/metal_graph/kernels/dense_linear.hpp:139-141).
#include "tc_device.h"
#include "tc_kernels.h"

#include <type_traits>

namespace tc {
namespace {

constexpr int kBM = 256, kBN = 256, kThreads = 256;
constexpr int kXPitch = 144;                 // bytes per activation row of a chunk in LDS
constexpr int kXBuf = kBM * kXPitch;         // 36864 bytes per buffer

struct WRegs {   // raw weight bytes of one chunk for one 32-column MFMA tile
    u32x4 q;     // Q4_K: 16 qs bytes; Q6_K: 16 ql bytes
    u32x4 h;     // Q4_K: block header (d, dmin, 12 scale bytes); Q6_K: 16 qh bytes
    uint32_t s;  // Q6_K: d (low 16 bits) | sc_lo byte << 16 | sc_hi byte << 24
};

template <uint32_t TYPE, int Q>
__device__ __forceinline__ void load_w(WRegs &r, const uint8_t *row, int sb, int h) {
    if constexpr (TYPE == kQ4K) {
        const uint8_t *blk = row + sb * kQ4KBytes;
        r.q = *reinterpret_cast<const u32x4 *>(blk + 16 + 32 * Q + 16 * h);
        r.h = *reinterpret_cast<const u32x4 *>(blk);
        r.s = 0;
    } else {
        constexpr int hh = Q >> 1, p = Q & 1;
        const uint8_t *blk = row + sb * kQ6KBytes;
        r.q = load16_align2(blk + 64 * hh + 32 * p + 16 * h);
        r.h = load16_align2(blk + 128 + 32 * hh + 16 * h);
        const uint32_t d = *reinterpret_cast<const uint16_t *>(blk + 208);
        const uint32_t s_lo = blk[192 + 8 * hh + 2 * p + h], s_hi = blk[192 + 8 * hh + 2 * p + 4 + h];
        r.s = d | (s_lo << 16) | (s_hi << 24);
    }
}

// Scale (a) and offset (b) of the two sub-blocks a lane meets in chunk Q: w = a*q - b.
// Half 0 (MFMA steps 0, 1) is sub-block 2Q (Q4_K) / Q&1 (Q6_K), half 1 (steps 2, 3) is
// 2Q+1 / (Q&1)+2. The products are exact (see tc_device.h).
struct ChunkScales {
    float a0, b0, a1, b1;
};

template <uint32_t TYPE, int Q>
__device__ __forceinline__ ChunkScales chunk_scales(const WRegs &r) {
    ChunkScales cs;
    if constexpr (TYPE == kQ4K) {
        const float d = half_to_float(r.h.x), dmin = half_to_float(r.h.x >> 16);
        uint32_t sc, m;
        scale_min_k4(2 * Q, r.h.y, r.h.z, r.h.w, sc, m);
        cs.a0 = d * (float)sc;
        cs.b0 = dmin * (float)m;
        scale_min_k4(2 * Q + 1, r.h.y, r.h.z, r.h.w, sc, m);
        cs.a1 = d * (float)sc;
        cs.b1 = dmin * (float)m;
    } else {
        const float d = half_to_float(r.s);
        cs.a0 = d * (float)(int8_t)(uint8_t)(r.s >> 16);
        cs.a1 = d * (float)(int8_t)(uint8_t)(r.s >> 24);
        cs.b0 = 32.f * cs.a0;  // (code - 32) * a = code * a - 32 a, exact
        cs.b1 = 32.f * cs.a1;
    }
    return cs;
}

// Dequantize the 8 weights this lane feeds to MFMA step S (0..3) of chunk Q of a block.
template <uint32_t TYPE, int Q, int S>
__device__ __forceinline__ bf16x8 dequant_step(const WRegs &r, const ChunkScales &cs) {
    const uint32_t w0 = (S & 1) ? r.q.z : r.q.x, w1 = (S & 1) ? r.q.w : r.q.y;
    const float a = (S >> 1) ? cs.a1 : cs.a0, b = (S >> 1) ? cs.b1 : cs.b0;
    uint32_t c0, c1;
    if constexpr (TYPE == kQ4K) {
        c0 = (S >> 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu;
        c1 = (S >> 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu;
    } else {
        constexpr uint32_t g = (Q & 1) + 2 * (S >> 1);
        const uint32_t h0 = (S & 1) ? r.h.z : r.h.x, h1 = (S & 1) ? r.h.w : r.h.y;
        c0 = ((S >> 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu) | (((h0 >> (2 * g)) & 0x03030303u) << 4);
        c1 = ((S >> 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu) | (((h1 >> (2 * g)) & 0x03030303u) << 4);
    }
    const float v0 = __builtin_fmaf(a, (float)(c0 & 0xffu), -b), v1 = __builtin_fmaf(a, (float)((c0 >> 8) & 0xffu), -b);
    const float v2 = __builtin_fmaf(a, (float)((c0 >> 16) & 0xffu), -b), v3 = __builtin_fmaf(a, (float)(c0 >> 24), -b);
    const float v4 = __builtin_fmaf(a, (float)(c1 & 0xffu), -b), v5 = __builtin_fmaf(a, (float)((c1 >> 8) & 0xffu), -b);
    const float v6 = __builtin_fmaf(a, (float)((c1 >> 16) & 0xffu), -b), v7 = __builtin_fmaf(a, (float)(c1 >> 24), -b);
    const u32x4 packed = {pack_bf16x2(v0, v1), pack_bf16x2(v2, v3), pack_bf16x2(v4, v5), pack_bf16x2(v6, v7)};
    return __builtin_bit_cast(bf16x8, packed);
}

// Column of 16-byte activation piece `piece` (0..7) of chunk Q of block sb: pieces 0..3
// cover the chunk's first 32-wide K run, pieces 4..7 the second.
template <uint32_t TYPE, int Q>
__device__ __forceinline__ int chunk_column(int sb, int piece) {
    int seg0, seg1;
    if constexpr (TYPE == kQ4K) {
        seg0 = 256 * sb + 64 * Q;
        seg1 = seg0 + 32;
    } else {
        seg0 = 256 * sb + 128 * (Q >> 1) + 32 * (Q & 1);
        seg1 = seg0 + 64;
    }
    return piece < 4 ? seg0 + 8 * piece : seg1 + 8 * (piece - 4);
}

template <uint32_t TYPE, bool HAS_BIAS>
__global__ __launch_bounds__(kThreads, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemm(const uint16_t *__restrict__ x, int64_t x_stride, int M, const uint8_t *__restrict__ w,
            int64_t w_pitch, int N, int K, uint16_t *__restrict__ y, int64_t y_stride,
            const uint16_t *__restrict__ bias, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kXBuf];

    // Tile order. Workgroup ids are dispatched round-robin over the 8 XCDs; remap them so
    // that each XCD (own L2) receives a contiguous run of tiles, then walk the run in
    // bands of 4 M-tiles so that resident workgroups share weight and activation tiles.
    const int total = tiles_m * tiles_n;
    int bid = (int)blockIdx.x;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    constexpr int kBand = 4;
    const int band = bid / (kBand * tiles_n), first_m = band * kBand;
    const int band_m = min(tiles_m - first_m, kBand);
    const int in_band = bid - band * kBand * tiles_n;
    const int tm = first_m + in_band % band_m, tn = in_band / band_m;
    const int m0 = tm * kBM, n0 = tn * kBN;

    const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const uint8_t *wrow0 = w + (int64_t)min(n0 + 64 * wave + l32, N - 1) * w_pitch;
    const uint8_t *wrow1 = w + (int64_t)min(n0 + 64 * wave + 32 + l32, N - 1) * w_pitch;

    // Activation staging: this thread moves 16-byte piece (tid & 7) of rows (tid >> 3) + 32 i.
    const int piece = tid & 7, prow = tid >> 3;
    const uint16_t *xrow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xrow[i] = x + (int64_t)min(m0 + prow + 32 * i, M - 1) * x_stride;

    f32x16 acc[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        acc[i][0] = f32x16{};
        acc[i][1] = f32x16{};
    }

    const int nsb = K / 256;
    u32x4 xr[8];
    WRegs wc0, wc1, wn0, wn1;
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4 *>(lds + buf * kXBuf + (prow + 32 * i) * kXPitch + piece * 16) = xr[i];
    };

    {
        const int col = chunk_column<TYPE, 0>(0, piece);
#pragma unroll
        for (int i = 0; i < 8; ++i) xr[i] = *reinterpret_cast<const u32x4 *>(xrow[i] + col);
    }
    load_w<TYPE, 0>(wc0, wrow0, 0, h);
    load_w<TYPE, 0>(wc1, wrow1, 0, h);
    store_x(0);
    __syncthreads();

    for (int sb = 0; sb < nsb; ++sb) {
        // One iteration per 64-wide chunk Q of super-block sb; chunk c = 4 sb + Q uses LDS
        // buffer Q & 1 while chunk c + 1 is fetched into registers.
        auto chunk = [&](auto qtag) {
            constexpr int Q = decltype(qtag)::value;
            constexpr int QN = (Q + 1) & 3;
            // Next chunk's loads are unconditional (the block index is clamped on the last
            // chunk; the extra loads and the write to the idle LDS buffer are never used).
            const int sbn = Q == 3 ? min(sb + 1, nsb - 1) : sb;
            {
                const int col = chunk_column<TYPE, QN>(sbn, piece);
#pragma unroll
                for (int i = 0; i < 8; ++i) xr[i] = *reinterpret_cast<const u32x4 *>(xrow[i] + col);
                load_w<TYPE, QN>(wn0, wrow0, sbn, h);
                load_w<TYPE, QN>(wn1, wrow1, sbn, h);
            }
            const uint8_t *xb = lds + (Q & 1) * kXBuf + l32 * kXPitch + 32 * h;
            const ChunkScales cs0 = chunk_scales<TYPE, Q>(wc0), cs1 = chunk_scales<TYPE, Q>(wc1);
            // Operands of step S are prepared while the 16 MFMAs of step S - 1 run.
            bf16x8 a_even[8], a_odd[8], b_even[2], b_odd[2];
            auto prepare = [&](auto stag, bf16x8(&a)[8], bf16x8(&b)[2]) {
                constexpr int S = decltype(stag)::value;
                constexpr int koff = 64 * (S >> 1) + 16 * (S & 1);
#pragma unroll
                for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const bf16x8 *>(xb + 32 * i * kXPitch + koff);
                b[0] = dequant_step<TYPE, Q, S>(wc0, cs0);
                b[1] = dequant_step<TYPE, Q, S>(wc1, cs1);
            };
            auto mfmas = [&](const bf16x8(&a)[8], const bf16x8(&b)[2]) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[0], acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[1], acc[i][1], 0, 0, 0);
                }
            };
            // Interleave: each MFMA (8 passes) covers one LDS read and up to 3 VALU ops.
            auto interleave = [&]() {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
            };
            prepare(std::integral_constant<int, 0>{}, a_even, b_even);
            prepare(std::integral_constant<int, 1>{}, a_odd, b_odd);
            mfmas(a_even, b_even);
            interleave();
            prepare(std::integral_constant<int, 2>{}, a_even, b_even);
            mfmas(a_odd, b_odd);
            interleave();
            prepare(std::integral_constant<int, 3>{}, a_odd, b_odd);
            mfmas(a_even, b_even);
            interleave();
            mfmas(a_odd, b_odd);
            store_x(QN & 1);
            __syncthreads();
            wc0 = wn0;
            wc1 = wn1;
        };
        chunk(std::integral_constant<int, 0>{});
        chunk(std::integral_constant<int, 1>{});
        chunk(std::integral_constant<int, 2>{});
        chunk(std::integral_constant<int, 3>{});
    }

    // Epilogue. Lane (l32, h) of tile (i, t) holds column n0 + 64w + 32t + l32 and rows
    // m0 + 32i + 8(j/4) + 4h + (j%4) for accumulator j = 0..15.
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int n = n0 + 64 * wave + 32 * t + l32;
        if (n >= N) continue;
        float bv = 0.f;
        if constexpr (HAS_BIAS) bv = bf16_to_float(bias[n]);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int m = m0 + 32 * i + 8 * (j >> 2) + 4 * h + (j & 3);
                if (m < M) {
                    uint32_t v = float_to_bf16_bits(acc[i][t][j]);
                    if constexpr (HAS_BIAS) v = float_to_bf16_bits(bf16_to_float(v) + bv);
                    y[(int64_t)m * y_stride + n] = (uint16_t)v;
                }
            }
    }
}

}  // namespace

hipError_t launch_gemm(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                       uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, hipStream_t stream) {
    const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
    const dim3 grid((unsigned)(tiles_m * tiles_n)), block(kThreads);
    const int64_t pitch = (int64_t)(K / 256) * (type == kQ4K ? kQ4KBytes : kQ6KBytes);
#define TC_GEMM_LAUNCH(T, B)                                                                                  \
    hipLaunchKernelGGL((k_gemm<T, B>), grid, block, 0, stream, x, x_stride, M, w, pitch, N, K, y, y_stride, \
                       bias_bf16, tiles_m, tiles_n)
    if (type == kQ4K) {
        if (bias_bf16) TC_GEMM_LAUNCH(kQ4K, true); else TC_GEMM_LAUNCH(kQ4K, false);
    } else {
        if (bias_bf16) TC_GEMM_LAUNCH(kQ6K, true); else TC_GEMM_LAUNCH(kQ6K, false);
    }
#undef TC_GEMM_LAUNCH
    return hipGetLastError();
}

}  // namespace tc
