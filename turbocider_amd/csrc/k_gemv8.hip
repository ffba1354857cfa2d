// Quantized GEMV for 2..8 activation rows (text-encoder prompts, small batches), Q4_K / Q5_K /
// Q6_K:
// y[m, n] = sum_k x[m, k] w[n, k] with w the exact fp32 dequantized weight, bf16 output (+ bias
// after the cast). HBM-bound: every weight byte is read once.
//
// Replaces the small-M side of mx::quantized_matmul (MLX qmv / qmm at M <= 8,
// native/backends/mlx.cpp:678) and the CPU-decode-then-GEMM pager route for short prompts
// (gguf_weight_pager.cpp:347-349,571-573).
//
// Scheme: one v_mfma_f32_16x16x32_bf16 per 32-weight sub-block ("group"): B is the group's
// codes for 16 weight rows (bf16 128 + code, exact, one byte permute per pair), A the group's
// 32 activations of up to 16 rows (rows past M read a zero row). The group's scale and min
// are applied to the 4 outputs each lane holds instead of to every weight:
//   y += d sc (D - 128 X) - dmin m X,   D = sum x * (128 + code),  X = sum x
// with X from a second MFMA of the same A against a B of ones. Q6_K's scale groups are 16
// weights, so a 32-column step spans two: A row r + 8 s (s = 0, 1) carries activation row r
// only in the 16 columns of group half s (zeros elsewhere), lane (n, h) then holds the four
// rows 4 (h & 1) + i of half h / 2, applies that group's scale (y += d sc (D - 160 X)), and
// the two halves are added across lanes at the end. No weight is rounded: the result is the
// fp32-dequant GEMV up to fp32 summation order.
//
// Memory: lane (n, h) of a 16-row tile loads the 8-byte pieces of weight row n that hold its
// eight codes of every step (Q4_K: qs[32 j + 8 h ..], low nibbles group 2 j, high 2 j + 1;
// Q5_K: the same at qs byte 48, plus qh[8 h ..] for the fifth bits, codes 0..31; Q6_K:
// ql[64 f + 32 q + 8 h ..] and qh[32 f + 8 h ..]) and the block's scales; a set is two Q4_K
// or Q5_K blocks or one Q6_K block. The activations of the set (M rows) go through a
// wavefront-private LDS area (each lane loads one 16-byte piece per row; for Q6_K's 256-column
// sets, half the lanes per row, two rows per load). Work split as in
// the one-row kernel: a workgroup owns a 16-row tile, its wavefronts interleave over the
// sets with two in flight, and partial sums are added through LDS in wavefront order.
#include "tc_device.h"
#include "tc_kernels.h"

#include <algorithm>

namespace tc {
namespace {

constexpr int kMaxRows = 8;
// Q4_K and Q5_K sets are two blocks (512 columns), Q6_K sets one (256).
template <uint32_t TYPE>
constexpr bool kPair = TYPE != kQ6K;
// One activation row of a set in LDS (bytes, padded): 512 columns (Q4_K, Q5_K) or 256 (Q6_K).
template <uint32_t TYPE>
constexpr int kRowLds = kPair<TYPE> ? 1024 + 16 : 512 + 16;
template <uint32_t TYPE>
constexpr int kWaveLds = (kMaxRows + 1) * kRowLds<TYPE>;  // M rows, then a zero row
// Activation load instructions per set: one row each (Q4_K, 64 lanes x 16 bytes = 1 KB), or
// two rows each (Q6_K: lanes 0..31 row 2 i, lanes 32..63 row 2 i + 1, 512 bytes each).
template <uint32_t TYPE, int MR>
constexpr int kXLoads = kPair<TYPE> ? MR : MR / 2;

// Set geometry: K columns and bytes per row (Q4_K, Q5_K: two blocks; Q6_K: one).
template <uint32_t TYPE>
constexpr int set_k() { return kPair<TYPE> ? 512 : 256; }
template <uint32_t TYPE>
constexpr int block_bytes() { return TYPE == kQ4K ? kQ4KBytes : TYPE == kQ5K ? kQ5KBytes : kQ6KBytes; }
template <uint32_t TYPE>
constexpr int set_bytes() { return kPair<TYPE> ? 2 * block_bytes<TYPE>() : kQ6KBytes; }

typedef uint32_t u32x2a8 __attribute__((ext_vector_type(2), aligned(8)));
typedef uint32_t u32x2a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32a2 __attribute__((aligned(2)));

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}
// Bytes 0, 1 and 2, 3 of t as bf16 pairs 0x4300 | byte = 128 + byte.
__device__ __forceinline__ uint32_t pair01(uint32_t t) { return __builtin_amdgcn_perm(0x43434343u, t, 0x04010400u); }
__device__ __forceinline__ uint32_t pair23(uint32_t t) { return __builtin_amdgcn_perm(0x43434343u, t, 0x04030402u); }

// One pipeline stage: the lane's weight pieces and scales of a set, and its 16-byte pieces of
// the set's activation rows (kXLoads of them). Q4_K: q[b][j] = qs[32 j + 8 h ..] of block b, hd[b] its
// header; Q5_K as well (qs at byte 48), with qh5[b] = qh[8 h ..]: bit g of byte c is the fifth
// code bit of column 8 h + c of group g (gguf_decode.cpp:77-90). Q6_K: q[0][2 f + u] =
// ql[64 f + 32 u + 8 h ..], q[1][f] = qh[32 f + 8 h ..], hd[0] = the 16 int8 scales,
// q[1][2].x = d (fp16 bits).
struct Stage {
    u32x2 q[2][4];
    u32x2 qh5[2];
    u32x4 hd[2];
    u32x4 xs[kMaxRows];
};

template <uint32_t TYPE, int MR>
__device__ __forceinline__ void issue(Stage &st, __amdgpu_buffer_rsrc_t xr, int64_t x_stride, const uint8_t *w,
                                      int64_t pitch, int N, int tile, int set, int nsb, int lane) {
    const int n = lane & 15, h = lane >> 4;
    const uint8_t *b0 = w + (int64_t)min(16 * tile + n, N - 1) * pitch + (int64_t)set * set_bytes<TYPE>();
    if constexpr (kPair<TYPE>) {
        constexpr int kQs = TYPE == kQ4K ? 16 : 48;  // the qs bytes (Q5_K: after the 32-byte qh plane)
        // A missing second block re-reads the first.
        const uint8_t *b1 = 2 * set + 1 < nsb ? b0 + block_bytes<TYPE>() : b0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            st.q[0][j] = *reinterpret_cast<const u32x2a8 *>(b0 + kQs + 32 * j + 8 * h);
            st.q[1][j] = *reinterpret_cast<const u32x2a8 *>(b1 + kQs + 32 * j + 8 * h);
        }
        if constexpr (TYPE == kQ5K) {
            st.qh5[0] = *reinterpret_cast<const u32x2a8 *>(b0 + 16 + 8 * h);
            st.qh5[1] = *reinterpret_cast<const u32x2a8 *>(b1 + 16 + 8 * h);
        }
        st.hd[0] = *reinterpret_cast<const u32x4 *>(b0);
        st.hd[1] = *reinterpret_cast<const u32x4 *>(b1);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) st.q[0][j] = *reinterpret_cast<const u32x2a2 *>(b0 + 64 * (j >> 1) + 32 * (j & 1) + 8 * h);
        st.q[1][0] = *reinterpret_cast<const u32x2a2 *>(b0 + 128 + 8 * h);
        st.q[1][1] = *reinterpret_cast<const u32x2a2 *>(b0 + 160 + 8 * h);
        st.hd[0] = *reinterpret_cast<const u32x4a2 *>(b0 + 192);
        st.q[1][2].x = *reinterpret_cast<const u32a2 *>(b0 + 206) >> 16;  // d (the block's last 2 bytes)
    }
    // Q4_K: row r's piece `lane` (columns set_k set + 8 lane .. + 7); Q6_K: row 2 i + lane / 32,
    // piece lane % 32. Past the matrix end the loads read 0.
#pragma unroll
    for (int i = 0; i < kXLoads<TYPE, MR>; ++i) {
        const int r = kPair<TYPE> ? i : 2 * i + (lane >> 5), p = kPair<TYPE> ? lane : lane & 31;
        const uint32_t off = (uint32_t)(2 * ((int64_t)r * x_stride + (int64_t)set * set_k<TYPE>() + 8 * p));
        st.xs[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    }
    asm volatile("" ::: "memory");  // keep the loads here, a full stage ahead of their use
}

template <uint32_t TYPE, int MR>
__device__ __forceinline__ void compute(const Stage &st, uint8_t *wl, const uint8_t *abase, int lane, int set,
                                        int nsb, f32x4 &acc) {
#pragma unroll
    for (int i = 0; i < kXLoads<TYPE, MR>; ++i) {
        const int r = kPair<TYPE> ? i : 2 * i + (lane >> 5), p = kPair<TYPE> ? lane : lane & 31;
        *reinterpret_cast<u32x4 *>(wl + r * kRowLds<TYPE> + 16 * p) = st.xs[i];
    }
    const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    if constexpr (TYPE == kQ6K) {
        // Step t (columns 32 t .. + 31): half f = t / 4, quarter g = t % 4; the lane's codes are
        // positions 8 h .. + 7 of the step, scale group 8 f + 2 g + h / 2.
        const int h = lane >> 4;
        const float d = half_to_float(st.q[1][2].x);
        const uint32_t sh = (uint32_t)(h >> 1);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int f = t >> 2, g = t & 3;
            const u32x2 ql = st.q[0][2 * f + (g & 1)], qh = st.q[1][f];
            const uint32_t l0 = g < 2 ? ql.x & 0x0f0f0f0fu : (ql.x >> 4) & 0x0f0f0f0fu;
            const uint32_t l1 = g < 2 ? ql.y & 0x0f0f0f0fu : (ql.y >> 4) & 0x0f0f0f0fu;
            const uint32_t c0 = l0 | (((qh.x >> (2 * g)) & 0x03030303u) << 4);
            const uint32_t c1 = l1 | (((qh.y >> (2 * g)) & 0x03030303u) << 4);
            const u32x4 B = {pair01(c0), pair23(c0), pair01(c1), pair23(c1)};
            const u32x4 A = *reinterpret_cast<const u32x4 *>(abase + 64 * t);
            const f32x4 D = mfma16(A, B, f32x4{0.f, 0.f, 0.f, 0.f});
            const f32x4 X = mfma16(A, ones, f32x4{0.f, 0.f, 0.f, 0.f});
            const int grp = 8 * f + 2 * g;  // + h / 2
            const uint32_t sw = st.hd[0][grp >> 2] >> (8 * ((grp & 3) + sh));
            const float a = d * (float)(int8_t)(uint8_t)sw;
            const float ax = 160.f * a;
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(a, D[i], __builtin_fmaf(-ax, X[i], acc[i]));
        }
        return;
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        if (b == 1 && 2 * set + 1 >= nsb) break;  // uniform: the set's second block does not exist
        const uint32_t dd = st.hd[b].x, s0 = st.hd[b].y, s1 = st.hd[b].z, s2 = st.hd[b].w;
        const float d = half_to_float(dd), dmin = half_to_float(dd >> 16);
#pragma unroll
        for (int gl = 0; gl < 8; ++gl) {
            const int j = gl >> 1, g = 8 * b + gl;
            const uint32_t w0 = st.q[b][j].x, w1 = st.q[b][j].y;
            uint32_t c0 = (gl & 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu;
            uint32_t c1 = (gl & 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu;
            if constexpr (TYPE == kQ5K) {  // fifth bit: bit gl of each qh byte (codes 0..31)
                c0 |= ((st.qh5[b].x >> gl) & 0x01010101u) << 4;
                c1 |= ((st.qh5[b].y >> gl) & 0x01010101u) << 4;
            }
            const u32x4 B = {pair01(c0), pair23(c0), pair01(c1), pair23(c1)};
            const u32x4 A = *reinterpret_cast<const u32x4 *>(abase + 64 * g);
            const f32x4 D = mfma16(A, B, f32x4{0.f, 0.f, 0.f, 0.f});
            const f32x4 X = mfma16(A, ones, f32x4{0.f, 0.f, 0.f, 0.f});
            uint32_t sc, m;
            scale_min_k4((uint32_t)gl, s0, s1, s2, sc, m);
            const float a = d * (float)sc, bm = dmin * (float)m;
            const float ax = __builtin_fmaf(128.f, a, bm);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(a, D[i], __builtin_fmaf(-ax, X[i], acc[i]));
        }
    }
}

// Workgroup: one 16-row weight tile, W wavefronts; wavefront w takes the sets w, w + W, ...
// with two sets in flight (ping-pong stages). Lane (n, h) accumulates y[4 h + i][16 tile + n]
// (MFMA output layout); the wavefronts' partial sums are added through LDS in order.
template <uint32_t TYPE, int MR>
__global__ __launch_bounds__(512) void k_gemv8(const uint16_t *__restrict__ x, int64_t x_stride, int M,
                                               Gemv1Segments segs, int64_t pitch, int nsb, int nks) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = (int)threadIdx.x, lane = tid & 63, h = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = (int)(blockDim.x >> 6);
    // Segment of this workgroup's tile: matrices sharing x (same K and type) laid end to end
    // in tile order.
    int seg = 0;
    while (seg + 1 < segs.count && (int)blockIdx.x >= segs.tile_begin[seg + 1]) ++seg;
    const int tile = (int)blockIdx.x - segs.tile_begin[seg];
    const uint8_t *__restrict__ w = segs.w[seg];
    uint16_t *__restrict__ y = segs.y[seg];
    const int64_t y_stride = segs.y_stride[seg];
    const uint16_t *__restrict__ bias = segs.bias[seg];
    const int N = segs.n[seg];
    uint8_t *wl = lds + wave * kWaveLds<TYPE>;
    float *red = reinterpret_cast<float *>(lds + nw * kWaveLds<TYPE>);  // [nw][16 rows][16 columns]
    // The zero row, for A rows past M.
    if (kPair<TYPE> || lane < 32) *reinterpret_cast<u32x4 *>(wl + MR * kRowLds<TYPE> + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
    // A row c: Q4_K activation row c; Q6_K row c % 8 in the 16 columns of half c / 8 (lanes
    // of the other half read zeros).
    const bool a_live = kPair<TYPE> ? c < M : ((c & 7) < M && (c >> 3) == (h >> 1));
    const uint8_t *abase = wl + (a_live ? (c & (kPair<TYPE> ? 15 : 7)) * kRowLds<TYPE> : MR * kRowLds<TYPE>) + 16 * h;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(x), 0, (int)(2 * ((int64_t)(M - 1) * x_stride + 256 * (int64_t)nsb)), 0x00020000);

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int nmine = wave < nks ? (nks - 1 - wave) / nw + 1 : 0;
    if (nmine > 0) {
        Stage A, B;
        int ks = wave;
        issue<TYPE, MR>(A, xr, x_stride, w, pitch, N, tile, ks, nsb, lane);
        for (int i = (nmine - 1) >> 1; i > 0; --i, ks += 2 * nw) {
            issue<TYPE, MR>(B, xr, x_stride, w, pitch, N, tile, ks + nw, nsb, lane);
            compute<TYPE, MR>(A, wl, abase, lane, ks, nsb, acc);
            issue<TYPE, MR>(A, xr, x_stride, w, pitch, N, tile, ks + 2 * nw, nsb, lane);
            compute<TYPE, MR>(B, wl, abase, lane, ks + nw, nsb, acc);
        }
        if ((nmine & 1) == 0) {
            issue<TYPE, MR>(B, xr, x_stride, w, pitch, N, tile, ks + nw, nsb, lane);
            compute<TYPE, MR>(A, wl, abase, lane, ks, nsb, acc);
            compute<TYPE, MR>(B, wl, abase, lane, ks + nw, nsb, acc);
        } else {
            compute<TYPE, MR>(A, wl, abase, lane, ks, nsb, acc);
        }
    }
    if constexpr (TYPE == kQ6K) {
        // Lanes h and h + 2 hold the two group halves of rows 4 (h & 1) + i: add them.
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += __shfl_xor(acc[i], 32);
        if (h < 2) {
#pragma unroll
            for (int i = 0; i < 4; ++i) red[(wave * 16 + 4 * h + i) * 16 + c] = acc[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(wave * 16 + 4 * h + i) * 16 + c] = acc[i];
    }
    __syncthreads();
    for (int t = tid; t < 16 * M; t += (int)blockDim.x) {
        const int m = t >> 4, col = t & 15, n = 16 * tile + col;
        if (n < N) {
            float v = 0.f;
            for (int k = 0; k < nw; ++k) v += red[(k * 16 + m) * 16 + col];  // wavefront order
            uint32_t out = float_to_bf16_bits(v);
            if (bias) out = float_to_bf16_bits(bf16_to_float(out) + bf16_to_float(bias[n]));
            if (segs.act == kActSiluGlu) {
                // t and t ^ 1 (gate and up of one output) are adjacent lanes of the same
                // iteration: blockDim.x is a multiple of 16 and N is even.
                const uint32_t up = (uint32_t)__shfl_xor((int)out, 1);
                if ((n & 1) == 0) y[(int64_t)m * y_stride + (n >> 1)] = (uint16_t)silu_glu_bits(out, up);
            } else {
                y[(int64_t)m * y_stride + n] = (uint16_t)(segs.act == kActGeluTanh ? gelu_tanh_bits(out) : out);
            }
        }
    }
}

}  // namespace

bool gemv8_supports(uint32_t type, int M, int K, int64_t x_stride) {
    // The activation descriptor spans rows 0..M-1 with 32-bit offsets.
    return (type == kQ4K || type == kQ5K || type == kQ6K) && M >= 2 && M <= kMaxRows &&
           2 * ((int64_t)(M - 1) * x_stride + (int64_t)K) < (1ll << 31);
}

hipError_t launch_gemv8_segments(uint32_t type, const uint16_t *x, int64_t x_stride, int M,
                                 const Gemv1Segments &segs, int K, hipStream_t stream, int force_w) {
    if (!gemv8_supports(type, M, K, x_stride) || K % 256) return hipErrorInvalidValue;
    const int nsb = K / 256, nks = type != kQ6K ? (nsb + 1) / 2 : nsb, tiles = segs.tile_begin[segs.count];
    int W = force_w > 0 ? force_w : std::min(8, std::max(4, 4096 / tiles));
    W = std::min(W, nks);
    const int64_t pitch = (int64_t)nsb * (type == kQ4K ? kQ4KBytes : type == kQ5K ? kQ5KBytes : kQ6KBytes);
    const size_t lds = (size_t)W * ((type != kQ6K ? kWaveLds<kQ4K> : kWaveLds<kQ6K>) + 16 * 16 * sizeof(float));
#define TC_GEMV8(T, R)                                                                                          \
    hipLaunchKernelGGL((k_gemv8<T, R>), dim3((unsigned)tiles), dim3((unsigned)(64 * W)), lds, stream, x, x_stride, \
                       M, segs, pitch, nsb, nks)
    if (type == kQ4K) {
        if (M <= 4) TC_GEMV8(kQ4K, 4); else TC_GEMV8(kQ4K, 8);
    } else if (type == kQ5K) {
        if (M <= 4) TC_GEMV8(kQ5K, 4); else TC_GEMV8(kQ5K, 8);
    } else {
        if (M <= 4) TC_GEMV8(kQ6K, 4); else TC_GEMV8(kQ6K, 8);
    }
#undef TC_GEMV8
    return hipGetLastError();
}

hipError_t launch_gemv8(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                        uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, hipStream_t stream, int force_w,
                        int act) {
    Gemv1Segments segs{};
    segs.count = 1;
    segs.act = act;
    segs.w[0] = w;
    segs.y[0] = y;
    segs.y_stride[0] = y_stride;
    segs.bias[0] = bias_bf16;
    segs.n[0] = N;
    segs.tile_begin[0] = 0;
    segs.tile_begin[1] = (N + 15) / 16;
    return launch_gemv8_segments(type, x, x_stride, M, segs, K, stream, force_w);
}

}  // namespace tc
