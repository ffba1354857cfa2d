// Skinny quantized linear for 2 <= M <= 8 (text-encoder tokens, adaLN modulation at M = 1):
// HBM-bound, so each weight byte is read once and the per-weight ALU work is minimal.
//
// Replaces the small-M side of mx::quantized_matmul (MLX qmv, native/backends/mlx.cpp:678)
// and the CPU-decode-then-GEMM pager route of the text encoder
// (native/runtime/streaming/gguf_weight_pager.cpp:347-349,571-573).
//
// Arithmetic: weights are used at their exact fp32 values. For a run of 16 weights that
// share one sub-block scale a (and min b), sum_k x_k (a q_k - b) = a * sum_k x_k q_k - b * sum_k x_k.
// The codes enter v_dot2_f32_bf16 as the bf16 numbers 128 + q (exact: 7 mantissa bits cover
// 128..255), so sum x (128 + q) - 128 sum x = sum x q. No weight is rounded to bf16, so the
// result is the CPU "dequant to fp32 + fp32 GEMM" up to fp32 summation order.
//
// Work split: a workgroup owns 8*RS consecutive weight rows and splits the K super-blocks
// over its KW wavefronts (wavefront w takes blocks w, w + KW, ...). Inside a wavefront a
// team of 8 lanes covers one super-block of one row, lane p holding one 16-byte qs/ql piece
// (32 weights); the 8 teams cover 8 rows. Activations for the wavefront's block stay in
// registers for all 8*RS rows. Partial sums are reduced over the team with lane shuffles and
// over the wavefronts through LDS, then cast to bf16 (+ bias after the cast).
#include "tc_device.h"
#include "tc_kernels.h"

namespace tc {
namespace {

// Wavefronts per workgroup: 16 (128 VGPRs each) for up to 2 activation rows, else 8
// (256 VGPRs each).
template <int MAXM>
constexpr int max_waves() { return MAXM <= 2 ? 16 : 8; }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Activations of one 16-wide run, rearranged into the pair order of the code pairs:
// pa[i] = (x[4i], x[4i+2]), pb[i] = (x[4i+1], x[4i+3]); s = sum of the 16 values.
struct XRun {
    uint32_t pa[4], pb[4];
    float s;
};

__device__ __forceinline__ void make_run(XRun &r, const u32x4 v0, const u32x4 v1) {
    const uint32_t d[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = d[2 * i], hi = d[2 * i + 1];  // (x0, x1), (x2, x3)
        r.pa[i] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        r.pb[i] = __builtin_amdgcn_perm(hi, lo, 0x07060302u);
        s += bf16_to_float(lo) + bf16_to_float(lo >> 16) + bf16_to_float(hi) + bf16_to_float(hi >> 16);
    }
    r.s = s;
}

// sum over the run of x * (128 + code) given the code pairs ca[i], cb[i] (bf16 128 + code).
__device__ __forceinline__ float run_dot(const XRun &x, const uint32_t ca[4], const uint32_t cb[4], float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = dot2(ca[i], x.pa[i], acc);
        acc = dot2(cb[i], x.pb[i], acc);
    }
    return acc;
}

// Raw bytes of one super-block column for this lane: activations of its two 16-wide runs
// for every row of x, and the weight piece (+ header / high bits / scales) of its RS rows.
template <uint32_t TYPE, int MAXM, int RS>
struct Stage {
    u32x4 x[MAXM][4];
    u32x4 q[RS];     // Q4_K: 16 qs bytes; Q6_K: 16 ql bytes
    u32x4 h[RS];     // Q4_K: block header; Q6_K: 16 qh bytes
    uint32_t s[RS];  // Q6_K: d | sc_lo << 16 | sc_hi << 24
};

template <uint32_t TYPE, int MAXM, int RS>
__device__ __forceinline__ void load_stage(Stage<TYPE, MAXM, RS> &st, const uint16_t *const (&xrow)[MAXM],
                                           const uint8_t *const (&wrow)[RS], int sb, int run0, int run1, int p) {
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        const uint16_t *xp = xrow[m] + 256 * sb;
        st.x[m][0] = *reinterpret_cast<const u32x4 *>(xp + run0);
        st.x[m][1] = *reinterpret_cast<const u32x4 *>(xp + run0 + 8);
        st.x[m][2] = *reinterpret_cast<const u32x4 *>(xp + run1);
        st.x[m][3] = *reinterpret_cast<const u32x4 *>(xp + run1 + 8);
    }
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
        if constexpr (TYPE == kQ4K) {
            const uint8_t *blk = wrow[rs] + sb * kQ4KBytes;
            st.q[rs] = *reinterpret_cast<const u32x4 *>(blk + 16 + 16 * p);
            st.h[rs] = *reinterpret_cast<const u32x4 *>(blk);
            st.s[rs] = 0;
        } else {
            const uint8_t *blk = wrow[rs] + sb * kQ6KBytes;
            const int hh = p >> 2, pg = (p >> 1) & 1, hf = p & 1;
            st.q[rs] = load16_align2(blk + 64 * hh + 32 * pg + 16 * hf);
            st.h[rs] = load16_align2(blk + 128 + 32 * hh + 16 * hf);
            const uint32_t d = *reinterpret_cast<const uint16_t *>(blk + 208);
            st.s[rs] = d | ((uint32_t)blk[192 + 8 * hh + 2 * pg + hf] << 16) |
                       ((uint32_t)blk[192 + 8 * hh + 2 * pg + 4 + hf] << 24);
        }
    }
}

// get_scale_min_k4 for a lane-dependent sub-block g, without branches.
__device__ __forceinline__ void scale_min_k4_any(uint32_t g, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc,
                                                 uint32_t &m) {
    const uint32_t sh = 8u * (g & 3u);
    const uint32_t sc_lo = __builtin_amdgcn_ubfe(s0, sh, 6), m_lo = __builtin_amdgcn_ubfe(s1, sh, 6);
    const uint32_t sc_hi = __builtin_amdgcn_ubfe(s2, sh, 4) | (__builtin_amdgcn_ubfe(s0, sh + 6, 2) << 4);
    const uint32_t m_hi = __builtin_amdgcn_ubfe(s2, sh + 4, 4) | (__builtin_amdgcn_ubfe(s1, sh + 6, 2) << 4);
    sc = g < 4 ? sc_lo : sc_hi;
    m = g < 4 ? m_lo : m_hi;
}

template <uint32_t TYPE, int MAXM, int RS>
__device__ __forceinline__ void compute_stage(const Stage<TYPE, MAXM, RS> &st, float (&acc)[RS][MAXM], int p) {
    XRun xa[MAXM], xb[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        make_run(xa[m], st.x[m][0], st.x[m][1]);
        make_run(xb[m], st.x[m][2], st.x[m][3]);
    }
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
        uint32_t la[4], lb[4], ha[4], hb[4];
        const uint32_t qw[4] = {st.q[rs].x, st.q[rs].y, st.q[rs].z, st.q[rs].w};
        if constexpr (TYPE == kQ4K) {
            const u32x4 hd = st.h[rs];
            const float d = half_to_float(hd.x), dmin = half_to_float(hd.x >> 16);
            const uint32_t g0 = 2 * (uint32_t)(p >> 1);
            uint32_t sc0, m0, sc1, m1;
            scale_min_k4_any(g0, hd.y, hd.z, hd.w, sc0, m0);
            scale_min_k4_any(g0 + 1, hd.y, hd.z, hd.w, sc1, m1);
            const float a0 = d * (float)sc0, b0 = dmin * (float)m0;
            const float a1 = d * (float)sc1, b1 = dmin * (float)m1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                la[i] = (qw[i] & 0x000f000fu) | 0x43004300u;
                lb[i] = ((qw[i] >> 8) & 0x000f000fu) | 0x43004300u;
                ha[i] = ((qw[i] >> 4) & 0x000f000fu) | 0x43004300u;
                hb[i] = ((qw[i] >> 12) & 0x000f000fu) | 0x43004300u;
            }
            // a * sum x q - b * sum x = a * sum x (128 + q) - (128 a + b) * sum x
            const float c0 = __builtin_fmaf(128.f, a0, b0), c1 = __builtin_fmaf(128.f, a1, b1);
#pragma unroll
            for (int m = 0; m < MAXM; ++m) {
                const float s0 = run_dot(xa[m], la, lb, 0.f), s1 = run_dot(xb[m], ha, hb, 0.f);
                float r = acc[rs][m];
                r = __builtin_fmaf(a0, s0, r);
                r = __builtin_fmaf(-c0, xa[m].s, r);
                r = __builtin_fmaf(a1, s1, r);
                r = __builtin_fmaf(-c1, xb[m].s, r);
                acc[rs][m] = r;
            }
        } else {
            const uint32_t pg = (uint32_t)(p >> 1) & 1u;
            const float d = half_to_float(st.s[rs]);
            const float a0 = d * (float)(int8_t)(uint8_t)(st.s[rs] >> 16);
            const float a1 = d * (float)(int8_t)(uint8_t)(st.s[rs] >> 24);
            const uint32_t hw[4] = {st.h[rs].x, st.h[rs].y, st.h[rs].z, st.h[rs].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t h0 = ((hw[i] >> (2 * pg)) & 0x03030303u) << 4;      // top bits, sub-block pg
                const uint32_t h1 = ((hw[i] >> (2 * pg + 4)) & 0x03030303u) << 4;  // top bits, sub-block pg + 2
                const uint32_t c0 = (qw[i] & 0x0f0f0f0fu) | h0, c1 = ((qw[i] >> 4) & 0x0f0f0f0fu) | h1;
                la[i] = (c0 & 0x00ff00ffu) | 0x43004300u;
                lb[i] = ((c0 >> 8) & 0x00ff00ffu) | 0x43004300u;
                ha[i] = (c1 & 0x00ff00ffu) | 0x43004300u;
                hb[i] = ((c1 >> 8) & 0x00ff00ffu) | 0x43004300u;
            }
            // a * sum x (code - 32) = a * (sum x (128 + code) - 160 sum x)
#pragma unroll
            for (int m = 0; m < MAXM; ++m) {
                const float s0 = run_dot(xa[m], la, lb, -160.f * xa[m].s);
                const float s1 = run_dot(xb[m], ha, hb, -160.f * xb[m].s);
                float r = acc[rs][m];
                r = __builtin_fmaf(a0, s0, r);
                r = __builtin_fmaf(a1, s1, r);
                acc[rs][m] = r;
            }
        }
    }
}

template <uint32_t TYPE, int MAXM, int RS>
__global__ __launch_bounds__(max_waves<MAXM>() * 64) void k_gemv(const uint16_t *__restrict__ x, int64_t x_stride, int M,
                                                      const uint8_t *__restrict__ w, int64_t w_pitch, int N,
                                                      int nsb, int KW, uint16_t *__restrict__ y, int64_t y_stride,
                                                      const uint16_t *__restrict__ bias) {
    constexpr int R = 8 * RS;
    __shared__ float red[max_waves<MAXM>()][R][MAXM];
    const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63, team = lane >> 3, p = lane & 7;
    const int n0 = (int)blockIdx.x * R;

    const uint8_t *wrow[RS];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) wrow[rs] = w + (int64_t)min(n0 + 8 * rs + team, N - 1) * w_pitch;
    const uint16_t *xrow[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) xrow[m] = x + (int64_t)min(m, M - 1) * x_stride;

    float acc[RS][MAXM];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
        for (int m = 0; m < MAXM; ++m) acc[rs][m] = 0.f;

    // Per-lane piece geometry (see tc_device.h for the block layouts).
    int run0, run1;      // K offsets (within the block) of the two 16-wide runs
    if constexpr (TYPE == kQ4K) {
        run0 = 64 * (p >> 1) + 16 * (p & 1);
        run1 = run0 + 32;
    } else {
        run0 = 128 * (p >> 2) + 32 * ((p >> 1) & 1) + 16 * (p & 1);
        run1 = run0 + 64;
    }

    // This wavefront's super-blocks are wave, wave + KW, ...; all loads of one block are
    // issued together, and latency is hidden by the other resident wavefronts.
    for (int sb = wave; sb < nsb; sb += KW) {
        Stage<TYPE, MAXM, RS> st;
        load_stage<TYPE, MAXM, RS>(st, xrow, wrow, sb, run0, run1, p);
        compute_stage<TYPE, MAXM, RS>(st, acc, p);
    }

    // Team reduction (8 lanes), then across wavefronts through LDS.
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            float v = acc[rs][m];
            v += __shfl_xor(v, 1);
            v += __shfl_xor(v, 2);
            v += __shfl_xor(v, 4);
            if (p == 0) red[wave][8 * rs + team][m] = v;
        }
    __syncthreads();
    for (int o = tid; o < R * MAXM; o += (int)blockDim.x) {
        const int r = o / MAXM, m = o % MAXM, n = n0 + r;
        if (n >= N || m >= M) continue;
        float v = 0.f;
        for (int k = 0; k < KW; ++k) v += red[k][r][m];
        uint32_t out = float_to_bf16_bits(v);
        if (bias) out = float_to_bf16_bits(bf16_to_float(out) + bf16_to_float(bias[n]));
        y[(int64_t)m * y_stride + n] = (uint16_t)out;
    }
}

template <uint32_t TYPE, int MAXM, int RS>
hipError_t launch_rs(const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K, uint16_t *y,
                     int64_t y_stride, const uint16_t *bias, hipStream_t stream) {
    const int nsb = K / 256, KW = nsb < max_waves<MAXM>() ? nsb : max_waves<MAXM>();
    const int64_t pitch = (int64_t)nsb * (TYPE == kQ4K ? kQ4KBytes : kQ6KBytes);
    const dim3 grid((unsigned)((N + 8 * RS - 1) / (8 * RS))), block((unsigned)(64 * KW));
    hipLaunchKernelGGL((k_gemv<TYPE, MAXM, RS>), grid, block, 0, stream, x, x_stride, M, w, pitch, N, nsb, KW, y,
                       y_stride, bias);
    return hipGetLastError();
}

// Rows per workgroup: 32 while every wavefront has at most one super-block of K to cover;
// 16 for longer K, which doubles the number of wavefronts in flight.
template <uint32_t TYPE, int MAXM>
hipError_t launch_t(const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K, uint16_t *y,
                    int64_t y_stride, const uint16_t *bias, hipStream_t stream) {
    if (K / 256 <= max_waves<MAXM>())
        return launch_rs<TYPE, MAXM, 4>(x, x_stride, M, w, N, K, y, y_stride, bias, stream);
    return launch_rs<TYPE, MAXM, 2>(x, x_stride, M, w, N, K, y, y_stride, bias, stream);
}

template <uint32_t TYPE>
hipError_t launch_m(const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K, uint16_t *y,
                    int64_t y_stride, const uint16_t *bias, hipStream_t stream) {
    if (M <= 1) return launch_t<TYPE, 1>(x, x_stride, M, w, N, K, y, y_stride, bias, stream);
    if (M <= 2) return launch_t<TYPE, 2>(x, x_stride, M, w, N, K, y, y_stride, bias, stream);
    if (M <= 4) return launch_t<TYPE, 4>(x, x_stride, M, w, N, K, y, y_stride, bias, stream);
    return launch_t<TYPE, 8>(x, x_stride, M, w, N, K, y, y_stride, bias, stream);
}

}  // namespace

hipError_t launch_gemv(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                       uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, hipStream_t stream) {
    if (type == kQ4K) return launch_m<kQ4K>(x, x_stride, M, w, N, K, y, y_stride, bias_bf16, stream);
    return launch_m<kQ6K>(x, x_stride, M, w, N, K, y, y_stride, bias_bf16, stream);
}

}  // namespace tc
