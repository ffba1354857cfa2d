// Standalone decode of every registered GGUF type (the device replacement of
// tc::gguf::decode_cpu_into, native/core/gguf_decode.cpp:56-158,320-367,433-465), the device
// quantizer, the load-time scale scan and the bias cast.
//
// K-quant work split: one wavefront per (target row, super-block); lane t produces the
// 4 consecutive weights 4t..4t+3 of the 256-weight block, which always share one
// sub-block scale. Full in-slice quads with a dense target are written with one 8-byte
// (bf16/f16) or 16-byte (f32) store; slice edges and strided targets use per-element
// stores. Source loads are dword loads when the source is dword aligned (Q4_K / Q5_K
// tensors whose base is), otherwise 2-byte loads (Q6_K blocks are 210 bytes apart).
#include "tc_device.h"
#include "tc_kernels.h"

namespace tc {
namespace {

// Decode weights 4t..4t+3 of one super-block into v[0..3]; returns false if the block's
// fp16 master scale(s) are not finite.
template <uint32_t TYPE>
__device__ __forceinline__ bool decode_quad(const uint8_t *blk, uint32_t t, float v[4]) {
    const uint32_t e0 = 4 * t;
    if constexpr (TYPE == kQ4K || TYPE == kQ5K) {
        const uint32_t dd = load_u32_any(blk);
        if (!half_finite(dd) || !half_finite(dd >> 16)) return false;
        const float d = half_to_float(dd), dmin = half_to_float(dd >> 16);
        const uint32_t g = e0 / 32, j0 = e0 % 32;
        uint32_t sc, m;
        scale_min_k4(g, load_u32_any(blk + 4), load_u32_any(blk + 8), load_u32_any(blk + 12), sc, m);
        const float a = d * (float)sc, b = dmin * (float)m;
        const uint32_t qs = load_u32_any(blk + (TYPE == kQ5K ? 48 : 16) + (g / 2) * 32 + j0);
        const uint32_t nib = (g & 1) ? (qs >> 4) : qs;
        uint32_t hi = 0;
        if constexpr (TYPE == kQ5K) hi = load_u32_any(blk + 16 + j0) >> g;  // bit g of each byte
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t code = (nib >> (8 * i)) & 15u;
            if constexpr (TYPE == kQ5K) code |= ((hi >> (8 * i)) & 1u) << 4;
            v[i] = __builtin_fmaf(a, (float)code, -b);
        }
    } else {
        const uint32_t dbits = load_u16_any(blk + 208);
        if (!half_finite(dbits)) return false;
        const float d = half_to_float(dbits);
        const uint32_t h = e0 / 128, g = (e0 % 128) / 32, j0 = e0 % 32;
        const uint32_t ql = load_u32_any(blk + h * 64 + (g & 1) * 32 + j0);
        const uint32_t qh = load_u32_any(blk + 128 + h * 32 + j0);
        const int sc = (int)(int8_t)blk[192 + h * 8 + 2 * g + j0 / 16];
        const float a = d * (float)sc;
        const uint32_t lo = (g < 2) ? ql : (ql >> 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int code = (int)(((lo >> (8 * i)) & 15u) | (((qh >> (8 * i + 2 * g)) & 3u) << 4)) - 32;
            v[i] = a * (float)code;
        }
    }
    return true;
}

// Error reporting of the decode kernels: err[0] holds kErr* flags; the two 64-bit words at
// err + 2 hold the first (lowest) target position r * columns + column of a non-finite
// value error and of a conversion overflow, so that the host reports whichever the
// reference, which decodes row by row and column by column, would have met first.
__device__ __forceinline__ void report(int *err, int flag, int which, uint64_t position) {
    atomicOr(err, flag);
    atomicMin(reinterpret_cast<unsigned long long *>(err + 2) + which, (unsigned long long)position);
}

// Writes v[0..3], the values of source columns c0 .. c0 + 3, to the slice [column_begin, end)
// of one target row (target positions rpos + column - column_begin): one 8-byte (bf16 / f16)
// or 16-byte (f32) store for a full in-slice quad with a dense, aligned target, else per
// element. CHECK_BF16: flag a bf16 rounding to infinity (only a float source can reach it).
template <bool CHECK_BF16>
__device__ __forceinline__ void store_quad(const float v[4], uint64_t c0, uint64_t column_begin, uint64_t end,
                                           uint8_t *row, uint64_t col_stride, uint32_t dtype, int *err,
                                           uint64_t rpos) {
    const uint64_t isz = dtype == 0 ? 4 : 2;
    const bool full = c0 >= column_begin && c0 + 4 <= end && col_stride == isz;
    uint8_t *p0 = row + (c0 - column_begin) * col_stride;  // only dereferenced when in slice
    if (dtype == 2) {
        if constexpr (CHECK_BF16) {
            for (int i = 0; i < 4; ++i)
                if (c0 + i >= column_begin && c0 + i < end && (float_to_bf16_bits(v[i]) & 0x7f80u) == 0x7f80u) {
                    report(err, kErrBF16Overflow, 1, rpos + c0 + i - column_begin);
                    break;
                }
        }
        if (full && (reinterpret_cast<uintptr_t>(p0) & 7u) == 0) {
            *reinterpret_cast<u32x2 *>(p0) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            return;
        }
        for (int i = 0; i < 4; ++i)
            if (c0 + i >= column_begin && c0 + i < end) {
                const uint32_t h = float_to_bf16_bits(v[i]);
                uint8_t *p = row + (c0 + i - column_begin) * col_stride;
                p[0] = (uint8_t)h;
                p[1] = (uint8_t)(h >> 8);
            }
    } else if (dtype == 0) {
        if (full && (reinterpret_cast<uintptr_t>(p0) & 15u) == 0) {
            *reinterpret_cast<f32x4 *>(p0) = f32x4{v[0], v[1], v[2], v[3]};
            return;
        }
        for (int i = 0; i < 4; ++i)
            if (c0 + i >= column_begin && c0 + i < end) {
                const uint32_t u = __builtin_bit_cast(uint32_t, v[i]);
                uint8_t *p = row + (c0 + i - column_begin) * col_stride;
                p[0] = (uint8_t)u; p[1] = (uint8_t)(u >> 8); p[2] = (uint8_t)(u >> 16); p[3] = (uint8_t)(u >> 24);
            }
    } else {
        uint32_t h[4];
        int bad = -1;
        for (int i = 0; i < 4; ++i) {
            h[i] = 0;
            if (c0 + i >= column_begin && c0 + i < end && !float_to_half_bits(v[i], h[i]) && bad < 0) bad = i;
        }
        if (bad >= 0) report(err, kErrF16Overflow, 1, rpos + c0 + bad - column_begin);
        if (full && (reinterpret_cast<uintptr_t>(p0) & 7u) == 0) {
            *reinterpret_cast<u32x2 *>(p0) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            return;
        }
        for (int i = 0; i < 4; ++i)
            if (c0 + i >= column_begin && c0 + i < end) {
                uint8_t *p = row + (c0 + i - column_begin) * col_stride;
                p[0] = (uint8_t)h[i];
                p[1] = (uint8_t)(h[i] >> 8);
            }
    }
}

template <uint32_t TYPE, uint32_t BLOCK_BYTES>
__global__ __launch_bounds__(256) void k_decode(const uint8_t *__restrict__ src, uint64_t row_bytes,
                                                const uint64_t *__restrict__ rows_idx, uint64_t row_begin,
                                                uint64_t rows, uint64_t first_block, uint64_t nblk,
                                                uint64_t column_begin, uint64_t columns, uint8_t *__restrict__ dst,
                                                uint64_t row_stride, uint64_t col_stride, uint32_t dtype,
                                                int *__restrict__ err) {
    const uint64_t item = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= rows * nblk) return;
    const uint64_t r = item / nblk, b = first_block + item % nblk;
    const uint64_t srow = rows_idx ? rows_idx[r] : row_begin + r;
    const uint8_t *blk = src + srow * row_bytes + b * BLOCK_BYTES;
    const uint32_t t = threadIdx.x & 63;
    float v[4];
    if (!decode_quad<TYPE>(blk, t, v)) {  // the whole block fails, at its first column in the slice
        if (t == 0) report(err, kErrNonfinite, 0, r * columns + max(b * 256, column_begin) - column_begin);
        return;
    }
    store_quad<false>(v, b * 256 + 4 * t, column_begin, column_begin + columns, dst + r * row_stride, col_stride,
                      dtype, err, r * columns);
}

// The other registered types: source columns c0 .. c0 + 3 of one row (c0 % 4 == 0; a quad
// never straddles a 32-weight block). Columns at or past `ncols` are not read (v = 0).
// Returns the non-finite mask: bit i for a non-finite element i (float types), all four bits
// for a non-finite scale / minimum (block types: the whole block fails). The expressions are
// gguf_decode.cpp:56-76; every product code * scale is exact in fp32, so
// fma(code, scale, minimum) is the reference's single rounding of the sum.
template <uint32_t TYPE>
__device__ __forceinline__ uint32_t decode_small_quad(const uint8_t *row, uint64_t c0, uint64_t ncols, float v[4]) {
    uint32_t bad = 0;
    if constexpr (TYPE == kF32 || TYPE == kF16 || TYPE == kBF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = 0.f;
            if (c0 + i >= ncols) continue;
            if constexpr (TYPE == kF32) {
                v[i] = __builtin_bit_cast(float, load_u32_any(row + 4 * (c0 + i)));
                if ((__builtin_bit_cast(uint32_t, v[i]) & 0x7f800000u) == 0x7f800000u) bad |= 1u << i;
            } else {
                const uint32_t bits = load_u16_any(row + 2 * (c0 + i));
                if constexpr (TYPE == kF16) {
                    if (!half_finite(bits)) bad |= 1u << i;
                    v[i] = half_to_float(bits);
                } else {
                    if ((bits & 0x7f80u) == 0x7f80u) bad |= 1u << i;
                    v[i] = bf16_to_float(bits);
                }
            }
        }
    } else {
        constexpr uint32_t kBytes = TYPE == kQ4_0 ? 18 : TYPE == kQ4_1 ? 20 : TYPE == kQ5_0 ? 22 : TYPE == kQ5_1 ? 24 : 34;
        const uint8_t *blk = row + (c0 / 32) * kBytes;
        const uint32_t e0 = (uint32_t)(c0 % 32);
        const uint32_t sbits = load_u16_any(blk);
        bool ok = half_finite(sbits);
        const float scale = half_to_float(sbits);
        if constexpr (TYPE == kQ8_0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = (float)(int8_t)blk[2 + e0 + i] * scale;
        } else {
            constexpr bool affine = TYPE == kQ4_1 || TYPE == kQ5_1, five = TYPE == kQ5_0 || TYPE == kQ5_1;
            float minimum = 0.f;
            if constexpr (affine) {
                const uint32_t mbits = load_u16_any(blk + 2);
                ok &= half_finite(mbits);
                minimum = half_to_float(mbits);
            }
            constexpr uint32_t offset = affine ? 4 : 2;
            const uint32_t high = five ? load_u32_any(blk + offset) : 0u;
            const uint8_t *low = blk + offset + (five ? 4 : 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t e = e0 + i;
                int code = e < 16 ? (low[e] & 15) : (low[e - 16] >> 4);
                if constexpr (five) code |= (int)((high >> e) & 1u) << 4;
                if constexpr (affine) {
                    v[i] = __builtin_fmaf((float)code, scale, minimum);
                } else {
                    code -= five ? 16 : 8;
                    v[i] = (float)code * scale;
                }
            }
        }
        if (!ok) bad = 15u;
    }
    return bad;
}

// One thread per quad of source columns [4 q, 4 q + 4) of one target row, q over the quads
// that meet the slice. `copy` (a float source into the same dtype with a dense target, the
// reference's checked byte copy, gguf_decode.cpp:119-158,327-331) only changes the error a
// non-finite element reports; the values written are the same bits either way.
template <uint32_t TYPE>
__global__ __launch_bounds__(256) void k_decode_small(const uint8_t *__restrict__ src, uint64_t row_bytes,
                                                      uint64_t ncols, const uint64_t *__restrict__ rows_idx,
                                                      uint64_t row_begin, uint64_t rows, uint64_t q_begin,
                                                      uint64_t nq, uint64_t column_begin, uint64_t columns,
                                                      uint8_t *__restrict__ dst, uint64_t row_stride,
                                                      uint64_t col_stride, uint32_t dtype, int copy,
                                                      int *__restrict__ err) {
    const uint64_t item = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (item >= rows * nq) return;
    const uint64_t r = item / nq, c0 = 4 * (q_begin + item % nq);
    const uint64_t srow = rows_idx ? rows_idx[r] : row_begin + r;
    float v[4];
    const uint64_t end = column_begin + columns;
    if (const uint32_t bad = decode_small_quad<TYPE>(src + srow * row_bytes, c0, ncols, v)) {
        // Block types: the block fails at its first column in the slice. Float types: the
        // first non-finite element in the slice (one outside it is never read by the
        // reference).
        constexpr bool block = !(TYPE == kF32 || TYPE == kF16 || TYPE == kBF16);
        if (block) {
            report(err, kErrNonfinite, 0, r * columns + max(c0 / 32 * 32, column_begin) - column_begin);
            return;
        }
        for (int i = 0; i < 4; ++i)
            if (((bad >> i) & 1u) && c0 + i >= column_begin && c0 + i < end) {
                report(err, copy ? kErrSourceFloat : kErrNonfinite, 0, r * columns + c0 + i - column_begin);
                return;
            }
    }
    store_quad<true>(v, c0, column_begin, end, dst + r * row_stride, col_stride, dtype, err, r * columns);
}

// ---------------------------------------------------------------------------------------
// Quantizers: the same steps, in the same fp32 order, as oracle/tc_oracle.c's
// oracle_quantize_q4_k_block / _q6_k_block (no reference counterpart). One thread per
// super-block; the work is tiny next to any use of the weights.
// ---------------------------------------------------------------------------------------
__device__ uint32_t half_bits_or_max(float v) {
    uint32_t h;
    return float_to_half_bits(v, h) ? h : 0x7bffu;
}

__device__ void quantize_q4k_block(const float *x, uint8_t *out) {
    float scale[8], minv[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) {
            lo = fminf(lo, x[32 * j + i]);
            hi = fmaxf(hi, x[32 * j + i]);
        }
        if (lo > 0.f) lo = 0.f;
        scale[j] = __fdiv_rn(__fsub_rn(hi, lo), 15.f);
        minv[j] = __fsub_rn(0.f, lo);  // +0 (never -0) for an all-non-negative sub-block
        max_scale = fmaxf(max_scale, scale[j]);
        max_min = fmaxf(max_min, minv[j]);
    }
    const uint32_t dh = half_bits_or_max(__fdiv_rn(max_scale, 63.f)), mh = half_bits_or_max(__fdiv_rn(max_min, 63.f));
    const float d = half_to_float(dh), dmin = half_to_float(mh);
    uint32_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        float s = d > 0.f ? rintf(__fdiv_rn(scale[j], d)) : 0.f, m = dmin > 0.f ? rintf(__fdiv_rn(minv[j], dmin)) : 0.f;
        ls[j] = (uint32_t)(s > 63.f ? 63.f : s);
        lm[j] = (uint32_t)(m > 63.f ? 63.f : m);
    }
    uint8_t blk[144];
    for (int i = 0; i < 144; ++i) blk[i] = 0;
    blk[0] = (uint8_t)dh; blk[1] = (uint8_t)(dh >> 8); blk[2] = (uint8_t)mh; blk[3] = (uint8_t)(mh >> 8);
    uint8_t *s = blk + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)(ls[j] | ((ls[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(lm[j] | ((lm[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((ls[j + 4] & 15) | ((lm[j + 4] & 15) << 4));
    }
    const uint32_t s0 = s[0] | (s[1] << 8) | (s[2] << 16) | ((uint32_t)s[3] << 24);
    const uint32_t s1 = s[4] | (s[5] << 8) | (s[6] << 16) | ((uint32_t)s[7] << 24);
    const uint32_t s2 = s[8] | (s[9] << 8) | (s[10] << 16) | ((uint32_t)s[11] << 24);
    for (int j = 0; j < 8; ++j) {
        uint32_t sc, m;
        scale_min_k4((uint32_t)j, s0, s1, s2, sc, m);
        const float a = __fmul_rn(d, (float)sc), b = __fmul_rn(dmin, (float)m);
        for (int i = 0; i < 32; ++i) {
            float q = 0.f;
            if (a > 0.f) {
                q = rintf(__fdiv_rn(__fadd_rn(x[32 * j + i], b), a));
                q = q < 0.f ? 0.f : (q > 15.f ? 15.f : q);
            }
            blk[16 + (j / 2) * 32 + i] |= (uint8_t)((int)q << ((j & 1) * 4));
        }
    }
    for (int i = 0; i < 144; i += 4)
        *reinterpret_cast<uint32_t *>(out + i) =
            blk[i] | (blk[i + 1] << 8) | (blk[i + 2] << 16) | ((uint32_t)blk[i + 3] << 24);
}

__device__ void quantize_q6k_block(const float *x, uint8_t *out) {
    float scale[16], max_abs_scale = 0.f, max_scale = 0.f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.f, vmax = 0.f;
        for (int i = 0; i < 16; ++i) {
            const float v = x[16 * j + i];
            if (fabsf(v) > amax) { amax = fabsf(v); vmax = v; }
        }
        scale[j] = __fdiv_rn(vmax, -32.f);
        if (fabsf(scale[j]) > max_abs_scale) { max_abs_scale = fabsf(scale[j]); max_scale = scale[j]; }
    }
    const uint32_t dh = half_bits_or_max(__fdiv_rn(max_scale, -127.f));
    const float d = half_to_float(dh);
    uint8_t blk[210];
    for (int i = 0; i < 210; ++i) blk[i] = 0;
    int sc[16];
    for (int j = 0; j < 16; ++j) {
        float s = d != 0.f ? rintf(__fdiv_rn(scale[j], d)) : 0.f;
        s = s > 127.f ? 127.f : (s < -128.f ? -128.f : s);
        sc[j] = (int)s;
        blk[192 + j] = (uint8_t)(int8_t)sc[j];
    }
    blk[208] = (uint8_t)dh; blk[209] = (uint8_t)(dh >> 8);
    for (int half = 0; half < 2; ++half)
        for (int g = 0; g < 4; ++g)
            for (int j = 0; j < 32; ++j) {
                const int idx = half * 128 + g * 32 + j;
                const float a = __fmul_rn(d, (float)sc[half * 8 + g * 2 + j / 16]);
                float q = 0.f;
                if (a != 0.f) {
                    q = rintf(__fdiv_rn(x[idx], a));
                    q = q < -32.f ? -32.f : (q > 31.f ? 31.f : q);
                }
                const int code = (int)q + 32;
                blk[half * 64 + j + (g & 1) * 32] |= (uint8_t)((code & 15) << ((g >> 1) * 4));
                blk[128 + half * 32 + j] |= (uint8_t)((code >> 4) << (2 * g));
            }
    for (int i = 0; i < 210; i += 2)
        *reinterpret_cast<uint16_t *>(out + i) = (uint16_t)(blk[i] | (blk[i + 1] << 8));
}

template <uint32_t TYPE>
__global__ __launch_bounds__(64) void k_quantize(const float *__restrict__ w, uint64_t nblocks, uint8_t *__restrict__ out) {
    const uint64_t b = (uint64_t)blockIdx.x * 64 + threadIdx.x;
    if (b >= nblocks) return;
    if constexpr (TYPE == kQ4K) quantize_q4k_block(w + b * 256, out + b * kQ4KBytes);
    else quantize_q6k_block(w + b * 256, out + b * kQ6KBytes);
}

template <uint32_t TYPE>
__global__ __launch_bounds__(256) void k_scan_scales(const uint8_t *__restrict__ w, uint64_t nblocks, int *err) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    bool ok;
    if constexpr (TYPE == kQ6K) {
        ok = half_finite(load_u16_any(w + b * kQ6KBytes + 208));
    } else {
        const uint32_t bytes = TYPE == kQ4K ? kQ4KBytes : kQ5KBytes;
        const uint32_t dd = load_u32_any(w + b * bytes);
        ok = half_finite(dd) && half_finite(dd >> 16);
    }
    if (!ok) atomicOr(err, kErrNonfinite);
}

__global__ __launch_bounds__(256) void k_bias_to_bf16(const void *__restrict__ bias, uint32_t dtype, uint64_t n,
                                                      uint16_t *__restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v;
    if (dtype == 0) v = reinterpret_cast<const float *>(bias)[i];
    else if (dtype == 1) v = half_to_float(reinterpret_cast<const uint16_t *>(bias)[i]);
    else v = bf16_to_float(reinterpret_cast<const uint16_t *>(bias)[i]);
    out[i] = (uint16_t)float_to_bf16_bits(v);
}

}  // namespace

hipError_t launch_decode(uint32_t type, const uint8_t *src, uint64_t row_bytes, uint64_t source_columns,
                         const uint64_t *d_rows, uint64_t row_begin, uint64_t rows, uint64_t column_begin,
                         uint64_t columns, uint8_t *dst, uint64_t row_stride, uint64_t col_stride, uint32_t dtype,
                         int copy, int *d_err, hipStream_t stream) {
    if (type == kQ4K || type == kQ5K || type == kQ6K) {
        const uint64_t first = column_begin / 256, last = (column_begin + columns - 1) / 256;
        const uint64_t nblk = last - first + 1, items = rows * nblk;
        const dim3 grid((unsigned)((items + 3) / 4)), block(256);
        if (type == kQ4K)
            hipLaunchKernelGGL((k_decode<kQ4K, kQ4KBytes>), grid, block, 0, stream, src, row_bytes, d_rows, row_begin,
                               rows, first, nblk, column_begin, columns, dst, row_stride, col_stride, dtype, d_err);
        else if (type == kQ5K)
            hipLaunchKernelGGL((k_decode<kQ5K, kQ5KBytes>), grid, block, 0, stream, src, row_bytes, d_rows, row_begin,
                               rows, first, nblk, column_begin, columns, dst, row_stride, col_stride, dtype, d_err);
        else
            hipLaunchKernelGGL((k_decode<kQ6K, kQ6KBytes>), grid, block, 0, stream, src, row_bytes, d_rows, row_begin,
                               rows, first, nblk, column_begin, columns, dst, row_stride, col_stride, dtype, d_err);
        return hipGetLastError();
    }
    const uint64_t q_begin = column_begin / 4, q_end = (column_begin + columns + 3) / 4, nq = q_end - q_begin;
    const dim3 grid((unsigned)((rows * nq + 255) / 256)), block(256);
#define TC_DECODE_SMALL(T)                                                                                     \
    hipLaunchKernelGGL((k_decode_small<T>), grid, block, 0, stream, src, row_bytes, source_columns, d_rows,     \
                       row_begin, rows, q_begin, nq, column_begin, columns, dst, row_stride, col_stride, dtype, \
                       copy, d_err)
    switch (type) {
    case kF32: TC_DECODE_SMALL(kF32); break;
    case kF16: TC_DECODE_SMALL(kF16); break;
    case kBF16: TC_DECODE_SMALL(kBF16); break;
    case kQ4_0: TC_DECODE_SMALL(kQ4_0); break;
    case kQ4_1: TC_DECODE_SMALL(kQ4_1); break;
    case kQ5_0: TC_DECODE_SMALL(kQ5_0); break;
    case kQ5_1: TC_DECODE_SMALL(kQ5_1); break;
    case kQ8_0: TC_DECODE_SMALL(kQ8_0); break;
    default: return hipErrorInvalidValue;
    }
#undef TC_DECODE_SMALL
    return hipGetLastError();
}

hipError_t launch_quantize(uint32_t type, const float *w, uint64_t rows, uint64_t cols, uint8_t *out,
                           hipStream_t stream) {
    const uint64_t nblocks = rows * (cols / 256);
    const dim3 grid((unsigned)((nblocks + 63) / 64)), block(64);
    if (type == kQ4K) hipLaunchKernelGGL(k_quantize<kQ4K>, grid, block, 0, stream, w, nblocks, out);
    else hipLaunchKernelGGL(k_quantize<kQ6K>, grid, block, 0, stream, w, nblocks, out);
    return hipGetLastError();
}

hipError_t launch_scan_scales(uint32_t type, const uint8_t *w, uint64_t nblocks, int *d_err, hipStream_t stream) {
    const dim3 grid((unsigned)((nblocks + 255) / 256)), block(256);
    if (type == kQ4K) hipLaunchKernelGGL(k_scan_scales<kQ4K>, grid, block, 0, stream, w, nblocks, d_err);
    else if (type == kQ5K) hipLaunchKernelGGL(k_scan_scales<kQ5K>, grid, block, 0, stream, w, nblocks, d_err);
    else hipLaunchKernelGGL(k_scan_scales<kQ6K>, grid, block, 0, stream, w, nblocks, d_err);
    return hipGetLastError();
}

hipError_t launch_bias_to_bf16(const void *bias, uint32_t dtype, uint64_t n, uint16_t *out, hipStream_t stream) {
    hipLaunchKernelGGL(k_bias_to_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, bias, dtype, n, out);
    return hipGetLastError();
}

}  // namespace tc
