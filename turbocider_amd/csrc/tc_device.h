// Device helpers for the GGUF K-quant kernels (gfx950 / CDNA4, wave64).
//
// Block layouts (native/core/gguf_decode.cpp:77-105, ggml block_q4_K / block_q6_K):
//   Q4_K (144 B): d fp16 @0, dmin fp16 @2, 12 bytes of packed 6-bit scales/mins @4,
//                 qs[128] @16. Weight 32g+j (g = sub-block 0..7, j = 0..31) uses the
//                 low nibble of qs[32*(g/2)+j] when g is even, the high nibble when odd.
//                 w = (d*sc_g)*q - dmin*m_g.
//   Q5_K (176 B): as Q4_K with qh[32] @16 (bit g of qh[j] is the 5th bit) and qs @48.
//   Q6_K (210 B): ql[128] @0, qh[64] @128, int8 scales[16] @192, d fp16 @208.
//                 Weight 128h+32g+j (h = 0..1, g = 0..3): low 4 bits from ql[64h+32(g&1)+j]
//                 (low nibble if g < 2), top 2 bits (qh[32h+j] >> 2g) & 3,
//                 w = (d*sc[8h+2g+j/16]) * (code-32).
// Every product above is exact in fp32 (d has <= 11 significant bits, sc/m <= 8 bits,
// codes <= 6 bits), so fma(a, q, -b) rounds exactly once, like the reference's
// mul-then-sub compiled with contraction off.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tc {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t kQ4K = 12, kQ5K = 13, kQ6K = 14;
constexpr uint32_t kQ4KBytes = 144, kQ5KBytes = 176, kQ6KBytes = 210;
// The other registered types (native/core/gguf_directory.hpp:21-26): F32 / F16 / BF16
// elements and the 32-weight Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0 blocks.
constexpr uint32_t kF32 = 0, kF16 = 1, kBF16 = 30, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8;

// Error flag bits written by kernels (atomicOr into a device word).
constexpr int kErrNonfinite = 1;       // non-finite d / dmin / scale, or non-finite element
constexpr int kErrF16Overflow = 2;     // fp16 target overflow
constexpr int kErrBF16Overflow = 4;    // bf16 target overflow (float sources only)
constexpr int kErrSourceFloat = 8;     // non-finite element on the same-dtype copy path

// fp16 bit pattern -> fp32 (v_cvt_f32_f16; fp16 denormals are preserved on gfx9 by default,
// which the golden vectors with d = 2^-24 check).
__device__ __forceinline__ float half_to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}
__device__ __forceinline__ bool half_finite(uint32_t bits) { return (bits & 0x7c00u) != 0x7c00u; }

__device__ __forceinline__ float bf16_to_float(uint32_t bits) {
    return __builtin_bit_cast(float, (bits & 0xffffu) << 16);
}
// Round-to-nearest-even fp32 -> bf16 bit pattern (gguf_decode.cpp:389-394 without the error
// path; callers only pass finite values whose bf16 rounding cannot overflow).
__device__ __forceinline__ uint32_t float_to_bf16_bits(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}
// Two fp32 -> packed bf16 pair, RNE (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Output activations of a projection (kActNone / kActGeluTanh / kActSiluGlu, tc_kernels.h),
// applied to the projection's bf16 outputs (after the bias) in fp32 and rounded once (RNE):
//   GELU, tanh form: 0.5 z (1 + tanh(sqrt(2/pi) (z + 0.044715 z^3)))
//     (native/models/qwen21/transformer.cpp:48-57);
//   SiLU-gated pair: silu(g) u = g u / (1 + exp(-g)) (native/backends/mlx.cpp:1627-1631 with
//     the gate/up product of native/models/qwen21/transformer.cpp:973-975).
// v * sigmoid(t) in fp32 without overflow or cancellation: v / (1 + exp(-t)) for t >= 0,
// v e / (1 + e) with e = exp(t) for t < 0, so that values in the fp32 / bf16 subnormal range
// (far negative t) come out as such instead of as zero.
__device__ __forceinline__ float times_sigmoid(float v, float t) {
    if (t >= 0.f) return v / (1.f + expf(-t));
    const float e = expf(t);
    return v * e / (1.f + e);
}
// GELU is evaluated as z sigmoid(2u), u = sqrt(2/pi) (z + 0.044715 z^3), which equals the tanh
// form (1 + tanh(u) = 2 sigmoid(2u)) without its cancellation for negative z (there 1 + tanh(u)
// in fp32 keeps few correct bits); a few fp32 ulps from the exact value everywhere.
__device__ __forceinline__ uint32_t gelu_tanh_bits(uint32_t z_bits) {
    const float z = bf16_to_float(z_bits);
    return float_to_bf16_bits(times_sigmoid(z, 1.5957691216057308f * (z + 0.044715f * (z * z * z))));
}
// silu(g) u = (g u) sigmoid(g), with g u exact in fp32 (two bf16 values). Where sigmoid(g) rounds
// to 1 in fp32 (g above about 16.6) the exact result is g u (1 - e), e = exp(-g) / (1 + exp(-g))
// > 0, just below |g u| in magnitude: a g u that sits exactly halfway between two bf16 values
// (frequent, a product of two 8-bit significands) then rounds toward zero, as the exact value
// does, instead of to even.
__device__ __forceinline__ uint32_t silu_glu_bits(uint32_t g_bits, uint32_t u_bits) {
    const float g = bf16_to_float(g_bits), p = g * bf16_to_float(u_bits);
    if (g >= 0.f) {
        const float d = 1.f + expf(-g);
        if (d == 1.f) {
            const uint32_t b = __builtin_bit_cast(uint32_t, p);
            return (b & 0xffffu) == 0x8000u ? b >> 16 : float_to_bf16_bits(p);
        }
        return float_to_bf16_bits(p / d);
    }
    const float e = expf(g);
    return float_to_bf16_bits(p * e / (1.f + e));
}
// Stores the finished bf16 outputs out[0..3] of columns col .. col + 3 (col % 4 == 0, N the
// row's width before the activation) into row `yrow` with output activation `act` (values 0,
// 1, 2 as kActNone, kActGeluTanh, kActSiluGlu of tc_kernels.h): kActSiluGlu writes columns
// col / 2 and col / 2 + 1. `vec`: yrow + col is 8-byte aligned (4-byte for the pair).
__device__ __forceinline__ void store_out4(uint16_t *yrow, int col, int N, const uint32_t out[4], bool vec, int act) {
    const bool full = col + 3 < N;
    if (act == 2) {
        const uint32_t h0 = silu_glu_bits(out[0], out[1]), h1 = silu_glu_bits(out[2], out[3]);
        uint16_t *yr = yrow + (col >> 1);
        if (vec && full) {
            *reinterpret_cast<uint32_t *>(yr) = h0 | (h1 << 16);
        } else {
            if (col + 1 < N) yr[0] = (uint16_t)h0;
            if (col + 3 < N) yr[1] = (uint16_t)h1;
        }
        return;
    }
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = act == 1 ? gelu_tanh_bits(out[c]) : out[c];
    uint16_t *yr = yrow + col;
    if (vec && full) {
        *reinterpret_cast<u32x2 *>(yr) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (col + c < N) yr[c] = (uint16_t)o[c];
    }
}

// fp32 -> fp16 RNE with subnormals; returns false when the value does not fit
// (gguf_decode.cpp:395-405).
__device__ __forceinline__ uint32_t round_right_even(uint32_t value, uint32_t shift) {
    const uint32_t q = value >> shift, rem = value & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}
__device__ __forceinline__ bool float_to_half_bits(float v, uint32_t &out) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v), mant = b & 0x7fffffu;
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 255u) - 127;
    if (e == 128) return false;
    if (e < -25) { out = sign; return true; }
    if (e > 15) return false;
    if (e < -14) { out = sign | round_right_even(0x800000u | mant, (uint32_t)(-e - 1)); return true; }
    const uint32_t r = (uint32_t)(e + 15) * 1024u + round_right_even(mant, 13);
    if (r >= 0x7c00u) return false;
    out = sign | r;
    return true;
}

// get_scale_min_k4 (gguf_decode.cpp:48-54) over the 12 packed bytes held as three dwords
// s0 = bytes 0..3, s1 = bytes 4..7, s2 = bytes 8..11.
__device__ __forceinline__ void scale_min_k4(uint32_t g, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc,
                                             uint32_t &m) {
    if (g < 4) {
        sc = (s0 >> (8 * g)) & 63u;
        m = (s1 >> (8 * g)) & 63u;
    } else {
        const uint32_t i = g - 4;
        sc = ((s2 >> (8 * i)) & 15u) | (((s0 >> (8 * i + 6)) & 3u) << 4);
        m = ((s2 >> (8 * i + 4)) & 15u) | (((s1 >> (8 * i + 6)) & 3u) << 4);
    }
}

// Hides a value's known bits from the optimizer (no instruction is emitted). Used on
// nibble-masked words so that byte-to-float conversions select v_cvt_f32_ubyte{0..3}
// instead of a bit-field extract followed by v_cvt_f32_ubyte0.
__device__ __forceinline__ uint32_t launder(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

// Byte-granular little-endian loads for sources with no alignment guarantee.
__device__ __forceinline__ uint32_t load_u16_any(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}
__device__ __forceinline__ uint32_t load_u32_any(const uint8_t *p) {
    if ((reinterpret_cast<uintptr_t>(p) & 3u) == 0) return *reinterpret_cast<const uint32_t *>(p);
    if ((reinterpret_cast<uintptr_t>(p) & 1u) == 0) {
        const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
        return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
    }
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// 16 bytes at an address that is at least 2-byte aligned (every field of a Q6_K block),
// assembled from a dword-aligned 16-byte load at p rounded down to 4 plus one trailing
// dword. The trailing dword is read from base + 16 only when p is 2 mod 4 (the bytes
// p - 2 .. p + 18 must then be readable); otherwise it re-reads base, so no byte outside
// [p, p + 16) rounded to dwords is touched.
__device__ __forceinline__ u32x4 load16_align2(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *base = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
    typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(base);
    const uint32_t sh = (uint32_t)(a & 2u);
    const uint32_t e = base[sh ? 4 : 0];
    return u32x4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                 __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh)};
}

}  // namespace tc
