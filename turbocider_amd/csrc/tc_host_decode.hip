// Host-pointer GGUF decode: tc_gguf_decode_host (include/tc_qlinear.h).
//
// The CPU counterpart of the device decoder, for callers that hold packed rows in host memory
// (the reference's CPU pager fills, native/runtime/streaming/gguf_weight_pager.cpp:347-349,
// 571-573). It keeps tc::gguf::decode_cpu_into / decode_cpu_gather's contract
// (native/core/gguf_decode.hpp:48-65, gguf_decode.cpp:160-183,320-367,433-465): the same
// geometry checks and messages in the same order, the same per-element arithmetic (one fp32
// rounding of the block expression, then RNE to the target type), errors in row / block / column
// order, cancellation checked on entry, before every block (every element of the same-dtype
// copy) and on exit, and the same receipt (a fixed 1024-byte block scratch; no vector path, so
// simd_blocks is 0 as on the reference's non-NEON build). Host code only; reentrant, no
// allocation: concurrent calls on disjoint targets may split a matrix by rows.
#include "../../include/tc_qlinear.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

#pragma clang fp contract(off)

namespace {

struct Stop : std::runtime_error {
    int status;
    Stop(const char *what, int s) : std::runtime_error(what), status(s) {}
};
[[noreturn]] void stop(const char *reason) { throw Stop(reason, 1); }
inline void need(bool ok, const char *reason) {
    if (!ok) stop(reason);
}
inline void poll(const volatile int *cancel) {
    if (cancel && *cancel) throw Stop("gguf_decode_cancelled", 2);
}
inline uint64_t mul(uint64_t a, uint64_t b) {
    need(a == 0 || b <= UINT64_MAX / a, "gguf_decode: multiplication overflow");
    return a * b;
}
inline uint64_t add(uint64_t a, uint64_t b) {
    need(b <= UINT64_MAX - a, "gguf_decode: addition overflow");
    return a + b;
}

constexpr const char *kNonfinite = "nonfinite weight/scale or conversion overflow";
constexpr uint32_t kBlockScratchBytes = 256 * sizeof(float);  // one decoded block

// Elements and bytes per block of each registered type (GGUF type table).
struct Layout {
    uint32_t elements, bytes;
};
Layout layout_of(uint32_t type) {
    switch (type) {
    case TC_GGML_TYPE_F32: return {1, 4};
    case TC_GGML_TYPE_F16: case TC_GGML_TYPE_BF16: return {1, 2};
    case TC_GGML_TYPE_Q4_0: return {32, 18};
    case TC_GGML_TYPE_Q4_1: return {32, 20};
    case TC_GGML_TYPE_Q5_0: return {32, 22};
    case TC_GGML_TYPE_Q5_1: return {32, 24};
    case TC_GGML_TYPE_Q8_0: return {32, 34};
    case TC_GGML_TYPE_Q4_K: return {256, 144};
    case TC_GGML_TYPE_Q5_K: return {256, 176};
    case TC_GGML_TYPE_Q6_K: return {256, 210};
    default: stop("gguf_decode: unsupported tensor type");
    }
}

inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
inline uint32_t le32(const uint8_t *p) { return (uint32_t)le16(p) | ((uint32_t)le16(p + 2) << 16); }
inline float bits_float(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}
inline uint32_t float_bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

// IEEE half -> float, exact for every encoding (subnormals scaled by 2^-24 in fp32, exact).
float half_value(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, frac = h & 0x3ff;
    if (exp == 0x1f) return bits_float(sign | 0x7f800000u | (frac << 13));
    if (exp == 0) {
        const float mag = (float)frac * 0x1p-24f;
        return sign ? -mag : mag;
    }
    return bits_float(sign | ((exp + 112) << 23) | (frac << 13));
}
inline float half_at(const uint8_t *p) { return half_value(le16(p)); }
inline void check_finite(float v) { need(std::isfinite(v), kNonfinite); }

// Round-to-nearest-even of a finite float to bf16 / fp16 bits; non-finite input and results
// that do not fit are errors.
uint16_t to_bf16(float v) {
    check_finite(v);
    const uint32_t b = float_bits(v);
    const uint32_t r = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
    need((r & 0x7f80u) != 0x7f80u, "BF16 conversion overflow");
    return (uint16_t)r;
}
uint16_t to_fp16(float v) {
    check_finite(v);
    const uint32_t b = float_bits(v);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const int e = (int)((b >> 23) & 0xff) - 127;
    const uint32_t mant = b & 0x7fffffu;
    auto rne = [](uint32_t value, uint32_t shift) {  // value >> shift, ties to even
        const uint32_t q = value >> shift, r = value & ((1u << shift) - 1), h = 1u << (shift - 1);
        return q + ((r > h || (r == h && (q & 1u))) ? 1u : 0u);
    };
    if (e < -25) return sign;  // below half the smallest subnormal
    need(e <= 15, "FP16 conversion overflow");
    if (e < -14) return (uint16_t)(sign | rne(0x800000u | mant, (uint32_t)(-e - 1)));  // subnormal
    const uint32_t h = ((uint32_t)(e + 15) << 10) + rne(mant, 13);  // a carry may round up the exponent
    need(h < 0x7c00u, "FP16 conversion overflow");
    return (uint16_t)(sign | h);
}

// The 6-bit scale and minimum of sub-block g of a K-quant block (12 packed bytes s):
// groups 0..3 keep the low 6 bits of s[g] / s[g + 4]; groups 4..7 take 4 bits from s[g + 4] and
// the top 2 bits of s[g - 4] / s[g].
inline void k_scale_min(const uint8_t *s, uint32_t g, uint32_t &sc, uint32_t &mn) {
    if (g < 4) {
        sc = s[g] & 63u;
        mn = s[g + 4] & 63u;
    } else {
        sc = (s[g + 4] & 0x0fu) | ((s[g - 4] >> 6) << 4);
        mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
}

// One block of `type` at p -> out[0 .. elements). Scales / minimums and every output must be
// finite.
void unpack_block(uint32_t type, const uint8_t *p, float *out) {
    switch (type) {
    case TC_GGML_TYPE_F32: out[0] = bits_float(le32(p)); break;
    case TC_GGML_TYPE_F16: out[0] = half_at(p); break;
    case TC_GGML_TYPE_BF16: out[0] = bits_float((uint32_t)le16(p) << 16); break;
    case TC_GGML_TYPE_Q8_0: {
        const float d = half_at(p);
        check_finite(d);
        for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)p[2 + i] * d;
        break;
    }
    case TC_GGML_TYPE_Q4_0: case TC_GGML_TYPE_Q4_1: case TC_GGML_TYPE_Q5_0: case TC_GGML_TYPE_Q5_1: {
        // 32 weights as 16 bytes of nibble pairs (weight i low, i + 16 high), Q5 with a 32-bit
        // word of fifth bits; symmetric types subtract the code midpoint, affine ones add a minimum.
        const bool affine = type == TC_GGML_TYPE_Q4_1 || type == TC_GGML_TYPE_Q5_1;
        const bool five = type == TC_GGML_TYPE_Q5_0 || type == TC_GGML_TYPE_Q5_1;
        const float d = half_at(p);
        check_finite(d);
        const float minimum = affine ? half_at(p + 2) : 0.f;
        check_finite(minimum);
        const uint8_t *q = p + (affine ? 4 : 2);
        const uint32_t fifth = five ? le32(q) : 0u;
        if (five) q += 4;
        const int mid = five ? 16 : 8;
        for (int i = 0; i < 16; ++i) {
            int lo = q[i] & 0x0f, hi = q[i] >> 4;
            if (five) {
                lo |= (int)((fifth >> i) & 1u) << 4;
                hi |= (int)((fifth >> (i + 16)) & 1u) << 4;
            }
            if (affine) {
                out[i] = (float)lo * d + minimum;
                out[i + 16] = (float)hi * d + minimum;
            } else {
                out[i] = (float)(lo - mid) * d;
                out[i + 16] = (float)(hi - mid) * d;
            }
        }
        break;
    }
    case TC_GGML_TYPE_Q4_K: case TC_GGML_TYPE_Q5_K: {
        // d, dmin, 12 bytes of packed 6-bit scales / minimums, [Q5_K: 32 bytes of fifth bits],
        // 128 bytes of nibbles: sub-block g (32 weights) uses byte run g / 2, low nibbles for even
        // g, high for odd. w = (d * sc) * q - dmin * m: both products exact, one rounding.
        const float d = half_at(p), dmin = half_at(p + 2);
        check_finite(d);
        check_finite(dmin);
        const bool five = type == TC_GGML_TYPE_Q5_K;
        const uint8_t *fifth = p + 16, *nib = p + (five ? 48 : 16);
        for (uint32_t g = 0; g < 8; ++g) {
            uint32_t sc, mn;
            k_scale_min(p + 4, g, sc, mn);
            const float a = d * (float)sc, b = dmin * (float)mn;
            const uint8_t *run = nib + 32 * (g >> 1);
            const int shift = (g & 1) ? 4 : 0;
            for (uint32_t j = 0; j < 32; ++j) {
                int q = (run[j] >> shift) & 0x0f;
                if (five && ((fifth[j] >> g) & 1u)) q += 16;
                out[32 * g + j] = a * (float)q - b;
            }
        }
        break;
    }
    case TC_GGML_TYPE_Q6_K: {
        // 128 bytes of low nibbles, 64 of 2-bit high parts, 16 int8 group scales, d last. Weight
        // 128 h + 32 g + j: low nibble of ql[64 h + 32 (g & 1) + j] (high nibble for g >= 2), high
        // bits (qh[32 h + j] >> 2 g) & 3, code - 32, scale sc[8 h + 2 g + j / 16]; (d * sc) * code.
        const float d = half_at(p + 208);
        check_finite(d);
        for (uint32_t h = 0; h < 2; ++h)
            for (uint32_t g = 0; g < 4; ++g)
                for (uint32_t j = 0; j < 32; ++j) {
                    const uint8_t lo = p[64 * h + 32 * (g & 1) + j];
                    const int code = (int)(((g < 2 ? lo : lo >> 4) & 0x0f) | (((p[128 + 32 * h + j] >> (2 * g)) & 3u) << 4)) - 32;
                    const float s = d * (float)(int8_t)p[192 + 8 * h + 2 * g + j / 16];
                    out[128 * h + 32 * g + j] = s * (float)code;
                }
        break;
    }
    default: stop("gguf_decode: unsupported tensor type");
    }
    const uint32_t n = layout_of(type).elements;
    for (uint32_t i = 0; i < n; ++i) check_finite(out[i]);
}

void store(uint8_t *dst, uint32_t dtype, float v) {
    if (dtype == TC_DTYPE_F32) {
        std::memcpy(dst, &v, 4);
    } else {
        const uint16_t h = dtype == TC_DTYPE_BF16 ? to_bf16(v) : to_fp16(v);
        std::memcpy(dst, &h, 2);
    }
}

struct Job {
    uint32_t type, dtype;
    Layout lay;
    const uint8_t *src;
    uint64_t source_rows, row_bytes;
    uint8_t *dst;
    uint64_t row_stride, column_stride, column_begin, columns;
    bool copy;  // a float source into its own dtype, dense columns: checked byte copy
    const volatile int *cancel;
};

// One target row from one source row; adds the row's figures to the receipt.
void decode_row(const Job &j, uint64_t source_row, uint64_t target_row, tc_decode_receipt &rc) {
    need(source_row < j.source_rows, "gather row out of bounds");
    const uint8_t *row = j.src + source_row * j.row_bytes;
    uint8_t *out = j.dst + target_row * j.row_stride;
    const uint64_t item = j.dtype == TC_DTYPE_F32 ? 4 : 2;
    if (j.copy) {
        const uint32_t w = j.lay.bytes;
        const uint32_t exp_mask = j.type == TC_GGML_TYPE_F32 ? 0x7f800000u : j.type == TC_GGML_TYPE_F16 ? 0x7c00u : 0x7f80u;
        const uint8_t *in = row + j.column_begin * w;
        for (uint64_t c = 0; c < j.columns; ++c) {
            poll(j.cancel);
            const uint32_t bits = w == 4 ? le32(in + c * w) : le16(in + c * w);
            need((bits & exp_mask) != exp_mask, "nonfinite source float");
            std::memcpy(out + c * w, in + c * w, w);
        }
        rc.source_bytes_processed = add(rc.source_bytes_processed, mul(j.columns, w));
        rc.bytes_written = add(rc.bytes_written, mul(j.columns, w));
    } else {
        float block[256];
        const uint64_t n = j.lay.elements, first = j.column_begin / n, last = (j.column_begin + j.columns - 1) / n;
        for (uint64_t b = first; b <= last; ++b) {
            poll(j.cancel);
            unpack_block(j.type, row + b * j.lay.bytes, block);
            const uint64_t lo = std::max(j.column_begin, b * n), hi = std::min(j.column_begin + j.columns, (b + 1) * n);
            for (uint64_t c = lo; c < hi; ++c) store(out + (c - j.column_begin) * j.column_stride, j.dtype, block[c - b * n]);
        }
        rc.source_bytes_processed = add(rc.source_bytes_processed, mul(last - first + 1, j.lay.bytes));
        rc.bytes_written = add(rc.bytes_written, mul(j.columns, item));
    }
    rc.elements_written = add(rc.elements_written, j.columns);
    rc.scratch_bytes = kBlockScratchBytes;
}

}  // namespace

extern "C" int tc_gguf_decode_host(uint32_t ggml_type, const void *source, uint64_t source_bytes, uint64_t source_rows,
                                   uint64_t source_columns, uint64_t row_begin, uint64_t rows, uint64_t column_begin,
                                   uint64_t columns, uint32_t dtype, void *target, uint64_t target_bytes,
                                   uint64_t row_stride, uint64_t column_stride, const uint64_t *row_indices,
                                   const volatile int *cancel, tc_decode_receipt *receipt, char **error) {
    if (error) *error = nullptr;
    if (receipt) std::memset(receipt, 0, sizeof *receipt);
    try {
        poll(cancel);
        if (!row_indices)
            need(row_begin <= source_rows && rows <= source_rows - row_begin, "row slice out of bounds");
        else
            need(row_begin == 0, "row_begin must be 0 for a gather");
        // Geometry (gguf_decode.cpp:160-183): type, storage, source shape, slice, sizes, strides,
        // pointer ranges, overlap.
        const Layout lay = layout_of(ggml_type);
        need(source && target, "null source/target storage");
        need(source_rows && source_columns && source_columns % lay.elements == 0, "invalid source geometry");
        need(rows && columns && column_begin <= source_columns && columns <= source_columns - column_begin,
             "invalid decode slice");
        const uint64_t row_bytes = mul(source_columns / lay.elements, lay.bytes);
        const uint64_t packed = mul(source_rows, row_bytes);
        need(packed <= source_bytes, "packed source too short");
        need(dtype <= TC_DTYPE_BF16, "gguf_decode: invalid target dtype");
        const uint64_t item = dtype == TC_DTYPE_F32 ? 4 : 2;
        need(column_stride >= item, "invalid/overlapping column stride");
        const uint64_t row_extent = add(mul(columns - 1, column_stride), item);
        need(row_stride >= row_extent, "invalid/overlapping row stride");
        const uint64_t extent = add(mul(rows - 1, row_stride), row_extent);
        need(extent <= target_bytes, "decode target too short");
        const uintptr_t s0 = reinterpret_cast<uintptr_t>(source), t0 = reinterpret_cast<uintptr_t>(target);
        need(packed <= UINTPTR_MAX - s0 && extent <= UINTPTR_MAX - t0, "pointer range overflow");
        need(s0 + packed <= t0 || t0 + extent <= s0, "packed source overlaps target");
        if (row_indices) {
            const uintptr_t i0 = reinterpret_cast<uintptr_t>(row_indices);
            const uint64_t ibytes = mul(rows, sizeof(uint64_t));
            need(ibytes <= UINTPTR_MAX - i0 && (i0 + ibytes <= t0 || t0 + extent <= i0), "gather indices overlap target");
            for (uint64_t r = 0; r < rows; ++r) need(row_indices[r] < source_rows, "gather row out of bounds");
        }
        Job j;
        j.type = ggml_type;
        j.dtype = dtype;
        j.lay = lay;
        j.src = static_cast<const uint8_t *>(source);
        j.source_rows = source_rows;
        j.row_bytes = row_bytes;
        j.dst = static_cast<uint8_t *>(target);
        j.row_stride = row_stride;
        j.column_stride = column_stride;
        j.column_begin = column_begin;
        j.columns = columns;
        j.copy = ((ggml_type == TC_GGML_TYPE_F32 && dtype == TC_DTYPE_F32) ||
                  (ggml_type == TC_GGML_TYPE_F16 && dtype == TC_DTYPE_F16) ||
                  (ggml_type == TC_GGML_TYPE_BF16 && dtype == TC_DTYPE_BF16)) &&
                 column_stride == lay.bytes;
        j.cancel = cancel;
        tc_decode_receipt rc{};
        for (uint64_t r = 0; r < rows; ++r) decode_row(j, row_indices ? row_indices[r] : row_begin + r, r, rc);
        poll(cancel);
        if (receipt) *receipt = rc;
        return 0;
    } catch (const Stop &e) {
        if (error) *error = strdup(e.what());
        return e.status;
    } catch (const std::exception &e) {
        if (error) *error = strdup(e.what());
        return 1;
    }
}
