/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the GGUF Q4_K/Q6_K quantized-linear path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or the timed CPU baseline). The product library
 * (turbocider_amd/libtc_qlinear.so) never links or calls it.
 *
 * It restates, in plain C, the arithmetic of the reference's ggml-derived decoder
 * (native/core/gguf_decode.cpp, pinned to llama.cpp 64e9bceb) so that the HIP kernels
 * can be checked bit-for-bit:
 *   - fp16 -> fp32 (gguf_decode.cpp:377-388), fp32 -> bf16 RNE (:389-394),
 *     fp32 -> fp16 RNE (:395-405), finite check (:43)
 *   - 6-bit scale/min unpack (:48-54)
 *   - F32 / F16 / BF16 elements (:56-58), Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0 blocks (:59-76),
 *     Q4_K / Q5_K decode (:77-90), Q6_K decode (:91-105), final finite check (:110)
 *   - checked geometry (:160-183), per-row slice decode (:320-367),
 *     decode_cpu_into / decode_cpu_gather (:433-465)
 * It is compiled with -ffp-contract=off like the reference (gguf_decode.cpp:5-7).
 *
 * Pins (tests/test_oracle_*.py): golden vectors written by the compiled reference
 * decoder (oracle/_ref), the exhaustive fp16 round trip and RNE tie KATs of
 * tests/native/test_gguf_execution.py:176-198, and an exact-rational closed form of
 * the K-quant expressions.
 *
 * The quantizers (oracle_quantize_q4_k / _q6_k) have no counterpart in the reference
 * (it ships no quantize_row_*): parity unpinned by design; they are pinned by
 * properties only (finite scales, bounded round-trip error, determinism, and
 * bit-identity with the product's GPU quantizer which implements the same steps).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OK 0
#define ORACLE_ERROR 1
#define ORACLE_CANCELLED 2

/* thread-local error text, like tc_gguf_test_error() (tests/native/gguf_core_probe.cpp:10,31) */
static __thread char g_error[256];
const char *oracle_error(void) { return g_error; }
static int fail(const char *reason) {
    snprintf(g_error, sizeof g_error, "%s", reason);
    return ORACLE_ERROR;
}

/* GGML type registry (native/core/gguf_directory.hpp:21-26): id, elements per block, bytes. */
typedef struct { uint32_t id, elements, bytes; } type_info;
static const type_info k_types[] = {{0, 1, 4},    {1, 1, 2},    {30, 1, 2},   {2, 32, 18},  {3, 32, 20},   {6, 32, 22},
                                    {7, 32, 24},  {8, 32, 34},  {12, 256, 144}, {13, 256, 176}, {14, 256, 210}};
static const type_info *find_type(uint32_t id) {
    for (size_t i = 0; i < sizeof k_types / sizeof k_types[0]; ++i)
        if (k_types[i].id == id) return &k_types[i];
    return NULL;
}

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* gguf_decode.cpp:377-388: exact fp16 decode incl. subnormals, inf and nan. */
float oracle_fp16_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exponent = (h >> 10) & 31, mantissa = h & 1023, bits;
    if (exponent == 0 && mantissa != 0) {
        int e = -14;
        while (!(mantissa & 1024)) { mantissa <<= 1; --e; }
        bits = sign | ((uint32_t)(e + 127) << 23) | ((mantissa & 1023) << 13);
    } else if (exponent == 0) {
        bits = sign;
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    }
    return u2f(bits);
}

/* gguf_decode.cpp:389-394: RNE to bf16; non-finite input or overflow to inf is an error. */
int oracle_float_to_bf16_rne(float v, uint16_t *out) {
    if (!isfinite(v)) return fail("nonfinite weight/scale or conversion overflow");
    uint32_t b = f2u(v);
    uint16_t r = (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
    if ((r & 0x7f80) == 0x7f80) return fail("BF16 conversion overflow");
    *out = r;
    return ORACLE_OK;
}

/* Unchecked bf16 RNE used by the epilogue restatement (native_lora_math_test.cpp:22-25). */
uint16_t oracle_bf16_bits(float v) {
    uint32_t b = f2u(v);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
static float bf16_value(uint16_t h) { return u2f((uint32_t)h << 16); }

static uint32_t round_right_even(uint32_t value, uint32_t shift) {
    uint32_t q = value >> shift, rem = value & ((1u << shift) - 1), half = 1u << (shift - 1);
    return q + (rem > half || (rem == half && (q & 1)));
}
/* gguf_decode.cpp:395-405: RNE to fp16 with subnormals; |v| rounding to >= 65520 is an error. */
int oracle_float_to_fp16_rne(float v, uint16_t *out) {
    if (!isfinite(v)) return fail("nonfinite weight/scale or conversion overflow");
    uint32_t b = f2u(v), mant = b & 0x7fffff;
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    int e = (int)((b >> 23) & 255) - 127;
    if (e < -25) { *out = sign; return ORACLE_OK; }
    if (e > 15) return fail("FP16 conversion overflow");
    if (e < -14) {
        *out = sign | (uint16_t)round_right_even(0x800000u | mant, (uint32_t)(-e - 1));
        return ORACLE_OK;
    }
    uint32_t r = (uint32_t)(e + 15) * 1024u + round_right_even(mant, 13);
    if (r >= 0x7c00) return fail("FP16 conversion overflow");
    *out = sign | (uint16_t)r;
    return ORACLE_OK;
}

/* gguf_decode.cpp:48-54: sub-block j of the 12-byte packed 6-bit scales/mins. */
void oracle_scale_min(uint32_t j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* gguf_decode.cpp:56-111: one block to fp32 (1 element for F32 / F16 / BF16, 32 for the
 * legacy Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0 blocks, 256 for the K-quants). Products are
 * evaluated in the reference's order (code*scale [+ minimum]; (d*sc)*q - dmin*m;
 * (d*sc)*(code-32)) without contraction. */
int oracle_decode_block(uint32_t type, const uint8_t *p, float *out) {
    uint32_t n = 256;
    if (type == 0 || type == 1 || type == 30) {
        n = 1;
        out[0] = type == 0 ? u2f(rd32(p)) : type == 1 ? oracle_fp16_to_float(rd16(p)) : bf16_value(rd16(p));
    } else if (type == 2 || type == 3 || type == 6 || type == 7 || type == 8) {
        n = 32;
        const float scale = oracle_fp16_to_float(rd16(p));
        if (!isfinite(scale)) return fail("nonfinite weight/scale or conversion overflow");
        if (type == 8) {
            for (uint32_t i = 0; i < 32; ++i) out[i] = (float)(int8_t)p[2 + i] * scale;
        } else {
            const int affine = type == 3 || type == 7, five = type == 6 || type == 7;
            const float minimum = affine ? oracle_fp16_to_float(rd16(p + 2)) : 0.f;
            if (!isfinite(minimum)) return fail("nonfinite weight/scale or conversion overflow");
            const uint32_t offset = affine ? 4 : 2;
            const uint32_t high = five ? rd32(p + offset) : 0;
            const uint8_t *low = p + offset + (five ? 4 : 0);
            for (uint32_t i = 0; i < 16; ++i) {
                int a = (low[i] & 15) | (five ? (int)((high >> i) & 1) << 4 : 0);
                int b = (low[i] >> 4) | (five ? (int)((high >> (i + 16)) & 1) << 4 : 0);
                if (!affine) { a -= five ? 16 : 8; b -= five ? 16 : 8; }
                if (affine) {
                    const float pa = (float)a * scale, pb = (float)b * scale;
                    out[i] = pa + minimum;
                    out[i + 16] = pb + minimum;
                } else {
                    out[i] = (float)a * scale;
                    out[i + 16] = (float)b * scale;
                }
            }
        }
    } else if (type == 12 || type == 13) {
        const float d = oracle_fp16_to_float(rd16(p)), dmin = oracle_fp16_to_float(rd16(p + 2));
        if (!isfinite(d) || !isfinite(dmin)) return fail("nonfinite weight/scale or conversion overflow");
        const uint8_t *scales = p + 4, *qh = p + 16, *qs = p + (type == 13 ? 48 : 16);
        for (uint32_t g = 0; g < 8; ++g) {
            uint8_t sc, m;
            oracle_scale_min(g, scales, &sc, &m);
            const float a = d * (float)sc, b = dmin * (float)m;
            for (uint32_t j = 0; j < 32; ++j) {
                const uint8_t byte = qs[(g / 2) * 32 + j];
                int code = (g & 1) ? (byte >> 4) : (byte & 15);
                if (type == 13 && (qh[j] & (1u << g))) code += 16;
                const float prod = a * (float)code;
                out[g * 32 + j] = prod - b;
            }
        }
    } else if (type == 14) {
        const float d = oracle_fp16_to_float(rd16(p + 208));
        if (!isfinite(d)) return fail("nonfinite weight/scale or conversion overflow");
        for (uint32_t half = 0; half < 2; ++half) {
            const uint8_t *ql = p + half * 64, *qh = p + 128 + half * 32;
            const int8_t *sc = (const int8_t *)(p + 192 + half * 8);
            for (uint32_t j = 0; j < 32; ++j)
                for (uint32_t g = 0; g < 4; ++g) {
                    const uint8_t lo = ql[j + (g & 1) * 32];
                    const int code = (int)(((g < 2) ? (lo & 15) : (lo >> 4)) |
                                           (((qh[j] >> (2 * g)) & 3) << 4)) - 32;
                    const float a = d * (float)sc[j / 16 + g * 2];
                    out[half * 128 + g * 32 + j] = a * (float)code;
                }
        }
    } else {
        return fail("gguf_decode: unsupported tensor type");
    }
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(out[i])) return fail("nonfinite weight/scale or conversion overflow");
    return ORACLE_OK;
}

/* gguf_decode.cpp:112-116 */
static int write_value(uint8_t *p, uint32_t dtype, float v) {
    if (dtype == 0) { memcpy(p, &v, 4); return ORACLE_OK; }
    uint16_t bits;
    int rc = dtype == 2 ? oracle_float_to_bf16_rne(v, &bits) : oracle_float_to_fp16_rne(v, &bits);
    if (rc) return rc;
    memcpy(p, &bits, 2);
    return ORACLE_OK;
}

static int mul_ok(uint64_t a, uint64_t b, uint64_t *r) {
    if (a && b > UINT64_MAX / a) return 0;
    *r = a * b;
    return 1;
}
static int add_ok(uint64_t a, uint64_t b, uint64_t *r) {
    if (b > UINT64_MAX - a) return 0;
    *r = a + b;
    return 1;
}

/* Receipt (gguf_decode.hpp:39-43); simd_blocks is always 0 here (scalar path). */
typedef struct { uint64_t source_bytes, elements, bytes_written, scratch_bytes, simd_blocks; } oracle_receipt;

/*
 * decode_cpu_into (gguf_decode.cpp:433-445) when gather == NULL, decode_cpu_gather
 * (:446-465) otherwise. Geometry checks follow validate() (:160-183). A set cancel flag
 * returns ORACLE_CANCELLED before anything is written.
 */
int oracle_decode(uint32_t type, const void *source, uint64_t source_bytes, uint64_t source_rows,
                  uint64_t source_columns, uint64_t row_begin, uint64_t rows, uint64_t column_begin,
                  uint64_t columns, uint32_t dtype, void *target, uint64_t target_bytes,
                  uint64_t row_stride, uint64_t column_stride, const uint64_t *gather,
                  uint64_t gather_count, int cancel, oracle_receipt *receipt) {
    if (cancel) { snprintf(g_error, sizeof g_error, "gguf_decode_cancelled"); return ORACLE_CANCELLED; }
    const type_info *t = find_type(type);
    if (!t) return fail("gguf_decode: unsupported tensor type");
    if (dtype > 2) return fail("gguf_decode: invalid target dtype");
    if (gather) rows = gather_count;
    else if (!(row_begin <= source_rows && rows <= source_rows - row_begin)) return fail("row slice out of bounds");
    if (!source || !target) return fail("null source/target storage");
    if (!source_rows || !source_columns || source_columns % t->elements) return fail("invalid source geometry");
    if (!rows || !columns || column_begin > source_columns || columns > source_columns - column_begin)
        return fail("invalid decode slice");
    uint64_t row_bytes, total, row_extent, target_extent, tmp;
    if (!mul_ok(source_columns / t->elements, t->bytes, &row_bytes) || !mul_ok(source_rows, row_bytes, &total))
        return fail("gguf_decode: multiplication overflow");
    if (total > source_bytes) return fail("packed source too short");
    const uint32_t item = dtype == 0 ? 4 : 2;
    if (column_stride < item) return fail("invalid/overlapping column stride");
    if (!mul_ok(columns - 1, column_stride, &tmp) || !add_ok(tmp, item, &row_extent))
        return fail("gguf_decode: multiplication overflow");
    if (row_stride < row_extent) return fail("invalid/overlapping row stride");
    if (!mul_ok(rows - 1, row_stride, &tmp) || !add_ok(tmp, row_extent, &target_extent))
        return fail("gguf_decode: multiplication overflow");
    if (target_extent > target_bytes) return fail("decode target too short");
    const uintptr_t s0 = (uintptr_t)source, t0 = (uintptr_t)target;
    if (!(s0 + total <= t0 || t0 + target_extent <= s0)) return fail("packed source overlaps target");
    if (gather) {
        const uintptr_t g0 = (uintptr_t)gather;
        if (!(g0 + gather_count * 8 <= t0 || t0 + target_extent <= g0)) return fail("gather indices overlap target");
        for (uint64_t i = 0; i < gather_count; ++i)
            if (gather[i] >= source_rows) return fail("gather row out of bounds");
    }
    const uint8_t *src = (const uint8_t *)source;
    uint8_t *dst = (uint8_t *)target;
    float scratch[256];
    oracle_receipt r = {0, 0, 0, 1024, 0};
    const uint64_t first = column_begin / t->elements, last = (column_begin + columns - 1) / t->elements;
    /* gguf_decode.cpp:119-123,125-158,327-331: a float source into the same dtype with a
     * dense target is copied, each element checked finite. */
    const int copy = ((type == 0 && dtype == 0) || (type == 1 && dtype == 1) || (type == 30 && dtype == 2)) &&
                     column_stride == t->bytes;
    for (uint64_t row = 0; row < rows; ++row) {
        const uint64_t srow = gather ? gather[row] : row_begin + row;
        if (copy) {
            const uint8_t *sp = src + srow * row_bytes + column_begin * t->bytes;
            for (uint64_t c = 0; c < columns; ++c) {
                const uint32_t bits = t->bytes == 4 ? rd32(sp + c * 4) : rd16(sp + c * 2);
                const uint32_t mask = type == 0 ? 0x7f800000u : type == 1 ? 0x7c00u : 0x7f80u;
                if ((bits & mask) == mask) return fail("nonfinite source float");
                memcpy(dst + row * row_stride + c * t->bytes, sp + c * t->bytes, t->bytes);
            }
            r.source_bytes += columns * t->bytes;
            r.elements += columns;
            r.bytes_written += columns * t->bytes;
            continue;
        }
        for (uint64_t blk = first; blk <= last; ++blk) {
            int rc = oracle_decode_block(type, src + srow * row_bytes + blk * t->bytes, scratch);
            if (rc) return rc;
            const uint64_t b = blk * t->elements > column_begin ? blk * t->elements : column_begin;
            const uint64_t e = (blk + 1) * t->elements < column_begin + columns ? (blk + 1) * t->elements
                                                                                 : column_begin + columns;
            for (uint64_t c = b; c < e; ++c) {
                rc = write_value(dst + row * row_stride + (c - column_begin) * column_stride, dtype,
                                 scratch[c - blk * t->elements]);
                if (rc) return rc;
            }
        }
        r.source_bytes += (last - first + 1) * t->bytes;
        r.elements += columns;
        r.bytes_written += columns * item;
    }
    if (receipt) *receipt = r;
    return ORACLE_OK;
}

/*
 * Row-parallel full-matrix decode for the CPU baseline: rows are split across
 * `threads` workers, as the reference's RowDecodePool does
 * (native/runtime/streaming/gguf_packed_bank.cpp:48-100). Output is dense row-major.
 */
int oracle_decode_rows_parallel(uint32_t type, const void *source, uint64_t rows, uint64_t columns,
                                uint32_t dtype, void *target, int threads) {
    const type_info *t = find_type(type);
    if (!t || columns % 256 || dtype > 2) return fail("invalid geometry");
    const uint64_t row_bytes = columns / 256 * t->bytes, item = dtype == 0 ? 4 : 2;
    int status = ORACLE_OK;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : status)
#endif
    for (int64_t row = 0; row < (int64_t)rows; ++row) {
        float scratch[256];
        const uint8_t *s = (const uint8_t *)source + (uint64_t)row * row_bytes;
        uint8_t *d = (uint8_t *)target + (uint64_t)row * columns * item;
        for (uint64_t blk = 0; blk < columns / 256 && !status; ++blk) {
            if (oracle_decode_block(type, s + blk * t->bytes, scratch)) { status |= 1; break; }
            for (int i = 0; i < 256; ++i)
                if (write_value(d + (blk * 256 + i) * item, dtype, scratch[i])) { status |= 1; break; }
        }
    }
    (void)threads;
    return status ? fail("decode failed") : ORACLE_OK;
}

/* ----------------------------------------------------------------------------------
 * Quantizers (no reference counterpart; parity unpinned, see header).
 *
 * Q4_K: per 32-weight sub-block an affine range [min(0, lo), hi] gives a scale
 * (hi - lo)/15 and a min -min(0, lo); the 8 scales and 8 mins are stored as 6-bit
 * integers relative to the super-block fp16 d = max_scale/63 and dmin = max_min/63,
 * packed with the get_scale_min_k4 layout, and codes are re-derived from the stored
 * (rounded) scales: q = clamp(rint((x + dmin*m) / (d*sc)), 0, 15).
 * Q6_K: per 16-weight sub-block a signed scale amax/32 (sign of the extreme value),
 * stored as int8 relative to fp16 d = max|scale|/127; q = clamp(rint(x/(d*sc)), -32, 31).
 * All steps are plain IEEE fp32 ops with round-to-nearest-even, so the GPU quantizer
 * (turbocider_amd/csrc/k_quantize.hip) produces identical bytes.
 * ---------------------------------------------------------------------------------- */
static uint16_t fp16_bits_or_zero(float v) {
    uint16_t h;
    if (oracle_float_to_fp16_rne(v, &h)) return 0x7bff; /* unreachable for |v| < 65504 */
    return h;
}

void oracle_quantize_q4_k_block(const float *x, uint8_t *out) {
    float scale[8], minv[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) {
            lo = fminf(lo, x[32 * j + i]);
            hi = fmaxf(hi, x[32 * j + i]);
        }
        if (lo > 0.f) lo = 0.f;
        scale[j] = (hi - lo) / 15.f;
        minv[j] = 0.f - lo; /* +0 (never -0) for an all-non-negative sub-block */
        max_scale = fmaxf(max_scale, scale[j]);
        max_min = fmaxf(max_min, minv[j]);
    }
    const uint16_t dh = fp16_bits_or_zero(max_scale / 63.f), mh = fp16_bits_or_zero(max_min / 63.f);
    const float d = oracle_fp16_to_float(dh), dmin = oracle_fp16_to_float(mh);
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        float s = d > 0.f ? rintf(scale[j] / d) : 0.f, m = dmin > 0.f ? rintf(minv[j] / dmin) : 0.f;
        ls[j] = (uint8_t)(s > 63.f ? 63.f : s);
        lm[j] = (uint8_t)(m > 63.f ? 63.f : m);
    }
    memset(out, 0, 144);
    out[0] = (uint8_t)(dh & 255); out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 255); out[3] = (uint8_t)(mh >> 8);
    uint8_t *s = out + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)(ls[j] | ((ls[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(lm[j] | ((lm[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((ls[j + 4] & 15) | ((lm[j + 4] & 15) << 4));
    }
    uint8_t *qs = out + 16;
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, m;
        oracle_scale_min((uint32_t)j, s, &sc, &m);
        const float a = d * (float)sc, b = dmin * (float)m;
        for (int i = 0; i < 32; ++i) {
            float q = 0.f;
            if (a > 0.f) {
                q = rintf((x[32 * j + i] + b) / a);
                q = q < 0.f ? 0.f : (q > 15.f ? 15.f : q);
            }
            qs[(j / 2) * 32 + i] |= (uint8_t)((int)q << ((j & 1) * 4));
        }
    }
}

void oracle_quantize_q6_k_block(const float *x, uint8_t *out) {
    float scale[16], max_abs_scale = 0.f, max_scale = 0.f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.f, vmax = 0.f;
        for (int i = 0; i < 16; ++i) {
            const float v = x[16 * j + i];
            if (fabsf(v) > amax) { amax = fabsf(v); vmax = v; }
        }
        scale[j] = vmax / -32.f;
        if (fabsf(scale[j]) > max_abs_scale) { max_abs_scale = fabsf(scale[j]); max_scale = scale[j]; }
    }
    const uint16_t dh = fp16_bits_or_zero(max_scale / -127.f);
    const float d = oracle_fp16_to_float(dh);
    memset(out, 0, 210);
    int8_t *sc = (int8_t *)(out + 192);
    for (int j = 0; j < 16; ++j) {
        float s = d != 0.f ? rintf(scale[j] / d) : 0.f;
        s = s > 127.f ? 127.f : (s < -128.f ? -128.f : s);
        sc[j] = (int8_t)s;
    }
    out[208] = (uint8_t)(dh & 255); out[209] = (uint8_t)(dh >> 8);
    for (int half = 0; half < 2; ++half) {
        uint8_t *ql = out + half * 64, *qh = out + 128 + half * 32;
        for (int g = 0; g < 4; ++g)
            for (int j = 0; j < 32; ++j) {
                const int idx = half * 128 + g * 32 + j;
                const float a = d * (float)sc[half * 8 + g * 2 + j / 16];
                float q = 0.f;
                if (a != 0.f) {
                    q = rintf(x[idx] / a);
                    q = q < -32.f ? -32.f : (q > 31.f ? 31.f : q);
                }
                const int code = (int)q + 32;
                ql[j + (g & 1) * 32] |= (uint8_t)((code & 15) << ((g >> 1) * 4));
                qh[j] |= (uint8_t)((code >> 4) << (2 * g));
            }
    }
}

/* Quantize `rows` rows of `columns` fp32 weights (columns % 256 == 0) into raw blocks. */
int oracle_quantize(uint32_t type, const float *x, uint64_t rows, uint64_t columns, void *out) {
    if ((type != 12 && type != 14) || columns % 256) return fail("unsupported quantize geometry");
    const uint64_t blocks = rows * (columns / 256), bytes = type == 12 ? 144 : 210;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t b = 0; b < (int64_t)blocks; ++b) {
        if (type == 12) oracle_quantize_q4_k_block(x + (uint64_t)b * 256, (uint8_t *)out + (uint64_t)b * bytes);
        else oracle_quantize_q6_k_block(x + (uint64_t)b * 256, (uint8_t *)out + (uint64_t)b * bytes);
    }
    return ORACLE_OK;
}

/* ----------------------------------------------------------------------------------
 * Runtime-LoRA and bias epilogue, scalar restatement of the reference sequence:
 *   per adapter, in order: low = f32(x)*f32(A)^T (fp32), delta = low*f32(B)^T (fp32),
 *   y = bf16(f32(y) + scale*delta)            (mlx.cpp:692-722, 957-984;
 *                                              native_lora_math_test.cpp:72-107)
 *   then bias last: y = bf16(f32(y) + f32(bf16(bias)))   (mlx.cpp:687-688,
 *                                              dense_linear.hpp:139-141)
 * Sums are accumulated in fp32 in index order, exactly like the reference's scalar spec.
 * `y` is updated in place for rows [row_begin, row_begin+row_count) and output columns
 * [out_begin, out_end); B holds rows for those columns only ([out_end-out_begin, rank]).
 * ---------------------------------------------------------------------------------- */
void oracle_lora_apply_bf16(const uint16_t *x, uint64_t k, uint64_t x_stride, uint16_t *y,
                            uint64_t y_stride, uint64_t row_begin, uint64_t row_count,
                            const uint16_t *a, const uint16_t *b, uint32_t rank, float scale,
                            uint64_t out_begin, uint64_t out_end) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t mi = 0; mi < (int64_t)row_count; ++mi) {
        const uint64_t m = row_begin + (uint64_t)mi;
        float low[1024];
        for (uint32_t r = 0; r < rank && r < 1024; ++r) {
            float sum = 0.f;
            for (uint64_t kk = 0; kk < k; ++kk) {
                const float p = bf16_value(x[m * x_stride + kk]) * bf16_value(a[(uint64_t)r * k + kk]);
                sum = sum + p;
            }
            low[r] = sum;
        }
        for (uint64_t n = out_begin; n < out_end; ++n) {
            float delta = 0.f;
            for (uint32_t r = 0; r < rank; ++r) {
                const float p = low[r] * bf16_value(b[(n - out_begin) * rank + r]);
                delta = delta + p;
            }
            const float t = scale * delta;
            y[m * y_stride + n] = oracle_bf16_bits(bf16_value(y[m * y_stride + n]) + t);
        }
    }
}

void oracle_bias_bf16(uint16_t *y, uint64_t rows, uint64_t n, uint64_t y_stride, const uint16_t *bias_bf16) {
    for (uint64_t m = 0; m < rows; ++m)
        for (uint64_t c = 0; c < n; ++c)
            y[m * y_stride + c] = oracle_bf16_bits(bf16_value(y[m * y_stride + c]) + bf16_value(bias_bf16[c]));
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
