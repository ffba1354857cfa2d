// TEST INFRASTRUCTURE ONLY. A C entry point around the reference's own decoder
// (/root/reference/native/core/gguf_decode.cpp, compiled unmodified from where it lies
// by oracle/Makefile into oracle/_ref/). Used to write and re-check the golden vectors
// and to validate the C restatement in oracle/tc_oracle.c. Argument order follows the
// reference's own ctypes probe, tc_gguf_test_decode (tests/native/gguf_core_probe.cpp:32).
#include "gguf_decode.hpp"
#include <cstdio>
#include <cstring>

namespace {
thread_local char g_error[256];
int fail(const char *what) {
    std::snprintf(g_error, sizeof g_error, "%s", what);
    return 1;
}
}  // namespace

extern "C" const char *tcref_error() { return g_error; }
extern "C" float tcref_half(uint16_t bits) { return tc::gguf::fp16_to_float(bits); }

// dtype: 1 -> fp16, 2 -> bf16 (tests/native/test_gguf_execution.py:186-198).
extern "C" int tcref_round(uint32_t dtype, float value, uint16_t *out) {
    try {
        *out = dtype == 2 ? tc::gguf::float_to_bf16_rne(value) : tc::gguf::float_to_fp16_rne(value);
        return 0;
    } catch (const std::exception &e) { return fail(e.what()); }
}

extern "C" int tcref_decode(uint32_t type, const void *source, uint64_t source_bytes, uint64_t source_rows,
                            uint64_t source_columns, uint64_t row_begin, uint64_t rows, uint64_t column_begin,
                            uint64_t columns, uint32_t dtype, void *target, uint64_t target_bytes,
                            uint64_t row_stride, uint64_t column_stride, const uint64_t *gather,
                            uint64_t gather_count, int cancel, uint64_t *stats) {
    using namespace tc::gguf;
    try {
        if (dtype > 2) return fail("gguf_decode: invalid target dtype");
        const PackedMatrix matrix{{static_cast<const std::byte *>(source), source_bytes}, type, source_rows,
                                  source_columns};
        const DecodeTarget out{{static_cast<std::byte *>(target), target_bytes}, static_cast<DecodeDType>(dtype),
                               row_stride, column_stride};
        std::atomic<bool> flag{cancel != 0};
        DecodeReceipt r = gather ? decode_cpu_gather(matrix, {gather, gather_count}, column_begin, columns, out, &flag)
                                 : decode_cpu_into(matrix, {row_begin, rows, column_begin, columns}, out, &flag);
        if (stats) {
            stats[0] = r.source_bytes_processed; stats[1] = r.elements_written;
            stats[2] = r.bytes_written; stats[3] = r.scratch_bytes;
        }
        return 0;
    } catch (const std::exception &e) {
        return std::strcmp(e.what(), "gguf_decode_cancelled") == 0 ? (fail(e.what()), 2) : fail(e.what());
    }
}
