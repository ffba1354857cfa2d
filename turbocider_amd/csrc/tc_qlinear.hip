// Host side of the tc_qlinear C ABI (include/tc_qlinear.h): argument validation, kernel
// selection and error reporting. Conventions follow the reference's C ABI
// (native/api/c_api.mm:79-90,382-391): status 0/1/2, strdup'd error strings, out-params
// nulled on entry, no exception crosses the boundary.
#include "../../include/tc_qlinear.h"
#include "tc_device.h"
#include "tc_kernels.h"

#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>

namespace {

struct Failure : std::runtime_error {
    int status;
    explicit Failure(const std::string &what, int s = 1) : std::runtime_error(what), status(s) {}
};

void require(bool ok, const char *what) {
    if (!ok) throw Failure(what);
}
void hip_check(hipError_t e, const char *where) {
    if (e != hipSuccess) throw Failure(std::string(where) + ": " + hipGetErrorString(e));
}

int fail(char **error, const std::exception &e) {
    if (error) *error = strdup(e.what());
    const auto *f = dynamic_cast<const Failure *>(&e);
    return f ? f->status : 1;
}

template <class F>
int guarded(char **error, F &&body) {
    if (error) *error = nullptr;
    try {
        body();
        return 0;
    } catch (const std::exception &e) {
        return fail(error, e);
    } catch (...) {
        if (error) *error = strdup("unknown error");
        return 1;
    }
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t &r) {
    if (a && b > UINT64_MAX / a) return false;
    r = a * b;
    return true;
}
bool add_ok(uint64_t a, uint64_t b, uint64_t &r) {
    if (b > UINT64_MAX - a) return false;
    r = a + b;
    return true;
}

uint32_t block_bytes(uint32_t type) {
    switch (type) {
    case TC_GGML_TYPE_Q4_K: return tc::kQ4KBytes;
    case TC_GGML_TYPE_Q5_K: return tc::kQ5KBytes;
    case TC_GGML_TYPE_Q6_K: return tc::kQ6KBytes;
    default: throw Failure("gguf_decode: unsupported tensor type");
    }
}

// Decodable types: elements and bytes per block (native/core/gguf_directory.hpp:21-26).
struct DecodeType {
    uint32_t elements, bytes;
};
DecodeType decode_type(uint32_t type) {
    switch (type) {
    case TC_GGML_TYPE_F32: return {1, 4};
    case TC_GGML_TYPE_F16: return {1, 2};
    case TC_GGML_TYPE_BF16: return {1, 2};
    case TC_GGML_TYPE_Q4_0: return {32, 18};
    case TC_GGML_TYPE_Q4_1: return {32, 20};
    case TC_GGML_TYPE_Q5_0: return {32, 22};
    case TC_GGML_TYPE_Q5_1: return {32, 24};
    case TC_GGML_TYPE_Q8_0: return {32, 34};
    case TC_GGML_TYPE_Q4_K: return {256, tc::kQ4KBytes};
    case TC_GGML_TYPE_Q5_K: return {256, tc::kQ5KBytes};
    case TC_GGML_TYPE_Q6_K: return {256, tc::kQ6KBytes};
    default: throw Failure("gguf_decode: unsupported tensor type");
    }
}

// Per-device scratch for the synchronous decode entry point: an error word and a gather
// index buffer. Guarded by one mutex: decode calls on one device are serialized.
struct DeviceScratch {
    int *err = nullptr;
    uint64_t *idx = nullptr;
    uint64_t idx_cap = 0;
};
std::mutex g_scratch_mutex;
std::unordered_map<int, DeviceScratch> g_scratch;

int current_device() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    return dev;
}

DeviceScratch &scratch_for(int dev) {
    DeviceScratch &s = g_scratch[dev];
    if (!s.err) hip_check(hipMalloc(&s.err, 256), "hipMalloc(error word)");
    return s;
}

// Decode error words (flags, then the first target positions of a value error and of a
// conversion overflow) -> status/message after the stream drained: the error the reference,
// decoding in row and column order, would have met first.
void reset_decode_errors(int *d_err, hipStream_t stream) {
    hip_check(hipMemsetAsync(d_err, 0, sizeof(int), stream), "hipMemsetAsync(error word)");
    hip_check(hipMemsetAsync(d_err + 2, 0xff, 2 * sizeof(uint64_t), stream), "hipMemsetAsync(error positions)");
}
void check_decode_errors(int *d_err, hipStream_t stream) {
    int host[6] = {};
    hip_check(hipMemcpyAsync(host, d_err, sizeof host, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(error words)");
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    uint64_t pos[2];
    std::memcpy(pos, host + 2, sizeof pos);
    const int flags = host[0];
    const bool value = flags & (tc::kErrSourceFloat | tc::kErrNonfinite);
    const bool over = flags & (tc::kErrF16Overflow | tc::kErrBF16Overflow);
    if (value && (!over || pos[0] < pos[1]))
        throw Failure(flags & tc::kErrSourceFloat ? "nonfinite source float"
                                                  : "nonfinite weight/scale or conversion overflow");
    if (over) throw Failure(flags & tc::kErrF16Overflow ? "FP16 conversion overflow" : "BF16 conversion overflow");
}

// Device error word -> status/message after the stream drained.
void check_error_word(int *d_err, hipStream_t stream) {
    int host = 0;
    hip_check(hipMemcpyAsync(&host, d_err, sizeof host, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(error word)");
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (host & tc::kErrSourceFloat) throw Failure("nonfinite source float");
    if (host & tc::kErrNonfinite) throw Failure("nonfinite weight/scale or conversion overflow");
    if (host & tc::kErrF16Overflow) throw Failure("FP16 conversion overflow");
    if (host & tc::kErrBF16Overflow) throw Failure("BF16 conversion overflow");
}

}  // namespace

// Types the hand-written dequant kernels read directly (the rest are decoded to bf16 once).
static bool fused_type(uint32_t t) {
    return t == TC_GGML_TYPE_Q4_K || t == TC_GGML_TYPE_Q5_K || t == TC_GGML_TYPE_Q6_K;
}

struct tc_qlinear {
    uint32_t type = 0;
    uint64_t n = 0, k = 0;
    const uint8_t *weight = nullptr;
    uint16_t *bias_bf16 = nullptr;  // owned: astype(bias, bf16)
    int device = 0;
    uint32_t path = 0;
    float *low = nullptr;           // owned LoRA workspace
    uint64_t low_bytes = 0;
    void *gemm_ws = nullptr;        // owned split-K workspace (GEMM and skinny-kernel partial sums)
    uint64_t gemm_ws_bytes = 0;
    // Weights of a type other than Q4_K / Q5_K / Q6_K: decoded once to bf16 [n, k] (owned) and
    // multiplied by the library GEMM (the reference's decode-then-dense-matmul route).
    uint16_t *dense = nullptr;
    rocblas_handle blas = nullptr;
    // Owned bf16 [m, n] pre-activation outputs of tc_qlinear_forward_act's unfused routes with
    // the gated activation (whose output is n/2 wide).
    uint16_t *pre = nullptr;
    uint64_t pre_bytes = 0;
};

namespace {
// K slices for the LoRA low product: enough workgroups (32 rows x 64 ranks each) to put about
// one and a half on every CU, at most 8 slices and one 128-wide chunk per slice (config 5's
// 160 tiles: 3 slices; 5 slices, about three workgroups per CU, measured 1.2 % slower on its
// block, 2 the same, 1 slower).
int lora_ksplit(const tc_lora_adapter *adapters, uint32_t count, uint64_t k) {
    uint64_t wgs = 0;
    for (uint32_t i = 0; i < count && i < (uint32_t)tc::kLoraBatch; ++i)
        wgs += (adapters[i].row_count + 31) / 32 * ((adapters[i].rank + 63) / 64);
    if (!wgs) return 1;
    const uint64_t want = (384 + wgs - 1) / wgs;
    return (int)std::max<uint64_t>(1, std::min<uint64_t>({want, 8, k / 128}));
}
}  // namespace

extern "C" uint32_t tc_qlinear_abi_version(void) { return TC_QLINEAR_ABI_VERSION; }

extern "C" void tc_qlinear_string_free(char *s) { free(s); }

extern "C" int tc_gguf_decode_device(uint32_t ggml_type, const void *source, uint64_t source_bytes,
                                     uint64_t source_rows, uint64_t source_columns, uint64_t row_begin,
                                     uint64_t rows, uint64_t column_begin, uint64_t columns, uint32_t dtype,
                                     void *target, uint64_t target_bytes, uint64_t row_stride,
                                     uint64_t column_stride, const uint64_t *row_indices,
                                     const volatile int *cancel, void *stream, tc_decode_receipt *receipt,
                                     char **error) {
    if (receipt) std::memset(receipt, 0, sizeof *receipt);
    return guarded(error, [&] {
        // gguf_decode.cpp:433-437 (cancel, row slice) and validate() :160-183.
        if (cancel && *cancel) throw Failure("gguf_decode_cancelled", 2);
        const DecodeType t = decode_type(ggml_type);
        const uint32_t bbytes = t.bytes;
        require(dtype <= TC_DTYPE_BF16, "gguf_decode: invalid target dtype");
        if (row_indices) require(row_begin == 0, "row_begin must be 0 for a gather");
        else require(row_begin <= source_rows && rows <= source_rows - row_begin, "row slice out of bounds");
        require(source && target, "null source/target storage");
        require(source_rows && source_columns && source_columns % t.elements == 0, "invalid source geometry");
        require(rows && columns && column_begin <= source_columns && columns <= source_columns - column_begin,
                "invalid decode slice");
        uint64_t row_bytes, total, tmp, row_extent, target_extent;
        require(mul_ok(source_columns / t.elements, bbytes, row_bytes) && mul_ok(source_rows, row_bytes, total),
                "gguf_decode: multiplication overflow");
        require(total <= source_bytes, "packed source too short");
        const uint64_t item = dtype == TC_DTYPE_F32 ? 4 : 2;
        require(column_stride >= item, "invalid/overlapping column stride");
        require(mul_ok(columns - 1, column_stride, tmp) && add_ok(tmp, item, row_extent),
                "gguf_decode: multiplication overflow");
        require(row_stride >= row_extent, "invalid/overlapping row stride");
        require(mul_ok(rows - 1, row_stride, tmp) && add_ok(tmp, row_extent, target_extent),
                "gguf_decode: multiplication overflow");
        require(target_extent <= target_bytes, "decode target too short");
        const uintptr_t s0 = reinterpret_cast<uintptr_t>(source), t0 = reinterpret_cast<uintptr_t>(target);
        require(total <= UINTPTR_MAX - s0 && target_extent <= UINTPTR_MAX - t0, "pointer range overflow");
        require(s0 + total <= t0 || t0 + target_extent <= s0, "packed source overlaps target");
        if (row_indices)
            for (uint64_t i = 0; i < rows; ++i) require(row_indices[i] < source_rows, "gather row out of bounds");
        const uint64_t first = column_begin / t.elements, last = (column_begin + columns - 1) / t.elements;
        const uint64_t per_row = t.elements == 256 ? last - first + 1 : (column_begin + columns + 3) / 4 - column_begin / 4;
        require(per_row <= (1ull << 33) && rows <= (1ull << 33) / per_row, "decode grid too large");
        // gguf_decode.cpp:119-123,327: a float source into its own dtype with a dense target.
        const bool copy = ((ggml_type == TC_GGML_TYPE_F32 && dtype == TC_DTYPE_F32) ||
                           (ggml_type == TC_GGML_TYPE_F16 && dtype == TC_DTYPE_F16) ||
                           (ggml_type == TC_GGML_TYPE_BF16 && dtype == TC_DTYPE_BF16)) &&
                          column_stride == bbytes;

        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        DeviceScratch &sc = scratch_for(current_device());
        const uint64_t *d_rows = nullptr;
        if (row_indices) {
            if (sc.idx_cap < rows) {
                if (sc.idx) hip_check(hipFree(sc.idx), "hipFree");
                sc.idx = nullptr;
                sc.idx_cap = 0;
                hip_check(hipMalloc(&sc.idx, rows * sizeof(uint64_t)), "hipMalloc(gather indices)");
                sc.idx_cap = rows;
            }
            hip_check(hipMemcpyAsync(sc.idx, row_indices, rows * sizeof(uint64_t), hipMemcpyHostToDevice, s),
                      "hipMemcpyAsync(gather indices)");
            d_rows = sc.idx;
        }
        reset_decode_errors(sc.err, s);
        hip_check(tc::launch_decode(ggml_type, static_cast<const uint8_t *>(source), row_bytes, source_columns,
                                    d_rows, row_begin, rows, column_begin, columns, static_cast<uint8_t *>(target),
                                    row_stride, column_stride, dtype, copy ? 1 : 0, sc.err, s),
                  "decode launch");
        check_decode_errors(sc.err, s);
        if (receipt) {
            receipt->source_bytes_processed = rows * (last - first + 1) * bbytes;
            receipt->elements_written = rows * columns;
            receipt->bytes_written = rows * columns * item;
            receipt->scratch_bytes = 0;
            receipt->simd_blocks = rows * (last - first + 1);
        }
    });
}

extern "C" int tc_gguf_quantize_device(uint32_t ggml_type, const float *weights, uint64_t rows, uint64_t columns,
                                       void *blocks, uint64_t block_bytes_total, void *stream, char **error) {
    return guarded(error, [&] {
        require(ggml_type == TC_GGML_TYPE_Q4_K || ggml_type == TC_GGML_TYPE_Q6_K, "unsupported quantize type");
        require(weights && blocks && rows && columns && columns % 256 == 0, "invalid quantize geometry");
        uint64_t need;
        require(mul_ok(rows * (columns / 256), block_bytes(ggml_type), need), "quantize size overflow");
        require(need <= block_bytes_total, "quantize target too short");
        require(ggml_type == TC_GGML_TYPE_Q4_K ? (reinterpret_cast<uintptr_t>(blocks) & 3u) == 0
                                               : (reinterpret_cast<uintptr_t>(blocks) & 1u) == 0,
                "misaligned quantize target");
        require(rows * (columns / 256) / 64 < (1ull << 31), "quantize grid too large");
        hip_check(tc::launch_quantize(ggml_type, weights, rows, columns, static_cast<uint8_t *>(blocks),
                                      static_cast<hipStream_t>(stream)),
                  "quantize launch");
    });
}

extern "C" int tc_qlinear_create(const tc_qlinear_desc *desc, tc_qlinear **out, char **error) {
    if (out) *out = nullptr;
    return guarded(error, [&] {
        require(desc && out, "missing descriptor or output handle");
        const DecodeType t = decode_type(desc->ggml_type);  // throws for an unregistered type
        const bool kquant = fused_type(desc->ggml_type);
        require(desc->n > 0 && desc->k > 0 && desc->k % 256 == 0, "invalid linear geometry (k % 256 != 0)");
        require(desc->n < (1ull << 31) && desc->k < (1ull << 31), "linear too large");
        require(desc->weight, "null weight");
        uint64_t need;
        require(mul_ok(desc->n, desc->k / t.elements * t.bytes, need) && need <= desc->weight_bytes,
                "weight buffer too short");
        if (desc->ggml_type == TC_GGML_TYPE_Q4_K)
            require((reinterpret_cast<uintptr_t>(desc->weight) & 15u) == 0, "Q4_K weight must be 16-byte aligned");
        else if (desc->ggml_type == TC_GGML_TYPE_Q5_K)
            require((reinterpret_cast<uintptr_t>(desc->weight) & 15u) == 0, "Q5_K weight must be 16-byte aligned");
        else if (desc->ggml_type == TC_GGML_TYPE_Q6_K)
            require((reinterpret_cast<uintptr_t>(desc->weight) & 3u) == 0, "Q6_K weight must be 4-byte aligned");
        require(desc->bias_dtype <= TC_DTYPE_BF16, "invalid bias dtype");

        auto *h = new tc_qlinear();
        try {
            h->type = desc->ggml_type;
            h->n = desc->n;
            h->k = desc->k;
            h->weight = static_cast<const uint8_t *>(desc->weight);
            h->device = current_device();
            std::lock_guard<std::mutex> lock(g_scratch_mutex);
            DeviceScratch &sc = scratch_for(h->device);
            if (kquant) {
                hip_check(hipMemset(sc.err, 0, sizeof(int)), "hipMemset(error word)");
                hip_check(tc::launch_scan_scales(h->type, h->weight, desc->n * (desc->k / 256), sc.err, nullptr),
                          "scale scan launch");
                check_error_word(sc.err, nullptr);
            } else {
                // Decode once to bf16 (bit-exact to the reference decoder, non-finite values
                // rejected with its messages), then the library GEMM per call.
                hip_check(hipMalloc(&h->dense, desc->n * desc->k * sizeof(uint16_t)), "hipMalloc(dense weight)");
                reset_decode_errors(sc.err, nullptr);
                hip_check(tc::launch_decode(h->type, h->weight, desc->k / t.elements * t.bytes, desc->k, nullptr, 0,
                                            desc->n, 0, desc->k, reinterpret_cast<uint8_t *>(h->dense),
                                            desc->k * sizeof(uint16_t), sizeof(uint16_t), TC_DTYPE_BF16, 0, sc.err,
                                            nullptr),
                          "dense decode launch");
                check_decode_errors(sc.err, nullptr);
                require(rocblas_create_handle(&h->blas) == rocblas_status_success, "rocblas_create_handle failed");
            }
            if (desc->bias) {
                hip_check(hipMalloc(&h->bias_bf16, desc->n * sizeof(uint16_t)), "hipMalloc(bias)");
                hip_check(tc::launch_bias_to_bf16(desc->bias, desc->bias_dtype, desc->n, h->bias_bf16, nullptr),
                          "bias cast launch");
                hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
            }
        } catch (...) {
            tc_qlinear_free(h);
            throw;
        }
        *out = h;
    });
}

// Grows the handle's split-K workspace (device memory, kept for later calls) to `need` bytes.
static void grow_gemm_workspace(tc_qlinear *L, uint64_t need) {
    if (need <= L->gemm_ws_bytes) return;
    if (L->gemm_ws) hip_check(hipFree(L->gemm_ws), "hipFree(GEMM workspace)");
    L->gemm_ws = nullptr;
    L->gemm_ws_bytes = 0;
    hip_check(hipMalloc(&L->gemm_ws, need), "hipMalloc(GEMM workspace)");
    L->gemm_ws_bytes = need;
}

extern "C" int tc_qlinear_set_path(tc_qlinear *linear, uint32_t path, char **error) {
    return guarded(error, [&] {
        require(linear, "null handle");
        require(path <= 3, "invalid path");
        linear->path = path;
    });
}

namespace {
// The kernel route of one forward call, decided on the host from the geometry alone (no
// device state), so that tc_qlinear_plan reports exactly what tc_qlinear_forward runs.
struct Plan {
    uint32_t kernel = 0;    // TC_QLINEAR_KERNEL_*
    int tail = 0;           // GEMM: rows at the end of M handed to the skinny kernel
    int splits = 1;         // K slices of the main launch (GEMM or skinny)
    int tail_splits = 1;    // K slices of the tail launch
    uint64_t ws_main = 0;   // split-K partials of the main launch
    uint64_t ws_tail = 0;   // split-K partials of the tail launch
};

// `capacity`: the most split-K partial bytes one launch may use (UINT64_MAX: the preferred
// splits; the allocation-free entry point passes its fixed scratch size, which can only lower
// the number of K slices).
Plan plan_forward(uint32_t type, bool dense, uint64_t n, uint64_t k, uint64_t m, uint64_t x_stride, uint32_t path,
                  uint64_t capacity = UINT64_MAX) {
    require(m >= 1 && m < (1ull << 31), "invalid row count");
    require(x_stride >= k, "invalid row stride");
    require(path <= 3, "invalid path");
    Plan p;
    if (dense) {
        // rocBLAS takes 32-bit sizes and leading dimensions.
        require(x_stride < (1ull << 31), "activation row stride too large for the library GEMM");
        p.kernel = TC_QLINEAR_KERNEL_DENSE;
        return p;
    }
    const int M = (int)m, N = (int)n, K = (int)k;
    const int64_t xs = (int64_t)x_stride;
    const bool gemv = path == 2 || (path == 0 && m == 1);
    require(!(gemv && m > 8), "the skinny path takes at most 8 rows");
    require(!(gemv && m > 1 && type == TC_GGML_TYPE_Q5_K), "the per-row GEMV takes Q4_K / Q6_K weights");
    if (gemv && m == 1) {
        p.kernel = TC_QLINEAR_KERNEL_GEMV1;
    } else if (path == 0 && tc::gemv8_supports(type, M, K, xs)) {
        p.kernel = TC_QLINEAR_KERNEL_GEMV8;
    } else if (gemv) {
        p.kernel = TC_QLINEAR_KERNEL_GEMV;
    } else if ((path == 3 || (path == 0 && m >= 9)) && tc::skinny_supports(type, M, N, K, xs)) {
        p.kernel = TC_QLINEAR_KERNEL_SKINNY;
        p.splits = tc::skinny_splits_within(M, N, K, capacity);
        p.ws_main = tc::skinny_workspace_bytes(M, N, p.splits);
    } else {
        // The GEMM addresses the rows of one output tile (at most 256) from the tile's first row
        // with 32-bit buffer offsets; the range of a tile's descriptor is clamped in the kernel.
        require(tc::gemm_supports(K, xs),
                "activation row stride too large: the GEMM addresses 256 rows with 32-bit offsets");
        p.kernel = TC_QLINEAR_KERNEL_GEMM;
        if (path == 0) {
            p.tail = tc::gemm_tail_rows(M, N, K);
            if (p.tail && !tc::skinny_supports(type, p.tail, N, K, xs)) p.tail = 0;
        }
        p.splits = tc::gemm_splits_within(M - p.tail, N, K, capacity);
        p.ws_main = tc::gemm_workspace_bytes(M - p.tail, N, K, p.splits);
        if (p.tail) {
            p.tail_splits = tc::skinny_splits_within(p.tail, N, K, capacity);
            p.ws_tail = tc::skinny_workspace_bytes(p.tail, N, p.tail_splits);
        }
    }
    return p;
}

// Split-K and LoRA workspace a forward call needs: the base launches' partial sums and, for
// adapters, the low of every adapter of one batch (kLoraBatch adapters) side by side, `ksplit`
// partial planes each.
struct Workspace {
    uint64_t gemm = 0, low = 0;
    int ksplit = 1;
};
Workspace forward_workspace(const tc_qlinear *L, const Plan &p, uint64_t m, const tc_lora_adapter *adapters,
                            uint32_t adapter_count, uint64_t capacity = UINT64_MAX) {
    // Adapters are checked first; `one` is the low of each batch at one K slice (the slices
    // multiply it), so that the K split can be lowered to fit `capacity`.
    uint64_t one = 0, max_one = 0;
    for (uint32_t i = 0; i < adapter_count; ++i) {
        const tc_lora_adapter &a = adapters[i];
        require(a.a && a.b, "null LoRA factor");
        require(a.rank >= 1 && a.rank <= 1024, "LoRA rank must be in 1..1024");
        require(std::isfinite(a.scale), "LoRA effective scale must be finite");
        require(a.row_count >= 1 && a.row_begin <= m && a.row_count <= m - a.row_begin, "invalid LoRA row range");
        require(a.output_begin < a.output_end && a.output_end <= L->n, "invalid runtime LoRA output range");
        require((reinterpret_cast<uintptr_t>(a.a) & 15u) == 0, "LoRA A must be 16-byte aligned");
        if (i % tc::kLoraBatch == 0) one = 0;
        one += a.row_count * ((uint64_t)(a.rank + 7) / 8 * 8) * sizeof(float);
        max_one = std::max(max_one, one);
    }
    Workspace ws;
    ws.gemm = std::max(p.ws_main, p.ws_tail);
    ws.ksplit = lora_ksplit(adapters, adapter_count, L->k);
    if (max_one) {
        require(max_one <= capacity, "runtime LoRA workspace exceeds the fixed scratch of the allocation-free "
                                     "entry point (use tc_qlinear_forward)");
        ws.ksplit = (int)std::min<uint64_t>((uint64_t)ws.ksplit, capacity / max_one);
    }
    ws.low = (uint64_t)ws.ksplit * max_one;
    return ws;
}

void check_forward_args(const tc_qlinear *L, const uint16_t *x, uint64_t m, uint64_t x_row_stride, const uint16_t *y,
                        uint64_t y_row_stride, const tc_lora_adapter *adapters, uint32_t adapter_count) {
    require(L, "null handle");
    require(x && y, "null activation/output");
    require(m >= 1 && m < (1ull << 31), "invalid row count");
    require(x_row_stride >= L->k && y_row_stride >= L->n, "invalid row stride");
    require((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && x_row_stride % 8 == 0,
            "activation rows must be 16-byte aligned");
    require(!adapter_count || adapters, "null adapter array");
    require(current_device() == L->device, "handle used on a different device than it was created on");
}

// Whether the planned route applies an output activation in its own epilogue (no runtime
// adapters, one of the hand-written kernels); otherwise forward_act runs the activation pass.
bool act_in_epilogue(const Plan &p, uint32_t adapter_count) {
    return adapter_count == 0 && (p.kernel == TC_QLINEAR_KERNEL_GEMM || p.kernel == TC_QLINEAR_KERNEL_GEMV1 ||
                                  p.kernel == TC_QLINEAR_KERNEL_GEMV8 || p.kernel == TC_QLINEAR_KERNEL_SKINNY);
}

// Enqueues the planned launches. `gemm_ws` / `low` hold at least forward_workspace()'s bytes.
// `act` (TC_QLINEAR_ACT_*) is applied by the kernels' epilogues; the caller passes it only
// where act_in_epilogue() holds (y is then n/2 wide for the gated activation).
void run_forward(tc_qlinear *L, const Plan &p, const Workspace &ws, const uint16_t *x, uint64_t m,
                 uint64_t x_row_stride, uint16_t *y, uint64_t y_row_stride, const tc_lora_adapter *adapters,
                 uint32_t adapter_count, void *gemm_ws, float *low, hipStream_t s, int act = tc::kActNone) {
    const uint16_t *bias_in_kernel = adapter_count ? nullptr : L->bias_bf16;
    const int M = (int)m, N = (int)L->n, K = (int)L->k;
    const int64_t xs = (int64_t)x_row_stride, ys = (int64_t)y_row_stride;
    require(act == tc::kActNone || act_in_epilogue(p, adapter_count), "internal: activation on an unfused route");
    switch (p.kernel) {
    case TC_QLINEAR_KERNEL_DENSE: {
        // y[m, n] = bf16(x . W^T) with fp32 accumulation: in column-major terms
        // y^T [n, m] = W [k, n]^T . x^T [k, m] (W rows are columns of length k).
        const float alpha = 1.f, beta = 0.f;
        require(rocblas_set_stream(L->blas, s) == rocblas_status_success, "rocblas_set_stream failed");
        const rocblas_status st = rocblas_gemm_ex(
            L->blas, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)L->n, (rocblas_int)m,
            (rocblas_int)L->k, &alpha, L->dense, rocblas_datatype_bf16_r, (rocblas_int)L->k, x,
            rocblas_datatype_bf16_r, (rocblas_int)x_row_stride, &beta, y, rocblas_datatype_bf16_r,
            (rocblas_int)y_row_stride, y, rocblas_datatype_bf16_r, (rocblas_int)y_row_stride,
            rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
        require(st == rocblas_status_success, "rocblas_gemm_ex failed");
        if (!adapter_count && L->bias_bf16)  // the bias pass (with adapters: after the last batch)
            hip_check(tc::launch_lora_epilogue(y, ys, M, N, tc::LoraBatch{}, L->bias_bf16, s), "bias launch");
        break;
    }
    case TC_QLINEAR_KERNEL_GEMV1:
        hip_check(tc::launch_gemv1(L->type, x, L->weight, N, K, y, bias_in_kernel, s, 0, act), "gemv launch");
        break;
    case TC_QLINEAR_KERNEL_GEMV8:
        hip_check(tc::launch_gemv8(L->type, x, xs, M, L->weight, N, K, y, ys, bias_in_kernel, s, 0, act),
                  "gemv launch");
        break;
    case TC_QLINEAR_KERNEL_GEMV:
        hip_check(tc::launch_gemv(L->type, x, xs, M, L->weight, N, K, y, ys, bias_in_kernel, s), "gemv launch");
        break;
    case TC_QLINEAR_KERNEL_SKINNY:
        hip_check(
            tc::launch_skinny(L->type, x, xs, M, L->weight, N, K, y, ys, bias_in_kernel, p.splits, gemm_ws, s, act),
            "skinny launch");
        break;
    default: {
        // A short last row of 256-row tiles that would need a grid round of its own goes to
        // the skinny kernel (a second launch on the same stream, after the GEMM).
        // With adapters, the LoRA pass below reads y back at once: keep its lines in the caches.
        const int m_main = M - p.tail;
        const int gemm_act = adapter_count ? tc::kActNoneKeep : act;
        hip_check(tc::launch_gemm(L->type, x, xs, m_main, L->weight, N, K, y, ys, bias_in_kernel, p.splits, gemm_ws,
                                  s, gemm_act),
                  "gemm launch");
        if (p.tail)
            hip_check(tc::launch_skinny(L->type, x + (uint64_t)m_main * x_row_stride, xs, p.tail, L->weight, N, K,
                                        y + (uint64_t)m_main * y_row_stride, ys, bias_in_kernel, p.tail_splits,
                                        gemm_ws, s, act),
                      "skinny launch (tail rows)");
    }
    }
    // Adapters in batches, in order: the low of the batch, then one pass over y that adds
    // the batch's terms (and, after the last batch, the bias).
    for (uint32_t first = 0; first < adapter_count; first += tc::kLoraBatch) {
        tc::LoraBatch batch{};
        batch.count = (int)std::min<uint32_t>(tc::kLoraBatch, adapter_count - first);
        uint64_t off = 0;
        for (int j = 0; j < batch.count; ++j) {
            const tc_lora_adapter &a = adapters[first + j];
            tc::LoraDesc &d = batch.d[j];
            const int stride = (int)((a.rank + 7) / 8 * 8);
            d.a = a.a;
            d.b = a.b;
            d.low = low + off / sizeof(float);
            d.rank = (int)a.rank;
            d.low_stride = stride;
            d.row_begin = (int)a.row_begin;
            d.row_count = (int)a.row_count;
            d.out_begin = (int)a.output_begin;
            d.out_count = (int)(a.output_end - a.output_begin);
            d.scale = a.scale;
            d.b_vec = a.rank % 8 == 0 && (reinterpret_cast<uintptr_t>(a.b) & 15u) == 0;
            d.ksplit = ws.ksplit;
            d.low_plane = (int64_t)a.row_count * stride;
            off += (uint64_t)ws.ksplit * a.row_count * (uint64_t)stride * sizeof(float);
        }
        const bool last = first + tc::kLoraBatch >= adapter_count;
        hip_check(tc::launch_lora_low(x, xs, K, batch, s), "LoRA low launch");
        hip_check(tc::launch_lora_epilogue(y, ys, M, N, batch, last ? L->bias_bf16 : nullptr, s),
                  "LoRA epilogue launch");
    }
}
}  // namespace

extern "C" int tc_qlinear_plan(uint32_t ggml_type, uint64_t n, uint64_t k, uint64_t m, uint64_t x_row_stride,
                               uint32_t path, tc_qlinear_plan_info *out, char **error) {
    if (out) std::memset(out, 0, sizeof *out);
    return guarded(error, [&] {
        require(out, "null plan output");
        (void)decode_type(ggml_type);  // throws for an unregistered type
        require(n > 0 && k > 0 && k % 256 == 0, "invalid linear geometry (k % 256 != 0)");
        require(n < (1ull << 31) && k < (1ull << 31), "linear too large");
        const bool dense = !fused_type(ggml_type);
        const Plan p = plan_forward(ggml_type, dense, n, k, m, x_row_stride, path);
        out->kernel = p.kernel;
        out->tail_rows = (uint32_t)p.tail;
        out->workspace_bytes = std::max(p.ws_main, p.ws_tail);
    });
}

extern "C" int tc_qlinear_forward(tc_qlinear *L, const uint16_t *x, uint64_t m, uint64_t x_row_stride, uint16_t *y,
                                  uint64_t y_row_stride, const tc_lora_adapter *adapters, uint32_t adapter_count,
                                  void *stream, char **error) {
    return guarded(error, [&] {
        check_forward_args(L, x, m, x_row_stride, y, y_row_stride, adapters, adapter_count);
        const Plan p = plan_forward(L->type, L->dense != nullptr, L->n, L->k, m, x_row_stride, L->path);
        const Workspace ws = forward_workspace(L, p, m, adapters, adapter_count);
        if (ws.low > L->low_bytes) {
            if (L->low) hip_check(hipFree(L->low), "hipFree(LoRA workspace)");
            L->low = nullptr;
            L->low_bytes = 0;
            hip_check(hipMalloc(&L->low, ws.low), "hipMalloc(LoRA workspace)");
            L->low_bytes = ws.low;
        }
        grow_gemm_workspace(L, ws.gemm);
        run_forward(L, p, ws, x, m, x_row_stride, y, y_row_stride, adapters, adapter_count, L->gemm_ws, L->low,
                    static_cast<hipStream_t>(stream));
    });
}

extern "C" int tc_qlinear_forward_act(tc_qlinear *L, uint32_t act, const uint16_t *x, uint64_t m,
                                      uint64_t x_row_stride, uint16_t *y, uint64_t y_row_stride,
                                      const tc_lora_adapter *adapters, uint32_t adapter_count, void *stream,
                                      char **error) {
    return guarded(error, [&] {
        require(act <= TC_QLINEAR_ACT_SILU_GLU, "unknown output activation");
        require(L, "null handle");
        const bool glu = act == TC_QLINEAR_ACT_SILU_GLU;
        require(!glu || L->n % 2 == 0, "the gated activation needs an even number of outputs");
        const uint64_t width = glu ? L->n / 2 : L->n;
        // The argument checks of tc_qlinear_forward, with y `width` wide.
        require(x && y, "null activation/output");
        require(m >= 1 && m < (1ull << 31), "invalid row count");
        require(x_row_stride >= L->k && y_row_stride >= width, "invalid row stride");
        require((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && x_row_stride % 8 == 0,
                "activation rows must be 16-byte aligned");
        require(!adapter_count || adapters, "null adapter array");
        require(current_device() == L->device, "handle used on a different device than it was created on");
        const Plan p = plan_forward(L->type, L->dense != nullptr, L->n, L->k, m, x_row_stride, L->path);
        const Workspace ws = forward_workspace(L, p, m, adapters, adapter_count);
        if (ws.low > L->low_bytes) {
            if (L->low) hip_check(hipFree(L->low), "hipFree(LoRA workspace)");
            L->low = nullptr;
            L->low_bytes = 0;
            hip_check(hipMalloc(&L->low, ws.low), "hipMalloc(LoRA workspace)");
            L->low_bytes = ws.low;
        }
        grow_gemm_workspace(L, ws.gemm);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        if (act == TC_QLINEAR_ACT_NONE || act_in_epilogue(p, adapter_count)) {
            run_forward(L, p, ws, x, m, x_row_stride, y, y_row_stride, adapters, adapter_count, L->gemm_ws, L->low, s,
                        (int)act);
            return;
        }
        // Unfused route: the finished outputs, then the activation pass (GELU in place; the
        // gated activation from an owned [m, n] buffer).
        uint16_t *pre = y;
        uint64_t pre_stride = y_row_stride;
        if (glu) {
            const uint64_t bytes = m * L->n * sizeof(uint16_t);
            if (bytes > L->pre_bytes) {
                if (L->pre) hip_check(hipFree(L->pre), "hipFree(activation workspace)");
                L->pre = nullptr;
                L->pre_bytes = 0;
                hip_check(hipMalloc(&L->pre, bytes), "hipMalloc(activation workspace)");
                L->pre_bytes = bytes;
            }
            pre = L->pre;
            pre_stride = L->n;
        }
        run_forward(L, p, ws, x, m, x_row_stride, pre, pre_stride, adapters, adapter_count, L->gemm_ws, L->low, s);
        hip_check(tc::launch_act(pre, (int64_t)pre_stride, (int)m, (int)L->n, y, (int64_t)y_row_stride, (int)act, s),
                  "activation launch");
    });
}

// ---- allocation-free forward ---------------------------------------------------------------
// Fixed device scratch of tc_qlinear_forward_noalloc: the split-K partial sums and the runtime
// LoRA `low` rows live here instead of in per-handle workspaces. Each device holds its own copy
// (at its own address) from the library's load until the process ends. In host code the name
// `scratch` is only a host-side stand-in: kernels receive the per-device address returned by
// hipGetSymbolAddress, never the name itself.
constexpr uint64_t kNoAllocScratchBytes = TC_QLINEAR_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mutex;
void *g_noalloc_scratch[kMaxDevices];  // device address of `scratch`, per device ordinal

// The scratch address on device `dev`, which must be the current device; looked up once per
// device (the first allocation-free call on it).
void *noalloc_scratch(int dev) {
    require(dev >= 0 && dev < kMaxDevices, "device ordinal out of range for the allocation-free scratch");
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    if (!g_noalloc_scratch[dev]) {
        void *ptr = nullptr;
        hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        require(ptr != nullptr, "hipGetSymbolAddress(scratch) returned no address");
        g_noalloc_scratch[dev] = ptr;
    }
    return g_noalloc_scratch[dev];
}
}  // namespace

extern "C" int tc_qlinear_forward_noalloc(tc_qlinear *L, const uint16_t *x, uint64_t m, uint64_t x_row_stride,
                                          uint16_t *y, uint64_t y_row_stride, const tc_lora_adapter *adapters,
                                          uint32_t adapter_count, void *stream, char **error) {
    return guarded(error, [&] {
        check_forward_args(L, x, m, x_row_stride, y, y_row_stride, adapters, adapter_count);
        require(!L->dense, "the allocation-free entry point takes Q4_K / Q5_K / Q6_K weights only");
        // Split counts are lowered (never raised) until each launch's partials fit the scratch.
        const Plan p = plan_forward(L->type, false, L->n, L->k, m, x_row_stride, L->path, kNoAllocScratchBytes);
        const Workspace ws = forward_workspace(L, p, m, adapters, adapter_count, kNoAllocScratchBytes);
        require(ws.gemm <= kNoAllocScratchBytes && ws.low <= kNoAllocScratchBytes,
                "workspace exceeds the fixed scratch of the allocation-free entry point");
        // The base launches' partials are consumed (summed) before the first adapter's low is
        // written, in stream order, so both start at the scratch's base.
        void *base = noalloc_scratch(L->device);
        run_forward(L, p, ws, x, m, x_row_stride, y, y_row_stride, adapters, adapter_count, base,
                    static_cast<float *>(base), static_cast<hipStream_t>(stream));
    });
}

extern "C" int tc_qlinear_forward_many(tc_qlinear *const *linears, uint32_t count, const uint16_t *x, uint64_t m,
                                       uint64_t x_row_stride, uint16_t *const *ys, const uint64_t *y_row_strides,
                                       void *stream, char **error) {
    return guarded(error, [&] {
        require(linears && ys && y_row_strides && count >= 1, "missing linears or outputs");
        require(x && m >= 1 && m < (1ull << 31), "invalid activation");
        const tc_qlinear *L0 = linears[0];
        require(L0, "null handle");
        // One launch over all the weights: the one-row kernel (m == 1), the 2..8-row kernel, or
        // the 9..64-row skinny kernel (unsplit K, when the weights give at least 128 tiles of 64
        // rows; fewer tiles run separately, each with its own K split).
        const bool multi = m >= 2 && tc::gemv8_supports(L0->type, (int)m, (int)L0->k, (int64_t)x_row_stride);
        const bool skinny = m >= 9 && m <= 64;
        bool fuse = (m == 1 || multi || skinny) && count >= 2 && count <= (uint32_t)tc::kGemv1MaxSegments;
        int skinny_tiles = 0;
        for (uint32_t i = 0; i < count; ++i) {
            const tc_qlinear *L = linears[i];
            require(L && ys[i], "null handle or output");
            require(L->k == L0->k, "projections of one activation must share k");
            fuse = fuse && L->type == L0->type && L->device == L0->device && !L->dense &&
                   (m == 1 ? L->path != 1 : L->path == 0) && y_row_strides[i] >= L->n;
            if (skinny)
                fuse = fuse && tc::skinny_supports(L->type, (int)m, (int)L->n, (int)L->k, (int64_t)x_row_stride);
            skinny_tiles += tc::skinny_tile_count((int)L->n);
        }
        if (skinny) fuse = fuse && skinny_tiles >= 128;
        if (!fuse) {
            // Separate projections of the same activation (Weights::project_many's loop), taken
            // two at a time through the grouped GEMM where both would run the GEMM (65 rows and
            // more): one persistent grid over both weights' output tiles on the shared x.
            for (uint32_t i = 0; i < count; i += 2) {
                const uint32_t c = std::min<uint32_t>(2, count - i);
                const uint16_t *xs2[2] = {x, x};
                const uint64_t ms2[2] = {m, m}, xst2[2] = {x_row_stride, x_row_stride};
                char *err = nullptr;
                if (tc_qlinear_forward_group(linears + i, c, TC_QLINEAR_ACT_NONE, xs2, ms2, xst2, ys + i,
                                             y_row_strides + i, stream, nullptr, &err) != 0) {
                    const std::string msg = err ? err : "forward failed";
                    free(err);
                    throw Failure(msg);
                }
            }
            return;
        }
        require(x_row_stride >= L0->k && x_row_stride % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0,
                "invalid activation row");
        require(current_device() == L0->device, "handle used on a different device than it was created on");
        tc::Gemv1Segments segs{};
        segs.count = (int)count;
        segs.tile_begin[0] = 0;
        for (uint32_t i = 0; i < count; ++i) {
            segs.w[i] = linears[i]->weight;
            segs.y[i] = ys[i];
            segs.bias[i] = linears[i]->bias_bf16;
            segs.n[i] = (int)linears[i]->n;
            segs.y_stride[i] = (int64_t)y_row_strides[i];
            segs.tile_begin[i + 1] =
                segs.tile_begin[i] + (skinny ? tc::skinny_tile_count((int)linears[i]->n) : (int)((linears[i]->n + 15) / 16));
        }
        if (skinny)
            hip_check(tc::launch_skinny_segments(L0->type, x, (int64_t)x_row_stride, (int)m, segs, (int)L0->k,
                                                 static_cast<hipStream_t>(stream)),
                      "skinny launch");
        else if (m == 1)
            hip_check(tc::launch_gemv1_segments(L0->type, x, segs, (int)L0->k, static_cast<hipStream_t>(stream), 0),
                      "gemv launch");
        else
            hip_check(tc::launch_gemv8_segments(L0->type, x, (int64_t)x_row_stride, (int)m, segs, (int)L0->k,
                                                static_cast<hipStream_t>(stream), 0),
                      "gemv launch");
    });
}

extern "C" int tc_qlinear_forward_group(tc_qlinear *const *linears, uint32_t count, uint32_t act,
                                        const uint16_t *const *xs, const uint64_t *ms, const uint64_t *x_row_strides,
                                        uint16_t *const *ys, const uint64_t *y_row_strides, void *stream,
                                        uint32_t *grouped, char **error) {
    if (grouped) *grouped = 0;
    return guarded(error, [&] {
        require(linears && xs && ms && x_row_strides && ys && y_row_strides, "missing linears, activations or outputs");
        require(count >= 1 && count <= TC_QLINEAR_GROUP_MAX, "a group holds 1 or 2 projections");
        require(act <= TC_QLINEAR_ACT_SILU_GLU, "unknown output activation");
        const bool glu = act == TC_QLINEAR_ACT_SILU_GLU;
        for (uint32_t i = 0; i < count; ++i) {
            const tc_qlinear *L = linears[i];
            require(L, "null handle");
            require(!glu || L->n % 2 == 0, "the gated activation needs an even number of outputs");
            // tc_qlinear_forward's checks, with y n / 2 wide for the gated activation.
            require(xs[i] && ys[i], "null activation/output");
            require(ms[i] >= 1 && ms[i] < (1ull << 31), "invalid row count");
            require(x_row_strides[i] >= L->k && y_row_strides[i] >= (glu ? L->n / 2 : L->n), "invalid row stride");
            require((reinterpret_cast<uintptr_t>(xs[i]) & 15u) == 0 && x_row_strides[i] % 8 == 0,
                    "activation rows must be 16-byte aligned");
            require(current_device() == L->device, "handle used on a different device than it was created on");
        }
        // One grouped GEMM launch when both members would run the GEMM on their own (no tail
        // rows) with the same type, K and activation row stride; otherwise each runs its own
        // route (tc_qlinear_forward_act), in order.
        bool one = count == 2;
        if (one) {
            const tc_qlinear *A = linears[0], *B = linears[1];
            one = A->type == B->type && A->k == B->k && fused_type(A->type) && !A->dense && !B->dense &&
                  A->path == 0 && B->path == 0 && x_row_strides[0] == x_row_strides[1] &&
                  tc::gemm_group_supports((int)ms[0], (int)ms[1], (int)A->k, (int64_t)x_row_strides[0]);
            for (uint32_t i = 0; one && i < 2; ++i) {
                const Plan p = plan_forward(linears[i]->type, false, linears[i]->n, linears[i]->k, ms[i],
                                            x_row_strides[i], 0);
                one = p.kernel == TC_QLINEAR_KERNEL_GEMM && p.tail == 0;
            }
        }
        if (!one) {
            for (uint32_t i = 0; i < count; ++i) {
                char *err = nullptr;
                if (tc_qlinear_forward_act(linears[i], act, xs[i], ms[i], x_row_strides[i], ys[i], y_row_strides[i],
                                           nullptr, 0, stream, &err) != 0) {
                    const std::string msg = err ? err : "forward failed";
                    free(err);
                    throw Failure(msg);
                }
            }
            return;
        }
        tc_qlinear *A = linears[0], *B = linears[1];
        const int M[2] = {(int)ms[0], (int)ms[1]}, N[2] = {(int)A->n, (int)B->n}, K = (int)A->k;
        const int splits = tc::gemm_group_splits_within(M[0], N[0], M[1], N[1], K, UINT64_MAX);
        grow_gemm_workspace(A, tc::gemm_group_workspace_bytes(M[0], N[0], M[1], N[1], K, splits));
        const hipStream_t s = static_cast<hipStream_t>(stream);
        // Split K: the slice reduction applies the activation. Unsplit: the GEMM writes the
        // pre-activation outputs (in place for GELU, into each handle's owned [m, n] buffer for
        // the gated activation), then the activation pass.
        const bool pass = act != TC_QLINEAR_ACT_NONE && splits == 1;
        uint16_t *pre[2] = {ys[0], ys[1]};
        int64_t pre_stride[2] = {(int64_t)y_row_strides[0], (int64_t)y_row_strides[1]};
        if (pass && glu) {
            for (int i = 0; i < 2; ++i) {
                tc_qlinear *L = linears[i];
                const uint64_t bytes = ms[i] * L->n * sizeof(uint16_t);
                if (bytes > L->pre_bytes) {
                    if (L->pre) hip_check(hipFree(L->pre), "hipFree(activation workspace)");
                    L->pre = nullptr;
                    L->pre_bytes = 0;
                    hip_check(hipMalloc(&L->pre, bytes), "hipMalloc(activation workspace)");
                    L->pre_bytes = bytes;
                }
                pre[i] = L->pre;
                pre_stride[i] = (int64_t)L->n;
            }
        }
        const uint16_t *const x2[2] = {xs[0], xs[1]};
        const uint8_t *const w2[2] = {A->weight, B->weight};
        const uint16_t *const b2[2] = {A->bias_bf16, B->bias_bf16};
        hip_check(tc::launch_gemm_group(A->type, x2, (int64_t)x_row_strides[0], M, w2, N, K, pre, pre_stride, b2,
                                        splits, A->gemm_ws, s, pass ? tc::kActNone : (int)act),
                  "grouped gemm launch");
        if (pass)
            for (int i = 0; i < 2; ++i)
                hip_check(tc::launch_act(pre[i], pre_stride[i], M[i], N[i], ys[i], (int64_t)y_row_strides[i], (int)act,
                                         s),
                          "activation launch");
        if (grouped) *grouped = 1;
    });
}

extern "C" void tc_qlinear_free(tc_qlinear *linear) {
    if (!linear) return;
    if (linear->bias_bf16) (void)hipFree(linear->bias_bf16);
    if (linear->low) (void)hipFree(linear->low);
    if (linear->gemm_ws) (void)hipFree(linear->gemm_ws);
    if (linear->dense) (void)hipFree(linear->dense);
    if (linear->pre) (void)hipFree(linear->pre);
    if (linear->blas) (void)rocblas_destroy_handle(linear->blas);
    delete linear;
}
