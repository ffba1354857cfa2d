/*
 * tc_qlinear -- MI355X (gfx950) GGUF K-quant quantized-linear operator ABI.
 *
 * Additive to the reference's C ABI 1 and following its conventions
 * (bindings/c/include/turbocider/turbocider.h:7-12, native/api/c_api.mm:79-90,382-391):
 *   - plain extern "C", no exceptions cross the boundary;
 *   - functions return int status: 0 ok, 1 error, 2 cancelled;
 *   - `char **error` (nullable) receives a strdup'd message on failure, released by the
 *     caller with tc_qlinear_string_free; out-params are nulled on entry;
 *   - opaque handles follow create / use / free (tc_coreml_ffn_*, turbocider.h:102-112),
 *     and one handle is used by one thread at a time (an engine serializes generation,
 *     turbocider.h:8).
 *
 * Memory: every tensor pointer below is a DEVICE pointer (HIP global memory on the
 * current device) unless documented otherwise. Work is enqueued on `stream`
 * (a hipStream_t; NULL = the default stream). Functions marked "synchronous" wait for
 * `stream` before returning so that device-side error flags can be reported.
 *
 * Layouts are the GGUF ones: a K-quant weight of logical shape [N, K] (GGML ne0 = K is
 * contiguous, native/core/gguf_directory.hpp:60-71) is N rows of K/256 raw super-blocks
 * (block_q4_K: 144 bytes, block_q6_K: 210 bytes), rows back to back, exactly as stored in
 * the .gguf file. Activations and outputs are row-major bf16 bit patterns.
 */
#ifndef TC_QLINEAR_H
#define TC_QLINEAR_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define TC_QLINEAR_ABI_VERSION 1u

/* GGML tensor type ids (native/core/gguf_directory.hpp:21-26). The quantized projection reads
 * Q4_K, Q5_K and Q6_K blocks in its own kernels; the decoder takes every one below. */
#define TC_GGML_TYPE_F32 0u
#define TC_GGML_TYPE_F16 1u
#define TC_GGML_TYPE_Q4_0 2u
#define TC_GGML_TYPE_Q4_1 3u
#define TC_GGML_TYPE_Q5_0 6u
#define TC_GGML_TYPE_Q5_1 7u
#define TC_GGML_TYPE_Q8_0 8u
#define TC_GGML_TYPE_Q4_K 12u
#define TC_GGML_TYPE_Q5_K 13u
#define TC_GGML_TYPE_Q6_K 14u
#define TC_GGML_TYPE_BF16 30u

/* Element types; same order as tc::gguf::DecodeDType (native/core/gguf_decode.hpp:18). */
#define TC_DTYPE_F32 0u
#define TC_DTYPE_F16 1u
#define TC_DTYPE_BF16 2u

/* Replaces: tc_abi_version (turbocider.h:24) for this operator family. */
uint32_t tc_qlinear_abi_version(void);

/* Replaces: tc_string_free (turbocider.h:7; c_api.mm:382-384). Frees strings returned in
 * `char **error`. Exported under a distinct name so that it can be linked beside the
 * reference's libturbocider without a duplicate symbol. */
void tc_qlinear_string_free(char *s);

/* Decode receipt; mirrors tc::gguf::DecodeReceipt (gguf_decode.hpp:39-43). simd_blocks
 * counts super-blocks decoded by the device fast path. */
typedef struct tc_decode_receipt {
    uint64_t source_bytes_processed, elements_written, bytes_written, scratch_bytes, simd_blocks;
} tc_decode_receipt;

/*
 * Device decode of a matrix slice of any TC_GGML_TYPE_* above. Replaces
 * tc::gguf::decode_cpu_into (native/core/gguf_decode.hpp:56-58; gguf_decode.cpp:433-445),
 * with the reference probe's flat argument order (tests/native/gguf_core_probe.cpp:32):
 *   source [source_rows, source_columns] raw blocks (source_bytes long);
 *   slice rows [row_begin, row_begin + rows) x columns [column_begin, column_begin + columns);
 *   target element (r, c) at byte offset r * row_stride + c * column_stride, dtype TC_DTYPE_*.
 * If `row_indices` (HOST array of `rows` entries, caller-owned like the reference's span)
 * is non-NULL the source rows are gathered in that order instead, duplicates allowed
 * (decode_cpu_gather, gguf_decode.hpp:62-65; every index is checked before any write),
 * and `row_begin` must be 0. Geometry is validated on the host exactly as
 * gguf_decode.cpp:160-183 does (overflow, slice bounds, strides, target size, no overlap
 * between source and target). Values are bit-identical to the reference: fp32
 * w = (d*sc)*q - dmin*m (Q4_K/Q5_K), (d*sc)*(q-32) (Q6_K), code*scale [+ minimum] (Q4_0,
 * Q4_1, Q5_0, Q5_1, Q8_0; gguf_decode.cpp:59-76) or the element itself (F32 / F16 / BF16),
 * then RNE to bf16/fp16. A non-finite scale/minimum or element returns 1 with
 * "nonfinite weight/scale or conversion overflow" ("nonfinite source float" where the
 * reference copies a float source into its own dtype, gguf_decode.cpp:119-158), a target
 * overflow "FP16 conversion overflow" / "BF16 conversion overflow"; the target is then
 * partially written and must be discarded (gguf_decode.hpp:53-55).
 * `cancel` (host pointer, nullable) set on entry returns 2 before any write.
 * Synchronous.
 */
int tc_gguf_decode_device(uint32_t ggml_type, const void *source, uint64_t source_bytes,
                          uint64_t source_rows, uint64_t source_columns, uint64_t row_begin,
                          uint64_t rows, uint64_t column_begin, uint64_t columns, uint32_t dtype,
                          void *target, uint64_t target_bytes, uint64_t row_stride,
                          uint64_t column_stride, const uint64_t *row_indices,
                          const volatile int *cancel, void *stream, tc_decode_receipt *receipt,
                          char **error);

/*
 * Host-pointer decode: the same arguments as tc_gguf_decode_device without the stream, on HOST
 * buffers. Replaces tc::gguf::decode_cpu_into / decode_cpu_gather (native/core/gguf_decode.hpp:
 * 56-65; gguf_decode.cpp:320-367,433-465) for callers that decode on the CPU (the reference's
 * pager fills, gguf_weight_pager.cpp:347-349,571-573): the same validation, messages, values,
 * error order and receipt (scratch_bytes 1024; simd_blocks 0, there is no vector path). `cancel`
 * is polled on entry, before every block (every element of a same-dtype float copy) and on exit:
 * status 2 "gguf_decode_cancelled", the target then partially written. Synchronous, reentrant,
 * allocation-free; concurrent calls on disjoint row ranges may split one matrix.
 */
int tc_gguf_decode_host(uint32_t ggml_type, const void *source, uint64_t source_bytes, uint64_t source_rows,
                        uint64_t source_columns, uint64_t row_begin, uint64_t rows, uint64_t column_begin,
                        uint64_t columns, uint32_t dtype, void *target, uint64_t target_bytes, uint64_t row_stride,
                        uint64_t column_stride, const uint64_t *row_indices, const volatile int *cancel,
                        tc_decode_receipt *receipt, char **error);

/*
 * Device quantizer, fp32 [rows, columns] -> raw Q4_K / Q6_K blocks (columns % 256 == 0).
 * The reference ships no quantizer (it only decodes files produced by ggml); this exists so
 * that synthetic weights can be made on the device. Asynchronous.
 */
int tc_gguf_quantize_device(uint32_t ggml_type, const float *weights, uint64_t rows, uint64_t columns,
                            void *blocks, uint64_t block_bytes, void *stream, char **error);

/* ------------------------------------------------------------------------------------
 * Quantized linear: y[M, N] = x[M, K] * deq(W)^T  (+ runtime LoRA) (+ bias)
 * Replaces: Weights::project, quantized branch (native/backends/mlx.hpp:203;
 * native/backends/mlx.cpp:626-690: mx::quantized_matmul + add_runtime_projection_loras +
 * bias) and the opt-in Metal kernels affine_gpu::projection_shared
 * (affine_gpu_shared.hpp:22-85) and dense_gpu::lora_b_epilogue (dense_gpu_lora_b.hpp:16-55).
 * ------------------------------------------------------------------------------------ */
typedef struct tc_qlinear tc_qlinear;

/* ggml_type: Q4_K / Q5_K / Q6_K run the fused dequant kernels on the raw blocks (Q5_K: the
 * M = 1 GEMV and the MFMA dequant-GEMM for every other row count; Q4_K / Q5_K weights 16-byte
 * aligned, Q6_K 4-byte aligned). Every other
 * TC_GGML_TYPE_* is decoded once at create time into an owned bf16 [n, k] copy (bit-exact to
 * the reference decoder; n * k * 2 bytes) and multiplied by the library GEMM (rocBLAS, fp32
 * accumulation), the reference's dense branch of Weights::project for such tensors
 * (native/backends/mlx.cpp:680-686); bias and runtime LoRA as for the K-quants. */
typedef struct tc_qlinear_desc {
    uint32_t ggml_type;   /* any TC_GGML_TYPE_* (see above) */
    uint64_t n, k;        /* output features (weight rows), input features (k % 256 == 0) */
    const void *weight;   /* device: n rows of raw GGUF blocks; borrowed until tc_qlinear_free */
    uint64_t weight_bytes;
    const void *bias;     /* device: [n] of bias_dtype, or NULL; borrowed */
    uint32_t bias_dtype;  /* TC_DTYPE_F32 / F16 / BF16 (cast to bf16 like astype, mlx.cpp:688) */
} tc_qlinear_desc;

/* One runtime (unmerged) LoRA application, mirroring a bound RuntimeLoRA entry
 * (mlx.cpp:1456-1459: {down, up, scale, output_start, output_end}). The reference applies
 * every adapter to all rows (mlx.cpp:692-722); `row_begin/row_count` restrict it to a row
 * segment so that different images of one batch can carry different adapters. Adapters
 * are applied in array order, each rounding y to bf16 once; the bias is added after all
 * of them (mlx.cpp:686-688). */
typedef struct tc_lora_adapter {
    const uint16_t *a;     /* device bf16 "down"/lora_A [rank, k], row-major */
    const uint16_t *b;     /* device bf16 "up"/lora_B [output_end - output_begin, rank] */
    uint32_t rank;         /* 1..1024 */
    float scale;           /* effective scale: strength * (alpha / rank if alpha) (mlx.cpp:1442-1452) */
    uint64_t row_begin, row_count;        /* rows of x / y this adapter applies to */
    uint64_t output_begin, output_end;    /* output columns (fused targets, mlx.cpp:703-717) */
} tc_lora_adapter;

/* Validates geometry and scans every super-block's fp16 d/dmin once (non-finite -> status 1,
 * "nonfinite weight/scale or conversion overflow", like gguf_decode.cpp:78,92). The weight
 * and bias memory stay owned by the caller. Synchronous (on the NULL stream). */
int tc_qlinear_create(const tc_qlinear_desc *desc, tc_qlinear **out, char **error);

/*
 * y = bf16(x * deq(W)^T); for each adapter in order y = bf16(f32(y) + f32(scale * delta))
 * with delta = f32(low * B^T), low = f32(x * A^T); then y = bf16(f32(y) + f32(bf16(bias))).
 * x: [m, k] bf16 with row stride x_row_stride (elements); y: [m, n] bf16, stride
 * y_row_stride. m >= 1. Asynchronous on `stream`; the handle's internal workspace
 * (grown on demand) is reused by the next call, so calls on one handle must not overlap.
 */
int tc_qlinear_forward(tc_qlinear *linear, const uint16_t *x, uint64_t m, uint64_t x_row_stride,
                       uint16_t *y, uint64_t y_row_stride, const tc_lora_adapter *adapters,
                       uint32_t adapter_count, void *stream, char **error);

/*
 * Projection with an output activation applied in the kernels' epilogue: y = act(forward(x)),
 * the activation evaluated in fp32 on each finished bf16 output (after the bias and any
 * runtime adapters) and rounded once to bf16 (RNE). Replaces the projection + activation
 * pairs of the reference's MLPs:
 *   TC_QLINEAR_ACT_GELU_TANH: gelu(project(x)), 0.5 z (1 + tanh(sqrt(2/pi) (z + 0.044715 z^3)))
 *     (native/models/qwen21/transformer.cpp:48-57, the text-input MLP at :628);
 *   TC_QLINEAR_ACT_SILU_GLU: silu(gate) * up of a gate_up projection
 *     (native/models/qwen21/transformer.cpp:971-975; silu = x sigmoid(x),
 *     native/backends/mlx.cpp:1627-1631). The handle's weight rows (and bias) must hold gate and
 *     up interleaved, row 2c = gate row c, row 2c + 1 = up row c (qlinear.glu_pair_rows builds
 *     them at bind time); y is n/2 wide: y[:, c] = silu(z[:, 2c]) * z[:, 2c + 1].
 * The reference rounds every intermediate of its activation ops to the activation dtype; this
 * entry point rounds once, so outputs may differ from that chain by the chain's own rounding.
 * The GEMM, GEMV and skinny kernels apply the activation in their epilogue (no pre-activation
 * round trip through memory); with runtime adapters or other types it is a second pass.
 * Asynchronous on `stream`; arguments and errors as tc_qlinear_forward, with y n/2 wide for
 * the gated activation (odd n: status 1).
 */
#define TC_QLINEAR_ACT_NONE 0u
#define TC_QLINEAR_ACT_GELU_TANH 1u
#define TC_QLINEAR_ACT_SILU_GLU 2u
int tc_qlinear_forward_act(tc_qlinear *linear, uint32_t act, const uint16_t *x, uint64_t m, uint64_t x_row_stride,
                           uint16_t *y, uint64_t y_row_stride, const tc_lora_adapter *adapters,
                           uint32_t adapter_count, void *stream, char **error);

/*
 * Allocation-free variant of tc_qlinear_forward: the same arguments, results and errors, but no
 * device memory is allocated or freed during the call (no hipMalloc / hipFree, no allocating
 * library routine). No counterpart in the reference: it exists for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid it).
 *   - The split-K partial sums and runtime-LoRA `low` rows go to a fixed scratch array of
 *     TC_QLINEAR_NOALLOC_SCRATCH_BYTES in device memory, one per device, held from the
 *     library's load until the process ends; no state persists between calls that a caller
 *     must clear.
 *   - Where tc_qlinear_forward would split K into partials larger than the scratch, this entry
 *     point uses fewer K slices (same values up to the fp32 summation order); runtime adapters
 *     whose `low` rows at one K slice exceed the scratch are rejected (status 1).
 *   - Q4_K / Q5_K / Q6_K weights only (other types run a library GEMM that may allocate):
 *     status 1.
 *   - Every call on one device shares that device's scratch: calls that overlap on one device
 *     (on different streams or threads, or with tc_qlinear_forward_noalloc calls of other
 *     handles) race and must be serialized by the caller.
 * Asynchronous on `stream`.
 */
#define TC_QLINEAR_NOALLOC_SCRATCH_BYTES (32ull << 20)
int tc_qlinear_forward_noalloc(tc_qlinear *linear, const uint16_t *x, uint64_t m, uint64_t x_row_stride,
                               uint16_t *y, uint64_t y_row_stride, const tc_lora_adapter *adapters,
                               uint32_t adapter_count, void *stream, char **error);

/*
 * Several projections of the same activation: ys[i] = forward(linears[i], x) without runtime
 * LoRA (apply adapters with tc_qlinear_forward). Replaces Weights::project_many
 * (native/backends/mlx.hpp:204, mlx.cpp:724-760; q/k/v at native/components/text/qwen3.cpp:
 * 216-218). For m <= 8 rows (Q4_K / Q6_K for m >= 2) with up to 8 weights of one type and k,
 * the projections run as one fused launch (the M = 1 GEMV, or the 2..8-row GEMV, over all
 * their row tiles), and likewise for 9..64 rows (the skinny kernel, K unsplit) when the
 * weights hold at least 128 tiles of 64 rows; otherwise one after the other.
 * Asynchronous on `stream`.
 */
int tc_qlinear_forward_many(tc_qlinear *const *linears, uint32_t count, const uint16_t *x, uint64_t m,
                            uint64_t x_row_stride, uint16_t *const *ys, const uint64_t *y_row_strides,
                            void *stream, char **error);

/*
 * Projections of different activations in one launch: ys[i][ms[i], n_i] = act(xs[i] . W_i^T
 * (+ bias_i)) for i < count (1 or 2; no runtime LoRA; `act` TC_QLINEAR_ACT_* as in
 * tc_qlinear_forward_act, ys n_i / 2 wide for the gated activation). Two projections with the same weight
 * type (Q4_K / Q5_K / Q6_K) and k, equal activation row strides, automatic path and a GEMM
 * route of their own (ms >= 65, no tail rows) run as ONE persistent dequant-GEMM grid over the
 * output tiles of both (grouped GEMM; *grouped = 1), so that two small GEMMs fill the
 * device's compute units together; otherwise each runs tc_qlinear_forward's route in order
 * (*grouped = 0). For the two streams of a dual-stream (MMDiT) block, whose image and text
 * tokens pass through separate weights of the same shape: the reference projects them one
 * after the other (qkv, attention out and feed-forward of each stream,
 * native/models/flux2/flux_transformer.cpp:995-1004, each a Weights::project call,
 * native/backends/mlx.cpp:626-690). The results equal what each projection gives on its own
 * up to the order of the fp32 K summation (the group may choose another tile height or K
 * split).
 * Split-K partial sums use the first handle's workspace. `grouped` may be null.
 */
#define TC_QLINEAR_GROUP_MAX 2u
int tc_qlinear_forward_group(tc_qlinear *const *linears, uint32_t count, uint32_t act, const uint16_t *const *xs,
                             const uint64_t *ms, const uint64_t *x_row_strides, uint16_t *const *ys,
                             const uint64_t *y_row_strides, void *stream, uint32_t *grouped, char **error);

/* Kernel selection hint for measurement and tests: 0 = automatic (default: the M = 1 GEMV
 * for one row, the 2..8-row GEMV at 2 <= m <= 8, the skinny kernel at 9 <= m <= 64, else the
 * MFMA dequant-GEMM with 128- or 256-row tiles; each for Q4_K / Q5_K / Q6_K), 1 = force the
 * MFMA dequant-GEMM, 2 = force the one-row GEMV per row (m <= 8 only; Q4_K / Q6_K for m >= 2),
 * 3 = force the skinny kernel for Q4_K / Q5_K / Q6_K at m <= 64 (the GEMM otherwise). */
int tc_qlinear_set_path(tc_qlinear *linear, uint32_t path, char **error);

/* Kernel routes of tc_qlinear_forward (tc_qlinear_plan_info.kernel). */
#define TC_QLINEAR_KERNEL_GEMM 1u    /* MFMA dequant-GEMM (128/256-row tiles; 32/64 when forced) */
#define TC_QLINEAR_KERNEL_GEMV1 2u   /* M = 1 GEMV */
#define TC_QLINEAR_KERNEL_GEMV8 3u   /* 2 <= M <= 8 GEMV */
#define TC_QLINEAR_KERNEL_SKINNY 4u  /* 9 <= M <= 64 skinny kernel */
#define TC_QLINEAR_KERNEL_GEMV 5u    /* forced one-row GEMV per row (path 2, M <= 8) */
#define TC_QLINEAR_KERNEL_DENSE 6u   /* types other than Q4_K / Q5_K / Q6_K: decoded bf16 copy, library GEMM */

typedef struct tc_qlinear_plan_info {
    uint32_t kernel;          /* TC_QLINEAR_KERNEL_* */
    uint32_t tail_rows;       /* GEMM: rows at the end of M run by the skinny kernel after it */
    uint64_t workspace_bytes; /* split-K partial sums the base launches need (without LoRA) */
} tc_qlinear_plan_info;

/*
 * The route tc_qlinear_forward takes for a handle of this type and geometry with `m` rows of
 * stride `x_row_stride` and kernel selection `path` (tc_qlinear_set_path), decided on the host
 * from the geometry alone; needs no device and touches no device memory. Returns 1 with
 * tc_qlinear_forward's message for a call it would reject (e.g. an activation row stride too
 * large for the kernels' 32-bit buffer offsets). No counterpart in the reference (its
 * Weights::project has a single route); it exists so that callers and tests can see which
 * kernel a shape runs and what workspace it needs.
 */
int tc_qlinear_plan(uint32_t ggml_type, uint64_t n, uint64_t k, uint64_t m, uint64_t x_row_stride, uint32_t path,
                    tc_qlinear_plan_info *out, char **error);

void tc_qlinear_free(tc_qlinear *linear);

/* ---- GGUF container reader (host) --------------------------------------------------------
 * Replaces tc::gguf::read_directory / validate_split_set (native/core/gguf_directory.hpp:
 * 199-304, types :19-26, limits :45-50): the same checks and "gguf_invalid: <reason>" /
 * "gguf_type_unsupported: <id>" / "gguf_tensor_missing: <name>" messages. The reader keeps
 * the file open (a held fd, like the reference's lease) and uploads raw tensor payloads to
 * device memory; it never decodes on the host. Strings returned in the info structs stay
 * valid until tc_gguf_close. */
typedef struct tc_gguf_file tc_gguf_file;

typedef struct tc_gguf_summary {
    uint32_t version, alignment;
    uint64_t tensor_count, metadata_count, file_bytes, data_offset;
} tc_gguf_summary;

/* One tensor descriptor (gguf_directory.hpp:59-70): dims in GGML order, dims[0] contiguous. */
typedef struct tc_gguf_tensor_info {
    const char *name;
    uint32_t ggml_type, rank;
    uint64_t dims[4];
    uint64_t elements, bytes, file_offset, relative_offset;
} tc_gguf_tensor_info;

/* One metadata entry (gguf_directory.hpp:51-58): scalar value fields by GGUF value type
 * (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64,
 * 12 f64); arrays report element_type and count only. */
typedef struct tc_gguf_meta_value {
    uint32_t type, element_type;
    uint64_t count, unsigned_value;
    int64_t signed_value;
    double float_value;
    const char *text;
    uint64_t text_bytes;
} tc_gguf_meta_value;

/* Opens and parses the directory (reads only the directory bytes). */
int tc_gguf_open(const char *path, tc_gguf_file **out, char **error);
void tc_gguf_close(tc_gguf_file *file);
/* Returns 0 and fills `out`; 1 on a null argument. */
int tc_gguf_describe(const tc_gguf_file *file, tc_gguf_summary *out);
int tc_gguf_tensor(const tc_gguf_file *file, uint64_t index, tc_gguf_tensor_info *out, char **error);
int tc_gguf_find_tensor(const tc_gguf_file *file, const char *name, uint64_t *index, char **error);
int tc_gguf_meta(const tc_gguf_file *file, const char *key, tc_gguf_meta_value *out, char **error);
/* Split-set consistency (gguf_directory.hpp:269-304); a lone file without split keys passes. */
int tc_gguf_validate_split(const tc_gguf_file *const *shards, uint32_t count, char **error);
/* Copies tensor `index`'s raw payload (bytes as in the file) to device memory
 * `device_dst` (at least info.bytes long) through pinned bounce buffers. Synchronous. */
int tc_gguf_read_tensor(const tc_gguf_file *file, uint64_t index, void *device_dst, uint64_t dst_bytes,
                        void *stream, char **error);

/* ---- Weight pager (host <-> device streaming of raw GGUF blocks) --------------------------
 * Replaces the reference's GgufWeightPager fill / bind / retire
 * (native/runtime/streaming/gguf_weight_pager.hpp:27-53) and its slot safety tracker
 * (slot_pool.hpp:11-45) for models whose weights do not all fit in device memory. Groups of
 * tensors (e.g. one transformer block's projections) are filled into a bounded set of
 * caller-owned device slots as their raw payloads at 256-byte aligned offsets
 * (tc_pager_group_layout), read by a worker thread through pinned bounce buffers and uploaded
 * on the pager's own copy stream, so that fills overlap compute.
 *   tc_pager_fill:    a Vacant or AwaitingFence slot starts loading `group` (asynchronous; the
 *                     upload waits on the device for the slot's last reader fence); returns a
 *                     ticket. `cancel`, when set, stops the fill between 4 MiB chunks.
 *   tc_pager_acquire: waits until the fill's reads are issued; `stream` (NULL: the host) then
 *                     waits for its upload. Status 2 when the fill was cancelled, 1 when it
 *                     failed ("gguf_pager: payload read failed or source changed"); the slot is
 *                     then vacant again.
 *   tc_pager_release: the reader fence, recorded on `stream` after the last use of the slot.
 * Stale tickets (a slot refilled since) and out-of-order calls are rejected (status 1). The
 * file handle and the slot buffers must outlive the pager; tc_pager_free finishes queued fills.
 * One thread drives a pager (its calls are serialized by an internal lock). */
typedef struct tc_pager tc_pager;
typedef struct tc_pager_ticket {
    uint32_t group, slot;
    uint64_t generation;
} tc_pager_ticket;
typedef struct tc_pager_metrics {
    uint64_t fills, bytes_read;
    double read_seconds;  /* worker time reading and issuing uploads */
    double wait_seconds;  /* caller time blocked in tc_pager_acquire */
} tc_pager_metrics;
/* group_begin[group_count + 1]: group g holds tensor_indices[group_begin[g] .. group_begin[g+1]). */
int tc_pager_create(const tc_gguf_file *file, uint32_t group_count, const uint32_t *group_begin,
                    const uint64_t *tensor_indices, uint32_t slot_count, void *const *slot_buffers, uint64_t slot_bytes,
                    tc_pager **out, char **error);
int tc_pager_group_layout(const tc_pager *pager, uint32_t group, uint64_t *offsets, uint32_t capacity, uint32_t *count,
                          uint64_t *bytes, char **error);
int tc_pager_fill(tc_pager *pager, uint32_t group, uint32_t slot, const volatile int *cancel, tc_pager_ticket *ticket,
                  char **error);
int tc_pager_acquire(tc_pager *pager, const tc_pager_ticket *ticket, void *stream, char **error);
int tc_pager_release(tc_pager *pager, const tc_pager_ticket *ticket, void *stream, char **error);
int tc_pager_get_metrics(tc_pager *pager, tc_pager_metrics *out);
void tc_pager_free(tc_pager *pager);

#ifdef __cplusplus
}
#endif
#endif
