// Internal launch interface between the C-ABI host layer (tc_qlinear.hip) and the kernel
// translation units. Every launcher validates nothing: the host layer checks geometry
// before calling, so that each kernel's grid and indexing assumptions hold.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tc {

// Output activation applied by a projection's epilogue to its bf16 outputs (after the bias):
// kActGeluTanh per output; kActSiluGlu per pair of adjacent output columns (2c, 2c + 1) =
// (gate_c, up_c), written to column c of an output N/2 wide (the weight rows of gate and up
// interleaved at bind time). Formulas: gelu_tanh_bits / silu_glu_bits (tc_device.h).
enum : int { kActNone = 0, kActGeluTanh = 1, kActSiluGlu = 2 };
// launch_gemm only: no activation, and the unsplit 128- / 256-row kernels store the output with
// ordinary (cached) stores instead of non-temporal ones, for a caller that reads the output back
// at once (the runtime LoRA pass). Other tile heights and split launches treat it as kActNone.
constexpr int kActNoneKeep = 3;

// k_decode.hip ------------------------------------------------------------------------
// Decode rows x [column_begin, column_begin + columns) of a matrix of any registered type
// ([*, source_columns]) into a strided f32/f16/bf16 target. Source row of target row r:
// d_rows ? d_rows[r] : row_begin + r. `copy`: the reference would take its same-dtype byte
// copy (a float source, target of its dtype, dense), whose non-finite error differs.
hipError_t launch_decode(uint32_t type, const uint8_t *src, uint64_t row_bytes, uint64_t source_columns,
                         const uint64_t *d_rows, uint64_t row_begin, uint64_t rows, uint64_t column_begin,
                         uint64_t columns, uint8_t *dst, uint64_t row_stride, uint64_t col_stride, uint32_t dtype,
                         int copy, int *d_err, hipStream_t stream);
hipError_t launch_quantize(uint32_t type, const float *w, uint64_t rows, uint64_t cols, uint8_t *out,
                           hipStream_t stream);
// Sets kErrNonfinite in *d_err if any block's fp16 d (or dmin) is inf/nan.
hipError_t launch_scan_scales(uint32_t type, const uint8_t *w, uint64_t nblocks, int *d_err, hipStream_t stream);
// astype(bias, bf16): f32/f16/bf16 -> bf16 RNE.
hipError_t launch_bias_to_bf16(const void *bias, uint32_t dtype, uint64_t n, uint16_t *out, hipStream_t stream);

// k_gemm.hip --------------------------------------------------------------------------
// y[M,N] = bf16(x[M,K] * deq(W)^T) (+ bias after the cast). Requires K % 256 == 0,
// x rows 16-byte aligned, W 16-byte aligned for Q4_K (2-byte for Q6_K). Grids with few
// output tiles split K over the CUs: `splits` K slices (gemm_splits_within: the preferred
// count, reduced until the fp32 partials fit `capacity` bytes; 1 = no split) whose partials
// go to `workspace` (gemm_workspace_bytes() of device memory) and are summed in a fixed order.
int gemm_splits_within(int M, int N, int K, uint64_t capacity);
size_t gemm_workspace_bytes(int M, int N, int K, int splits);
// The GEMM addresses the rows of one output tile (up to 256) from the tile's first row with
// 32-bit buffer offsets: 2 * (255 * x_stride + K) must stay below 2^31.
bool gemm_supports(int K, int64_t x_stride);
// Rows at the end of M (1..64, else 0) worth handing to the skinny kernel: the GEMM's grid of
// 256-row tiles runs in rounds of one tile per CU, and a short last row of tiles that needs a
// round of its own costs as much as a full one.
int gemm_tail_rows(int M, int N, int K);
// `act`: output activation (kAct*, or kActNoneKeep); y is N/2 wide for kActSiluGlu (N even).
hipError_t launch_gemm(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                       uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, int splits, void *workspace,
                       hipStream_t stream, int act = kActNone);
// Grouped launch: two problems of one weight type and K whose activations share a row stride
// (y_i[M_i, N_i] = bf16(x_i * deq(W_i)^T) (+ bias_i)) in one persistent grid over the output
// tiles of both, so that two small GEMMs fill the CUs together. Both need M >= 65 (128- or
// 256-row tiles, chosen from the two problems' tiles together, as are the K slices).
bool gemm_group_supports(int M0, int M1, int K, int64_t x_stride);
int gemm_group_splits_within(int M0, int N0, int M1, int N1, int K, uint64_t capacity);
size_t gemm_group_workspace_bytes(int M0, int N0, int M1, int N1, int K, int splits);
// `act` (kAct*) only with splits > 1: the slice reduction applies it (y[i] is N[i] / 2 wide
// for kActSiluGlu).
hipError_t launch_gemm_group(uint32_t type, const uint16_t *const x[2], int64_t x_stride, const int M[2],
                             const uint8_t *const w[2], const int N[2], int K, uint16_t *const y[2],
                             const int64_t y_stride[2], const uint16_t *const bias_bf16[2], int splits,
                             void *workspace, hipStream_t stream, int act = kActNone);

// k_gemv.hip --------------------------------------------------------------------------
// Skinny path for M <= 8: exact fp32 weights (a*q - b folded per sub-block), fp32 sums.
hipError_t launch_gemv(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                       uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, hipStream_t stream);

// k_gemv1.hip -------------------------------------------------------------------------
// M = 1: exact fp32 weights, dot products on the matrix cores with a block-diagonal
// activation operand. force_waves (0 = automatic) sets the wavefronts per workgroup.
hipError_t launch_gemv1(uint32_t type, const uint16_t *x, const uint8_t *w, int N, int K, uint16_t *y,
                        const uint16_t *bias_bf16, hipStream_t stream, int force_waves, int act = kActNone);
// Several weight matrices of one type and K applied to the same row x in one launch (fused
// projections such as q/k/v or gate/up): segment s covers 16-row tiles
// [tile_begin[s], tile_begin[s + 1]) of the grid, tile_begin[s + 1] - tile_begin[s] =
// ceil(n[s] / 16).
constexpr int kGemv1MaxSegments = 8;
struct Gemv1Segments {
    const uint8_t *w[kGemv1MaxSegments];
    uint16_t *y[kGemv1MaxSegments];
    const uint16_t *bias[kGemv1MaxSegments];
    int n[kGemv1MaxSegments];
    int64_t y_stride[kGemv1MaxSegments];  // y row stride (elements; the multi-row kernel)
    int tile_begin[kGemv1MaxSegments + 1];
    int count;
    int act;  // output activation of every segment (kAct*; y[s] is n[s]/2 wide for kActSiluGlu)
};
hipError_t launch_gemv1_segments(uint32_t type, const uint16_t *x, const Gemv1Segments &segs, int K,
                                 hipStream_t stream, int force_waves);

// k_gemv8.hip -------------------------------------------------------------------------
// 2 <= M <= 8 rows, Q4_K / Q6_K: exact fp32 weights, one MFMA per 32-column step over all
// rows, scales applied to the outputs. Requires K % 256 == 0, 16-byte aligned x rows (and
// Q4_K weights). The segment form runs several matrices of one type and K on the same x
// (fused projections), as launch_gemv1_segments does for one row.
bool gemv8_supports(uint32_t type, int M, int K, int64_t x_stride);
hipError_t launch_gemv8(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                        uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, hipStream_t stream, int force_w,
                        int act = kActNone);
hipError_t launch_gemv8_segments(uint32_t type, const uint16_t *x, int64_t x_stride, int M,
                                 const Gemv1Segments &segs, int K, hipStream_t stream, int force_w);

// k_skinny.hip ------------------------------------------------------------------------
// 1 <= M <= 64 rows, Q4_K / Q6_K (used for 9..64): bf16-rounded exact weights (the GEMM's
// decode), fp32 accumulation, activations shared through LDS, no per-tile partial planes.
// Requires K % 256 == 0, 16-byte aligned x rows (and Q4_K weights). Few-tile grids split K
// into `splits` slices (skinny_splits_within: the preferred count reduced until the fp32
// partials fit `capacity` bytes; 1 = no split) whose partials go to `workspace`
// (skinny_workspace_bytes() of device memory) and are summed in a fixed order.
bool skinny_supports(uint32_t type, int M, int N, int K, int64_t x_stride);
int skinny_splits_within(int M, int N, int K, uint64_t capacity);
size_t skinny_workspace_bytes(int M, int N, int splits);
hipError_t launch_skinny(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                         uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, int splits, void *workspace,
                         hipStream_t stream, int act = kActNone);
// 64-row weight tiles of an N-row matrix (the skinny kernel's grid unit).
int skinny_tile_count(int N);
// Several weight matrices of one type and K on the same x in one launch (fused projections),
// K not split: segment s covers 64-row tiles [tile_begin[s], tile_begin[s + 1]),
// tile_begin[s + 1] - tile_begin[s] = skinny_tile_count(n[s]).
hipError_t launch_skinny_segments(uint32_t type, const uint16_t *x, int64_t x_stride, int M,
                                  const Gemv1Segments &segs, int K, hipStream_t stream);

// k_lora.hip --------------------------------------------------------------------------
// One runtime LoRA adapter as the kernels see it (all row/column indices relative to the
// call's x / y). low: the adapter's fp32 workspace, ksplit planes of [row_count, low_stride],
// low_stride a multiple of 8, 16-byte aligned. b_vec: B rows are 16-byte aligned (rank % 8 == 0 and an
// aligned base), allowing 16-byte loads of B.
struct LoraDesc {
    const uint16_t *a;  // [rank, K] bf16
    const uint16_t *b;  // [out_count, rank] bf16
    float *low;
    int rank, low_stride;
    int row_begin, row_count;
    int out_begin, out_count;
    float scale;
    int b_vec;
    int ksplit;          // K slices of low (partial planes, summed by the epilogue in slice order)
    int64_t low_plane;   // floats between the planes
};
constexpr int kLoraBatch = 8;
struct LoraBatch {
    LoraDesc d[kLoraBatch];
    int count;
};
// low = x[row_begin .. row_begin + row_count, K] * A^T for every adapter of the batch (fp32
// accumulation of exact bf16 products). Requires K % 256 == 0 and 16-byte aligned x / A rows.
hipError_t launch_lora_low(const uint16_t *x, int64_t x_stride, int K, const LoraBatch &batch, hipStream_t stream);
// One pass over y[M, N]: for each adapter in order, on its rows and output columns,
// y = bf16(f32(y) + f32(scale * f32(low . B))); then, when bias_bf16 is given, over all of y,
// y = bf16(f32(y) + f32(bias)).
hipError_t launch_lora_epilogue(uint16_t *y, int64_t y_stride, int M, int N, const LoraBatch &batch,
                                const uint16_t *bias_bf16, hipStream_t stream);

// k_act.hip ---------------------------------------------------------------------------
// The output activation as a pass of its own over finished projection outputs pre[M, N]
// (the routes whose epilogue does not apply it: runtime LoRA, the library GEMM, the forced
// per-row GEMV): y = act(pre), y N/2 wide for kActSiluGlu. y may alias pre for kActGeluTanh.
hipError_t launch_act(const uint16_t *pre, int64_t pre_stride, int M, int N, uint16_t *y, int64_t y_stride, int act,
                      hipStream_t stream);

}  // namespace tc
