// Fused K-quant dequant + bf16 MFMA GEMM for gfx950:  y[M,N] = bf16(x[M,K] * deq(W)^T) (+bias).
//
// Replaces the reference's Metal quantized matmul (mx::quantized_matmul affine QMM,
// native/backends/mlx.cpp:678-679, and affine_gpu::projection_shared,
// native/backends/affine_gpu_shared.hpp:41-84), decoding raw GGUF blocks instead of the
// reference's lossy affine repack (native/core/gguf_affine.cpp:147-307).
//
// Kernel template shared by the per-variant translation units (k_gemm_variant.hip, compiled
// once per (TYPE, SPLIT, MT)); the dispatch is in k_gemm.hip.
//
// Tiling (one workgroup of 4 wavefronts):
//   * block tile 32 MT (M) x 256 (N), MT = 8 for large M (one wavefront per SIMD), 2 or 1
//     for skinny M (64 / 32 rows; up to two workgroups per CU); wavefront w owns all rows
//     of the tile and the 64 columns [64w, 64w + 64) of N as MT x 2 tiles of
//     v_mfma_f32_32x32x16_bf16, so every weight is dequantized exactly once per workgroup;
//   * the K loop walks 64-wide chunks. A chunk is one 32-byte qs segment of a Q4_K block
//     (sub-blocks 2p and 2p+1: low and high nibbles), or one ql segment of a Q6_K block
//     (sub-blocks p and p+2). Its K set is two 32-wide runs, seg0 and seg1; the MFMA K
//     order inside a chunk follows the nibble layout, which is legal because the sum over
//     K does not depend on the order in which A and B visit it;
//   * activations for the chunk (256 rows x 64 bf16) are copied global -> LDS by the
//     buffer-load DMA, four chunks ahead, into four 32 KB buffers (16-byte pieces XOR
//     swizzled per row so that fragment reads do not conflict); the raw weight bytes go
//     straight from global memory to registers (16-byte loads, two chunks ahead), are
//     dequantized to bf16 in registers by the lane that feeds them to the MFMA, and never
//     touch LDS;
//   * persistent workgroups (one per CU) walk their output tiles as one K stream: the
//     prefetches of a tile's last super-block already fetch the next tile's first chunks,
//     and the epilogue's stores stay in flight under the next tile's first chunks.
// Dequantization is bit-exact: fp32 fma(d*sc, q, -dmin*m) (Q4_K) / (d*sc)*(q-32) (Q6_K)
// rounded once (every product is exact), then RNE to bf16 (v_cvt_pk_bf16_f32).
// Epilogue: y = RNE_bf16(acc); with a bias y = RNE_bf16(f32(y) + f32(bias_bf16))
// (bias added after the cast, native/backends/metal_graph/kernels/dense_linear.hpp:139-141).
#pragma once
#include "k_gemm.h"
#include "tc_device.h"
#include "tc_kernels.h"

#include <algorithm>
#include <type_traits>

namespace tc {
namespace {

constexpr int kBN = 256, kThreads = 256;

// Raw weight bytes of one chunk for one 32-column MFMA tile, kept exactly as loaded (any
// arithmetic on them at load time would make the load wait for its data immediately).
struct WRegs {
    u32x4 q;  // Q4_K / Q5_K: 16 qs bytes; Q6_K: 16 ql bytes
    u32x4 h;  // Q6_K: 16 qh bytes (unused otherwise)
};
// Per-super-block bytes of one row, loaded once per block (not per chunk).
struct BRegs {
    u32x4 s;     // Q4_K / Q5_K: block header (d, dmin, 12 scale bytes); Q6_K: the 16 int8 scales
    uint32_t d;  // Q6_K: d (fp16 bits); unused otherwise
    u32x4 qh;    // Q5_K: the lane's 16 high-bit bytes (columns 16h .. 16h + 15 of every group)
};
// Q4_K and Q5_K share the K layout of a chunk (one 32-byte qs segment: the low and high
// nibbles of groups 2Q and 2Q + 1) and the scale header; Q5_K adds a fifth code bit per
// weight from a 32-byte plane (bit g of byte j: group g, column j), gguf_decode.cpp:77-90.
template <uint32_t TYPE>
constexpr bool kNibbleChunks = TYPE == kQ4K || TYPE == kQ5K;
template <uint32_t TYPE>
constexpr uint32_t kBlockBytes = TYPE == kQ4K ? kQ4KBytes : TYPE == kQ5K ? kQ5KBytes : kQ6KBytes;
typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));

// Vector-memory instructions per wavefront (two MFMA tiles) for one chunk's weights and for
// one block's scale bytes.
template <uint32_t TYPE>
constexpr int kChunkLoads = kNibbleChunks<TYPE> ? 2 : 4;
template <uint32_t TYPE>
constexpr int kBlockLoads = TYPE == kQ4K ? 2 : 4;
// Weight loads issued at the start of chunk Q (chunk Q + 2's bytes; chunk 0 also fetches the
// next block's scale bytes, three chunks before their first use).
// Q6_K chunks 2p and 2p + 1 share their 16 high-bit bytes (qh 32 p .. 32 p + 31 hold the top
// bits of both ql segments of half p): only the even chunk loads them.
template <uint32_t TYPE>
constexpr int weight_loads(int Q) {
    return (TYPE == kQ6K && (Q & 1) ? 2 : kChunkLoads<TYPE>) + (Q == 0 ? kBlockLoads<TYPE> : 0);
}

template <uint32_t TYPE, int Q>
__device__ __forceinline__ void load_w(WRegs &r, const uint8_t *row, int sb, int h) {
    if constexpr (kNibbleChunks<TYPE>) {
        const uint8_t *blk = row + sb * kBlockBytes<TYPE>;
        r.q = *reinterpret_cast<const u32x4 *>(blk + (TYPE == kQ5K ? 48 : 16) + 32 * Q + 16 * h);
        r.h = u32x4{0u, 0u, 0u, 0u};
    } else {
        // Q6_K blocks are 2-byte aligned: 16-byte loads at 2-byte alignment (the hardware's
        // unaligned access mode, which the compiler itself relies on for such loads).
        constexpr int hh = Q >> 1, p = Q & 1;
        const uint8_t *blk = row + sb * kQ6KBytes;
        r.q = *reinterpret_cast<const u32x4a2 *>(blk + 64 * hh + 32 * p + 16 * h);
        if constexpr (p == 0) r.h = *reinterpret_cast<const u32x4a2 *>(blk + 128 + 32 * hh + 16 * h);
    }
}

template <uint32_t TYPE>
__device__ __forceinline__ void load_b(BRegs &r, const uint8_t *row, int sb, int h) {
    if constexpr (TYPE == kQ4K) {
        r.s = *reinterpret_cast<const u32x4 *>(row + sb * kQ4KBytes);
        r.d = 0u;
    } else if constexpr (TYPE == kQ5K) {
        const uint8_t *blk = row + sb * kQ5KBytes;
        r.s = *reinterpret_cast<const u32x4 *>(blk);
        r.qh = *reinterpret_cast<const u32x4 *>(blk + 16 + 16 * h);
        r.d = 0u;
    } else {
        const uint8_t *blk = row + sb * kQ6KBytes;
        r.s = *reinterpret_cast<const u32x4a2 *>(blk + 192);
        r.d = *reinterpret_cast<const uint16_t *>(blk + 208);
    }
}

// An ordering point for the scale bytes: a volatile asm that redefines the registers, so that no
// computation on them is scheduled before it (it stays after the preceding volatile asm).
template <uint32_t TYPE>
__device__ __forceinline__ void pin(BRegs &r) {
    asm volatile("" : "+v"(r.s.x), "+v"(r.s.y), "+v"(r.s.z), "+v"(r.s.w), "+v"(r.d));
    if constexpr (TYPE == kQ5K) asm volatile("" : "+v"(r.qh.x), "+v"(r.qh.y), "+v"(r.qh.z), "+v"(r.qh.w));
}

// Scale (a) and offset (b) of the two sub-blocks a lane meets in chunk Q: w = a*q - b.
// Half 0 (MFMA steps 0, 1) is sub-block 2Q (Q4_K) / Q&1 (Q6_K), half 1 (steps 2, 3) is
// 2Q+1 / (Q&1)+2. The products are exact (see tc_device.h).
struct ChunkScales {
    float a0, b0, a1, b1;
};

template <uint32_t TYPE, int Q>
__device__ __forceinline__ ChunkScales chunk_scales(const BRegs &r, int h) {
    ChunkScales cs;
    if constexpr (kNibbleChunks<TYPE>) {
        const float d = half_to_float(r.s.x), dmin = half_to_float(r.s.x >> 16);
        uint32_t sc, m;
        scale_min_k4(2 * Q, r.s.y, r.s.z, r.s.w, sc, m);
        cs.a0 = d * (float)sc;
        cs.b0 = dmin * (float)m;
        scale_min_k4(2 * Q + 1, r.s.y, r.s.z, r.s.w, sc, m);
        cs.a1 = d * (float)sc;
        cs.b1 = dmin * (float)m;
    } else {
        // sc[8hh + 2p + h] and sc[8hh + 2p + 4 + h]: dwords 2hh and 2hh + 1, byte 2p + h.
        constexpr int hh = Q >> 1, p = Q & 1;
        const float d = half_to_float(r.d);
        const uint32_t sh = 8u * (uint32_t)(2 * p + h);
        cs.a0 = d * (float)(int8_t)(uint8_t)(r.s[2 * hh] >> sh);
        cs.a1 = d * (float)(int8_t)(uint8_t)(r.s[2 * hh + 1] >> sh);
        cs.b0 = 32.f * cs.a0;  // (code - 32) * a = code * a - 32 a, exact
        cs.b1 = 32.f * cs.a1;
    }
    return cs;
}

// Dequantize the 8 weights this lane feeds to MFMA step S (0..3) of chunk Q of a block
// (`blk`: the block's bytes, for the Q5_K high bits; `hb`: the Q6_K high bits, loaded with the
// even chunk of the pair).
template <uint32_t TYPE, int Q, int S>
__device__ __forceinline__ bf16x8 dequant_step(const WRegs &r, const ChunkScales &cs, const BRegs &blk,
                                               const u32x4 &hb) {
    const uint32_t w0 = (S & 1) ? r.q.z : r.q.x, w1 = (S & 1) ? r.q.w : r.q.y;
    const float a = (S >> 1) ? cs.a1 : cs.a0, b = (S >> 1) ? cs.b1 : cs.b0;
    uint32_t c0, c1;
    if constexpr (TYPE == kQ4K) {
        c0 = launder((S >> 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu);
        c1 = launder((S >> 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu);
    } else if constexpr (TYPE == kQ5K) {
        // Group g = 2Q + S/2: bit g of each high byte becomes bit 4 of the code.
        constexpr int g = 2 * Q + (S >> 1);
        const uint32_t h0 = (S & 1) ? blk.qh.z : blk.qh.x, h1 = (S & 1) ? blk.qh.w : blk.qh.y;
        const uint32_t b0 = g <= 4 ? (h0 << (4 - g)) & 0x10101010u : (h0 >> (g - 4)) & 0x10101010u;
        const uint32_t b1 = g <= 4 ? (h1 << (4 - g)) & 0x10101010u : (h1 >> (g - 4)) & 0x10101010u;
        c0 = launder(((S >> 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu) | b0);
        c1 = launder(((S >> 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu) | b1);
    } else {
        constexpr uint32_t g = (Q & 1) + 2 * (S >> 1);
        const uint32_t h0 = (S & 1) ? hb.z : hb.x, h1 = (S & 1) ? hb.w : hb.y;
        c0 = launder(((S >> 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu) | (((h0 >> (2 * g)) & 0x03030303u) << 4));
        c1 = launder(((S >> 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu) | (((h1 >> (2 * g)) & 0x03030303u) << 4));
    }
    const float v0 = __builtin_fmaf(a, (float)(c0 & 0xffu), -b), v1 = __builtin_fmaf(a, (float)((c0 >> 8) & 0xffu), -b);
    const float v2 = __builtin_fmaf(a, (float)((c0 >> 16) & 0xffu), -b), v3 = __builtin_fmaf(a, (float)(c0 >> 24), -b);
    const float v4 = __builtin_fmaf(a, (float)(c1 & 0xffu), -b), v5 = __builtin_fmaf(a, (float)((c1 >> 8) & 0xffu), -b);
    const float v6 = __builtin_fmaf(a, (float)((c1 >> 16) & 0xffu), -b), v7 = __builtin_fmaf(a, (float)(c1 >> 24), -b);
    const u32x4 packed = {pack_bf16x2(v0, v1), pack_bf16x2(v2, v3), pack_bf16x2(v4, v5), pack_bf16x2(v6, v7)};
    return __builtin_bit_cast(bf16x8, packed);
}

// K column of 16-byte activation piece `piece` (0..7) of chunk Q of block sb is
// chunk_base(sb, Q) + piece_column(piece): pieces 0..3 cover the chunk's first 32-wide K run,
// pieces 4..7 the second, which starts 32 (Q4_K) or 64 (Q6_K) columns later.
template <uint32_t TYPE, int Q>
__device__ __forceinline__ int chunk_base(int sb) {
    if constexpr (kNibbleChunks<TYPE>) return 256 * sb + 64 * Q;
    else return 256 * sb + 128 * (Q >> 1) + 32 * (Q & 1);
}
template <uint32_t TYPE>
__device__ __forceinline__ int piece_column(int piece) {
    constexpr int second = kNibbleChunks<TYPE> ? 32 : 64;
    return piece < 4 ? 8 * piece : second + 8 * (piece - 4);
}

// Activation chunk tiles live in four LDS buffers: chunk Q of every super-block uses
// buffer Q, so each buffer index is a compile-time constant. A tile is 32 MT rows x 128 bytes
// (64 bf16), row r at r * 128; its eight 16-byte pieces are stored XOR-swizzled
// (slot = piece ^ swz(r)) so that the 16-byte fragment reads of 8 or 16 consecutive lanes
// (consecutive rows, same piece) hit distinct banks.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

typedef __attribute__((address_space(3))) void lds_void;

// One unit of work: output tile (m0, n0) over super-blocks [sb_begin, sb_end) of K. In a
// grouped launch (GroupItem) `second` marks the second problem's tiles, and `tile` counts the
// tiles of both. (An int: a bool would leave padding bytes that the copies keep in memory.)
struct Item {
    int m0, n0, tile, slice, sb_begin, sb_end;
};
struct GroupItem : Item {
    int second;
};
template <bool GROUP>
using ItemT = std::conditional_t<GROUP, GroupItem, Item>;
template <bool GROUP>
__device__ __forceinline__ bool is_second(const ItemT<GROUP> &it) {
    if constexpr (GROUP) return it.second != 0;
    else return false;
}

// Work item `it` = slice * tiles + r. The tile-order index r is remapped so that each XCD
// (own L2; workgroup b runs on XCD b % 8, and a persistent workgroup's items keep that
// residue) receives a contiguous run of tiles, which it walks in bands of 4 M-tiles so
// that concurrently resident workgroups share weight and activation tiles. In a grouped
// launch (GROUP) the second problem's tiles_m1 x tiles_n1 tiles follow the first problem's.
template <int MT, bool GROUP>
__device__ __forceinline__ ItemT<GROUP> item_at(int it, int tiles_m, int tiles_n, int splits, int nsb_all,
                                                int tiles_m1, int tiles_n1) {
    const int t0 = tiles_m * tiles_n, total = GROUP ? t0 + tiles_m1 * tiles_n1 : t0;
    const int slice = it / total;
    int r = it - slice * total;
    if ((total & 7) == 0) r = (r & 7) * (total >> 3) + (r >> 3);
    const bool second = GROUP && r >= t0;
    if (second) {
        r -= t0;
        tiles_m = tiles_m1;
        tiles_n = tiles_n1;
    }
    constexpr int kBand = 4;
    const int band = r / (kBand * tiles_n), first_m = band * kBand;
    const int band_m = min(tiles_m - first_m, kBand);
    const int in_band = r - band * kBand * tiles_n;
    const int tm = first_m + in_band % band_m, tn = in_band / band_m;
    ItemT<GROUP> g;
    g.m0 = tm * 32 * MT;
    g.n0 = tn * kBN;
    g.tile = (second ? t0 : 0) + tm * tiles_n + tn;
    g.slice = slice;
    if constexpr (GROUP) g.second = second ? 1 : 0;
    g.sb_begin = (int)((int64_t)slice * nsb_all / splits);
    g.sb_end = (int)((int64_t)(slice + 1) * nsb_all / splits);
    return g;
}

// Per-wavefront epilogue staging (16 rows x 64 fp32 columns, 272-byte row pitch: rows 4
// apart fall in different banks), separate from the activation buffers, which already hold
// the next item's first chunks while an item's outputs are written.
constexpr int kStagePitch = 272;
__shared__ __attribute__((aligned(16))) uint8_t g_stage[4 * 16 * kStagePitch];

// Waits until at most VM of this wavefront's vector-memory operations are outstanding, then
// joins the workgroup barrier.
template <int VM>
__device__ __forceinline__ void wait_vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(VM) : "memory");
}

// Block kinds of the K stream: MID; LAST (chunks c + 2 and c + 4 come from where the
// stream continues); AFTER_FULL: the first block after the epilogue of a full tile, whose
// 4 MT output stores per wavefront sit in the queue between the DMA of this block's chunks
// and later loads, so that its first three barriers can wait for the DMA alone and leave
// the stores in flight.
enum BlockKind { kMid, kLast, kAfterFull };

// Persistent workgroups: workgroup b processes items b, b + G, b + 2G, ... (G = grid size,
// at most one workgroup per CU). The K loop runs as one stream over all of a workgroup's
// items: during an item's last super-block the weight loads and activation DMA already
// fetch the next item's first chunks, so the pipeline never drains between output tiles and
// the epilogue overlaps those loads. SPLIT items write raw fp32 accumulators to `partials`
// (see k_splitk_reduce) instead of bf16 outputs. GROUP: the work list also holds the output
// tiles of a second problem `g2` (same type, K, activation row stride and MT); each item
// reads its own problem's activation, weight and output.
// The second problem arrives as the one element of `second` (empty without GROUP, so that the
// one-problem kernels keep their argument list).
template <uint32_t TYPE, bool SPLIT, int MT, int ACT, bool GROUP, typename... Second>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, MT >= 4 ? 1 : 2)))
void k_gemm(const uint16_t *__restrict__ x, int64_t x_stride, int M, const uint8_t *__restrict__ w,
            int64_t w_pitch, int N, int K, uint16_t *__restrict__ y, int64_t y_stride,
            const uint16_t *__restrict__ bias, int tiles_m, int tiles_n, int splits, float *__restrict__ partials,
            Second... second) {
    static_assert(sizeof...(Second) == (GROUP ? 1 : 0), "a grouped launch takes one second problem");
    GemmSecond g2{};
    if constexpr (GROUP) g2 = GemmSecond(second...);
    static_assert(!SPLIT || ACT == kActNone, "split variants leave the activation to the slice reduction");
    static_assert(ACT != kActNoneKeep || MT >= 4, "cached-output variants: 128- and 256-row tiles only");
    static_assert(!GROUP || ACT == kActNone, "grouped variants take no output activation");
    // The problem an item belongs to (always the first without GROUP).
    using It = ItemT<GROUP>;
    auto pick = [&](const It &it, auto first, auto other) { return is_second<GROUP>(it) ? other : first; };
    // Four separate LDS objects (not one array): the compiler's tracking of the DMA's LDS
    // writes then tells the buffers apart, and a fragment read waits only for the DMA of its
    // own buffer instead of for every DMA in flight.
    __shared__ __attribute__((aligned(16))) uint8_t xbuf0[32 * MT * 128];
    __shared__ __attribute__((aligned(16))) uint8_t xbuf1[32 * MT * 128];
    __shared__ __attribute__((aligned(16))) uint8_t xbuf2[32 * MT * 128];
    __shared__ __attribute__((aligned(16))) uint8_t xbuf3[32 * MT * 128];
    auto xbuf = [&](auto btag) -> uint8_t * {
        constexpr int B = decltype(btag)::value;
        if constexpr (B == 0) return xbuf0;
        else if constexpr (B == 1) return xbuf1;
        else if constexpr (B == 2) return xbuf2;
        else return xbuf3;
    };
    const int nsb_all = K / 256;
    const int ntiles = tiles_m * tiles_n + (GROUP ? g2.tiles_m * g2.tiles_n : 0);
    const int items = ntiles * splits, grid = (int)gridDim.x;
    int item = (int)blockIdx.x;
    It cur = item_at<MT, GROUP>(item, tiles_m, tiles_n, splits, nsb_all, g2.tiles_m, g2.tiles_n);

    const int tid = (int)threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    // Uniform wave index: the per-wave LDS destinations of the DMA then stay scalar (M0 is
    // set from SGPRs, with no v_readfirstlane per load).
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wcol0 = 64 * wave + l32, wcol1 = wcol0 + 32;
    auto wrow = [&](const It &it, int col) {
        return pick(it, w, g2.w) + (int64_t)min(it.n0 + col, pick(it, N, g2.N) - 1) * w_pitch;
    };
    const uint8_t *wrow0 = wrow(cur, wcol0), *wrow1 = wrow(cur, wcol1);

    // Direct global->LDS staging (buffer loads with the lds bit): instruction i (0..MT-1) of
    // wavefront w writes tile rows 8 (MT w + i) + lane/8 (1 KB, lane-linear); the lane carries
    // LDS slot lane%8, i.e. logical piece (lane%8) ^ swz(row) with
    // swz(row) = (lane/8) ^ ((MT w + i) & 1).
    // The buffer descriptor starts at the tile's first row and ends at row M, and the
    // per-lane byte offset (row within the tile, piece) is fixed for the whole kernel: rows
    // >= M are out of range and read as zero. The chunk's column base goes in soffset. The
    // range is a 32-bit byte count: a span from the tile's first row to row M of 4 GiB or more
    // is clamped to 2^32 - 1, which still covers every row of the tile (the host requires
    // 2 (255 x_stride + K) < 2^31, so such a span holds far more than the tile's 256 rows).
    const int dma_row = 8 * MT * wave + (lane >> 3);
    const int piece_even = (lane & 7) ^ (lane >> 3), piece_odd = piece_even ^ 1;
    auto x_rsrc = [&](const It &it) {
        const int64_t span = (int64_t)(pick(it, M, g2.M) - it.m0) * x_stride * 2;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(pick(it, x, g2.x) + (int64_t)it.m0 * x_stride),
                                                 (short)0, (int)(uint32_t)std::min<int64_t>(span, 0xffffffffll),
                                                 0x00020000);
    };
    __amdgpu_buffer_rsrc_t xrsrc = x_rsrc(cur);
    int voff[8];  // first MT used (a template-sized array captured by the lambdas below makes
                  // the host-side instantiation of the kernel invalid, dropping its launch stub)
#pragma unroll
    for (int i = 0; i < MT; ++i)
        voff[i] = (int)(((int64_t)(dma_row + 8 * i) * x_stride +
                         piece_column<TYPE>(((MT * wave + i) & 1) ? piece_odd : piece_even)) * 2);
    auto dma = [&](auto btag, __amdgpu_buffer_rsrc_t rs, int sbd) {
        constexpr int B = decltype(btag)::value;  // buffer = chunk index within the block
        const int soff = 2 * chunk_base<TYPE, B>(sbd);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(xbuf(btag) + (8 * (MT * wave + i)) * 128), 16,
                                                     voff[i], soff, 0, 0);
        asm volatile("" ::: "memory");  // keep each chunk's DMA batch in issue order
    };

    f32x16 acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        acc[i][0] = f32x16{};
        acc[i][1] = f32x16{};
    }

    // Raw weights of chunks c .. c + 2 in flight: chunk Q of a block lives in wset[Q] (two
    // 32-column MFMA tiles each), loaded two chunks before its use.
    WRegs wset[4][2];
    // Scale bytes of the current block and of the next one (loaded with chunk 2's weights).
    BRegs bcur[2], bnxt[2];
    // Fragment read offsets: lane (l32, h) reads row 32 i + l32, logical piece
    // 4 (S >> 1) + 2 h + (S & 1) for MFMA step S.
    const int frag_row = l32 * 128;
    const int frag_swz = swz(l32);
    bf16x8 a_even[MT], a_odd[MT], b_even[2], b_odd[2];
    ChunkScales cs0, cs1;
    auto prepare = [&](auto qtag, auto stag, bf16x8(&a)[MT], bf16x8(&b)[2]) {
        constexpr int Q = decltype(qtag)::value, S = decltype(stag)::value;
        constexpr int pc = 4 * (S >> 1) + (S & 1);
        const uint8_t *xb = xbuf(qtag) + frag_row + 16 * ((pc + 2 * h) ^ frag_swz);
#pragma unroll
        for (int i = 0; i < MT; ++i) a[i] = *reinterpret_cast<const bf16x8 *>(xb + 32 * i * 128);
        b[0] = dequant_step<TYPE, Q, S>(wset[Q][0], cs0, bcur[0], wset[Q & 2][0].h);
        b[1] = dequant_step<TYPE, Q, S>(wset[Q][1], cs1, bcur[1], wset[Q & 2][1].h);
    };
    auto mfmas = [&](const bf16x8(&a)[MT], const bf16x8(&b)[2]) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[0], acc[i][0], 0, 0, 0);
            acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[1], acc[i][1], 0, 0, 0);
        }
    };
    // Interleave: each MFMA (8 passes) covers an LDS read and a few VALU ops. With fewer
    // row blocks (MT < 8) the step has 2 MT MFMAs and the dequant VALU spreads over them.
    // MT = 8: the next step's 8 fragment reads go out with the step's first 8 MFMAs, a full
    // step before their use, with 4 VALU each, then 3 VALU per MFMA (reads left to the
    // compiler's schedule came in the last quarter of the step; this order measured 0.3-1.7 %
    // faster at the north star, 8 reads at once 3 % slower).
    auto interleave = [&]() {
        if constexpr (MT == 8 && TYPE == kQ6K) {
            // Q6_K spends about 4.6 VALU per MFMA (3.5 for Q4_K): 5 with each read, then 4
            // (config 4 block and config 3 at 4096 tokens about 1 % faster than 4 / 3).
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
        } else if constexpr (MT == 8) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
        } else if constexpr (MT == 4) {
            // The same shape for 128-row tiles: 4 reads with 8 VALU each, then 6 (config 1
            // 0.3-2 % faster than 7 per MFMA throughout; 9 / 5 and 10 / 4 slower).
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            }
#pragma unroll
            for (int k = 4; k < 8; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 2 * MT; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (k < MT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 56 / (2 * MT), 0);
            }
        }
    };

    // Prologue (first item only): weights of chunks 0 and 1, the four chunks of the first
    // block into buffers 0..3, then wait for this wave's chunk-0 DMA (the 24 loads of chunks
    // 1..3 may stay in flight) and every other wave's, and prepare step 0.
    load_b<TYPE>(bcur[0], wrow0, cur.sb_begin, h);
    load_b<TYPE>(bcur[1], wrow1, cur.sb_begin, h);
    load_w<TYPE, 0>(wset[0][0], wrow0, cur.sb_begin, h);
    load_w<TYPE, 0>(wset[0][1], wrow1, cur.sb_begin, h);
    load_w<TYPE, 1>(wset[1][0], wrow0, cur.sb_begin, h);
    load_w<TYPE, 1>(wset[1][1], wrow1, cur.sb_begin, h);
    dma(std::integral_constant<int, 0>{}, xrsrc, cur.sb_begin);
    dma(std::integral_constant<int, 1>{}, xrsrc, cur.sb_begin);
    dma(std::integral_constant<int, 2>{}, xrsrc, cur.sb_begin);
    dma(std::integral_constant<int, 3>{}, xrsrc, cur.sb_begin);
    wait_vm_barrier<3 * MT>();  // the DMA of chunks 1..3 may stay in flight
    cs0 = chunk_scales<TYPE, 0>(bcur[0], h);
    cs1 = chunk_scales<TYPE, 0>(bcur[1], h);
    prepare(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, a_even, b_even);

    // The previous item was a full tile (so its epilogue issued exactly 4 MT vector stores per
    // wavefront) and the next block may use the AFTER_FULL waits. Never for SPLIT items,
    // whose epilogue stores are more numerous.
    bool after_full = false;
    const bool y_vec0 = (y_stride % 8) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    const bool y_vec1 = GROUP && (g2.y_stride % 8) == 0 && (reinterpret_cast<uintptr_t>(g2.y) & 15u) == 0;
    for (;;) {
        // Where the stream continues after this item's last block: the next item's first
        // block, or (no next item) this item's last block again, loaded redundantly so that
        // every chunk issues the same loads (the hand-written vmcnt waits count on it).
        const int next_item = item + grid;
        const bool has_next = next_item < items;
        const It nxt =
            has_next ? item_at<MT, GROUP>(next_item, tiles_m, tiles_n, splits, nsb_all, g2.tiles_m, g2.tiles_n) : cur;
        const int sb_next = has_next ? nxt.sb_begin : cur.sb_end - 1;
        const uint8_t *wnext0 = has_next ? wrow(nxt, wcol0) : wrow0;
        const uint8_t *wnext1 = has_next ? wrow(nxt, wcol1) : wrow1;
        const __amdgpu_buffer_rsrc_t xrsrc_next = has_next ? x_rsrc(nxt) : xrsrc;

        // Chunk Q of block sb (activations in buffer Q). Operands of each MFMA step are
        // prepared during the previous step; step 0 of the next chunk during step 3. The
        // barrier sits between steps 2 and 3: before it, this wave waits for its DMA of the
        // next chunk (16 later DMA loads may remain in flight); after it, every wave is done
        // reading buffer Q (its last reads feed step 3 and were issued during step 2), so
        // the DMA of chunk c + 4 goes into buffer Q. LAST: sb is the item's last block, so
        // chunks c + 2 (Q >= 2) and c + 4 come from where the stream continues.
        auto chunk = [&](auto qtag, auto kindtag, int sb) {
            constexpr int Q = decltype(qtag)::value;
            constexpr int KIND = decltype(kindtag)::value;
            constexpr bool LAST = KIND == kLast;
            // Operations issued after the DMA this barrier waits for (chunk c + 1): normally
            // at least 2 MT (two later DMA batches); after a full tile's epilogue, for Q < 3,
            // also the 4 MT stores and three chunks' weight loads.
            constexpr int VM = (KIND == kAfterFull && Q < 3)
                                   ? std::min(63, weight_loads<TYPE>((Q + 2) & 3) + weight_loads<TYPE>((Q + 3) & 3) +
                                                      weight_loads<TYPE>(Q) + 6 * MT)
                                   : 2 * MT;
            constexpr int QN = (Q + 1) & 3;
            constexpr int Q2 = (Q + 2) & 3;
            if constexpr (Q < 2) {
                load_w<TYPE, Q2>(wset[Q2][0], wrow0, sb, h);
                load_w<TYPE, Q2>(wset[Q2][1], wrow1, sb, h);
            } else if constexpr (!LAST) {
                load_w<TYPE, Q2>(wset[Q2][0], wrow0, sb + 1, h);
                load_w<TYPE, Q2>(wset[Q2][1], wrow1, sb + 1, h);
            } else {
                load_w<TYPE, Q2>(wset[Q2][0], wnext0, sb_next, h);
                load_w<TYPE, Q2>(wset[Q2][1], wnext1, sb_next, h);
            }
            // The scale bytes of the block after this one (of the next item's first block when
            // this is the item's last), needed from the end of chunk 3.
            if constexpr (Q == 0 && !LAST) {
                load_b<TYPE>(bnxt[0], wrow0, sb + 1, h);
                load_b<TYPE>(bnxt[1], wrow1, sb + 1, h);
            } else if constexpr (Q == 0) {
                load_b<TYPE>(bnxt[0], wnext0, sb_next, h);
                load_b<TYPE>(bnxt[1], wnext1, sb_next, h);
            }
            asm volatile("" ::: "memory");  // issue the weight loads here, a full chunk ahead
            prepare(qtag, std::integral_constant<int, 1>{}, a_odd, b_odd);
            mfmas(a_even, b_even);
            interleave();
            prepare(qtag, std::integral_constant<int, 2>{}, a_even, b_even);
            mfmas(a_odd, b_odd);
            interleave();
            prepare(qtag, std::integral_constant<int, 3>{}, a_odd, b_odd);
            mfmas(a_even, b_even);
            interleave();
            wait_vm_barrier<VM>();
            if constexpr (!LAST) dma(qtag, xrsrc, sb + 1);
            else dma(qtag, xrsrc_next, sb_next);
            if constexpr (QN == 0) {
                // Keep the next block's scale decode here, after the barrier: hoisted up to its
                // load, it would make the wave wait for a load issued moments earlier.
                pin<TYPE>(bnxt[0]);
                pin<TYPE>(bnxt[1]);
                cs0 = chunk_scales<TYPE, 0>(bnxt[0], h);
                cs1 = chunk_scales<TYPE, 0>(bnxt[1], h);
                bcur[0] = bnxt[0];
                bcur[1] = bnxt[1];
            } else {
                cs0 = chunk_scales<TYPE, QN>(bcur[0], h);
                cs1 = chunk_scales<TYPE, QN>(bcur[1], h);
            }
            prepare(std::integral_constant<int, QN>{}, std::integral_constant<int, 0>{}, a_even, b_even);
            mfmas(a_odd, b_odd);
            interleave();
        };
        auto block = [&](auto kindtag, int sb) {
            chunk(std::integral_constant<int, 0>{}, kindtag, sb);
            chunk(std::integral_constant<int, 1>{}, kindtag, sb);
            chunk(std::integral_constant<int, 2>{}, kindtag, sb);
            chunk(std::integral_constant<int, 3>{}, kindtag, sb);
        };
        int sb = cur.sb_begin;
        if (after_full && sb < cur.sb_end - 1) block(std::integral_constant<int, kAfterFull>{}, sb++);
        for (; sb < cur.sb_end - 1; ++sb) block(std::integral_constant<int, kMid>{}, sb);
        block(std::integral_constant<int, kLast>{}, cur.sb_end - 1);

        // The lane geometry of the epilogue is recomputed here (the asm hides the thread id
        // from CSE), so no value lives across the K loop only for the epilogue.
        int tid_e = (int)threadIdx.x;
        asm volatile("" : "+v"(tid_e));
        const int lane_e = tid_e & 63, l32e = lane_e & 31, he = lane_e >> 5;
        // This item's problem.
        const int cM = pick(cur, M, g2.M), cN = pick(cur, N, g2.N);
        uint16_t *const cy = pick(cur, y, g2.y);
        const int64_t cys = pick(cur, y_stride, g2.y_stride);
        const uint16_t *const cbias = pick(cur, bias, g2.bias);
        const bool y_vec = pick(cur, y_vec0, y_vec1);
        if constexpr (SPLIT) {
            // Raw accumulators, MFMA-native order: value v = 16 (2 i + t) + j of lane `lane` of
            // wavefront w of tile `tile`, slice s, at
            // ((((s * tiles + tile) * 4 + w) * 32 MT + v) * 64 + lane); row blocks i past M are
            // skipped (never read back).
            float *dst = partials + ((((int64_t)cur.slice * ntiles + cur.tile) * 4 + wave) * (32 * MT)) * 64 + lane_e;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                if (cur.m0 + 32 * i >= cM) break;
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int j = 0; j < 16; ++j) dst[(16 * (2 * i + t) + j) * 64] = acc[i][t][j];
            }
        } else {
            // One 16-row half of a 32-row block i at a time. Lane (l32, h) of MFMA tile (i, t)
            // holds column 64w + 32t + l32 and rows 32i + 8(j/4) + 4h + (j%4) of accumulator
            // j, so half f holds j in [8f, 8f + 8). The raw fp32 accumulators go to this
            // wavefront's staging rows first (straight from the accumulator registers: reading
            // them into VGPRs for the conversion would make the register allocator copy and
            // spill them); each lane then reads 8 consecutive columns of a row, rounds to bf16
            // (then adds the bias and rounds again) and writes 16 bytes.
            uint8_t *stage = g_stage + wave * (16 * kStagePitch);
            const int ncol0 = cur.n0 + 64 * wave;
            const bool full_n = ncol0 + 64 <= cN;
            const int rd_row = lane_e >> 3, rd_col = 8 * (lane_e & 7);  // 8 rows x 8 column groups per pass
            float bv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[e] = 0.f;
            if (cbias) {
#pragma unroll
                for (int e = 0; e < 8; ++e) bv[e] = bf16_to_float(cbias[min(ncol0 + rd_col + e, cN - 1)]);
            }
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                if (cur.m0 + 32 * i >= cM) break;
#pragma unroll
                for (int f = 0; f < 2; ++f) {
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int jj = 0; jj < 8; ++jj) {
                            const int j = 8 * f + jj;
                            const int row = 8 * (jj >> 2) + 4 * he + (jj & 3), col = 32 * t + l32e;
                            *reinterpret_cast<float *>(stage + row * kStagePitch + 4 * col) = acc[i][t][j];
                        }
                    // Same-wave LDS traffic: the compiler orders the reads after the writes
                    // (lgkmcnt), and the next half's writes after these reads.
#pragma unroll
                    for (int pass = 0; pass < 2; ++pass) {
                        const int row = 8 * pass + rd_row, m = cur.m0 + 32 * i + 16 * f + row;
                        const f32x4 v0 = *reinterpret_cast<const f32x4 *>(stage + row * kStagePitch + 4 * rd_col);
                        const f32x4 v1 = *reinterpret_cast<const f32x4 *>(stage + row * kStagePitch + 4 * rd_col + 16);
                        const float fv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                        // RNE pairs with v_cvt_pk_bf16_f32; the bias is added to the widened bf16
                        // values and rounded again (the same two roundings as the scalar formula).
                        uint32_t o[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            o[q] = pack_bf16x2(fv[2 * q], fv[2 * q + 1]);
                            if (cbias)
                                o[q] = pack_bf16x2(__builtin_bit_cast(float, o[q] << 16) + bv[2 * q],
                                                   __builtin_bit_cast(float, o[q] & 0xffff0000u) + bv[2 * q + 1]);
                        }
                        // Output activation: one store instruction per pass either way (a full
                        // tile's epilogue issues exactly 4 MT stores per wavefront, which the
                        // AFTER_FULL waits count on). The full-width stores are non-temporal (the
                        // output is not read again by this launch, and its lines would otherwise
                        // displace activation and weight lines that the band's other tiles reuse
                        // from L2), except under kActNoneKeep, whose caller reads y back at once.
                        if constexpr (ACT == kActSiluGlu) {
                            // Columns 2c, 2c + 1 are (gate_c, up_c): 4 outputs at column c.
                            uint32_t hv[4];
#pragma unroll
                            for (int q = 0; q < 4; ++q) hv[q] = silu_glu_bits(o[q] & 0xffffu, o[q] >> 16);
                            if (m < cM) {
                                uint16_t *dst = cy + (int64_t)m * cys + ((ncol0 + rd_col) >> 1);
                                if (full_n && y_vec) {
                                    __builtin_nontemporal_store(u32x2{hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16)},
                                                                reinterpret_cast<u32x2 *>(dst));
                                } else {
#pragma unroll
                                    for (int q = 0; q < 4; ++q)
                                        if (ncol0 + rd_col + 2 * q < cN) dst[q] = (uint16_t)hv[q];
                                }
                            }
                        } else {
                            if constexpr (ACT == kActGeluTanh) {
#pragma unroll
                                for (int q = 0; q < 4; ++q)
                                    o[q] = gelu_tanh_bits(o[q] & 0xffffu) | (gelu_tanh_bits(o[q] >> 16) << 16);
                            }
                            if (m < cM) {
                                uint16_t *dst = cy + (int64_t)m * cys + ncol0 + rd_col;
                                if (full_n && y_vec) {
                                    if constexpr (ACT == kActNoneKeep)
                                        *reinterpret_cast<u32x4 *>(dst) = u32x4{o[0], o[1], o[2], o[3]};
                                    else
                                        __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]},
                                                                    reinterpret_cast<u32x4 *>(dst));
                                } else {
#pragma unroll
                                    for (int e = 0; e < 8; ++e)
                                        if (ncol0 + rd_col + e < cN) dst[e] = (uint16_t)(o[e >> 1] >> (16 * (e & 1)));
                                }
                            }
                        }
                    }
                }
            }
        }
        if (!has_next) break;
        after_full = !SPLIT && y_vec && cur.m0 + 32 * MT <= cM && cur.n0 + kBN <= cN;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            acc[i][0] = f32x16{};
            acc[i][1] = f32x16{};
        }
        item = next_item;
        cur = nxt;
        wrow0 = wnext0;
        wrow1 = wnext1;
        xrsrc = xrsrc_next;
    }
    // Every DMA this wave issued (including the redundant ones past its last item) must land
    // before the workgroup's LDS is released.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Launches k_gemm<TYPE, SPLIT, MT, ACT, GROUP> over a.grid persistent workgroups (GROUP: with
// the second problem b).
template <uint32_t TYPE, bool SPLIT, int MT, int ACT, bool GROUP = false>
hipError_t gemm_variant(const GemmArgs &a, hipStream_t stream, const GemmSecond &b = GemmSecond{}) {
    if constexpr (GROUP)
        hipLaunchKernelGGL((k_gemm<TYPE, SPLIT, MT, ACT, true, GemmSecond>), dim3((unsigned)a.grid), dim3(kThreads), 0,
                           stream, a.x,
                           a.x_stride, a.M, a.w, a.w_pitch, a.N, a.K, a.y, a.y_stride, a.bias, a.tiles_m, a.tiles_n,
                           a.splits, a.partials, b);
    else
        hipLaunchKernelGGL((k_gemm<TYPE, SPLIT, MT, ACT, false>), dim3((unsigned)a.grid), dim3(kThreads), 0, stream, a.x,
                           a.x_stride, a.M, a.w, a.w_pitch, a.N, a.K, a.y, a.y_stride, a.bias, a.tiles_m, a.tiles_n,
                           a.splits, a.partials);
    return hipGetLastError();
}

}  // namespace
}  // namespace tc
