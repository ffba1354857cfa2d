// Quantized GEMV for one activation row (adaLN modulation, single-token text encoding):
// y[n] = sum_k x[k] w[n][k] with w the exact fp32 dequantized weight, bf16 output (+ bias
// after the cast). HBM-bound: every weight byte is read once.
//
// Replaces the M = 1 side of mx::quantized_matmul (MLX qmv, native/backends/mlx.cpp:678)
// and the CPU-decode-then-GEMM pager route (gguf_weight_pager.cpp:347-349,571-573).
//
// Scheme: the dot products run on the matrix cores (v_mfma_f32_16x16x32_bf16) with a
// block-diagonal activation operand. One "set" is a K range whose 16 scale groups (Q4_K: 16
// sub-blocks of 32 = two super-blocks; Q6_K: 16 groups of 16 = one super-block) become the
// 16 rows of A; the 16 columns of B are 16 weight rows. In each MFMA, lane group h (lanes
// 16h..16h+15) supplies 8 consecutive weights of one group for each of the 16 weight rows,
// and A carries the matching 8 activations only in the A row of that group (zeros
// elsewhere). After the set's MFMAs, D[g][n] = sum over group g of x * (128 + code): a dense
// 16 x 16 tile of per-(row, group) dot products, and lane (h, n) holds groups 4h..4h+3 of row
// n, whose scales it decodes from the header it loaded itself.
//
// Codes enter B as the bf16 numbers 128 + code (exact for codes < 128, built with one
// byte permute per pair), so sum x * code = D - 128 X with X = sum of x over the group.
// X comes from the same A operands times a B of ones (two MFMAs per set).
//   Q4_K: w = d sc q - dmin m       -> y += d (sum_g sc_g (D_g - 128 X_g)) - dmin sum_g m_g X_g
//   Q6_K: w = d sc (code - 32)      -> y += d sum_g sc_g (D_g - 160 X_g)
// No weight is rounded: the result is the fp32-dequant GEMV up to fp32 summation order.
//
// Memory access. Q4_K: each lane loads its own MFMA pieces of its row straight into
// registers (qs chunks h and 4 + h of both blocks, and the header of block h >> 1), so one
// load instruction reads 16 rows x a 64-byte run; measured on MI355X this streams as fast as
// row-major 1 KB runs and saves the LDS round trip. Q6_K (scales and high bits in separate
// small fields) loads its 16 rows x one set row-major, with consecutive lanes on consecutive
// 16-byte chunks of a row, stages them in a wavefront-private LDS tile and reads its MFMA
// pieces from there. The zero-padded A operands come from a per-wavefront LDS area: lanes
// that own an activation slice store it there, and every MFMA reads either the lane's own
// slot or a zero slot. Work split: a workgroup owns one 16-row tile; its wavefronts
// interleave over the K sets with two sets in flight each, and their partial sums are added
// through LDS in a fixed order.
#include <algorithm>
#include <utility>

#include "tc_device.h"
#include "tc_kernels.h"

namespace tc {
namespace {

typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32a2 __attribute__((aligned(2)));

template <uint32_t TYPE>
struct Geo;
// kChunks: 16-byte chunks per row and set (Q6_K: 13 chunks + the 2-byte d); kRowLds: bytes
// per row in the LDS tile (padded so that the 16 rows fall on distinct LDS banks);
// kLoads: chunk loads per lane and set.
template <>
struct Geo<kQ4K> {
    static constexpr int kBlocksPerSet = 2, kMfma = 16, kSetK = 512, kSlots = 64;
    static constexpr int kSetBytes = 2 * kQ4KBytes, kChunks = 18, kRowLds = 304, kLoads = 5;
    static constexpr bool kStaged = false;  // loads land in the lanes that use them
};
template <>
struct Geo<kQ5K> {
    // As Q4_K, plus the 16 high-bit bytes of each of the set's two blocks per lane.
    static constexpr int kBlocksPerSet = 2, kMfma = 16, kSetK = 512, kSlots = 64;
    static constexpr int kSetBytes = 2 * kQ5KBytes, kChunks = 22, kRowLds = 352, kLoads = 7;
    static constexpr bool kStaged = false;
};
template <>
struct Geo<kQ6K> {
    static constexpr int kBlocksPerSet = 1, kMfma = 8, kSetK = 256, kSlots = 32;
    static constexpr int kSetBytes = kQ6KBytes, kChunks = 14, kRowLds = 240, kLoads = 4;
    static constexpr bool kStaged = true;  // row-major loads through an LDS tile
};

// Dynamic LDS per wavefront: the staged rows (Q6_K), then the A-operand slots.
template <uint32_t TYPE>
constexpr int wave_lds_bytes() {
    return (Geo<TYPE>::kStaged ? 16 * Geo<TYPE>::kRowLds : 0) + 16 * (Geo<TYPE>::kSlots + 4);
}

constexpr uint32_t kOOR = 0x80000000u;  // buffer offset beyond any range: the load returns 0

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// (t.b0, t.b1) and (t.b2, t.b3) as bf16 pairs 0x4300 | byte = 128 + byte.
__device__ __forceinline__ uint32_t pair01(uint32_t t) { return __builtin_amdgcn_perm(0x43434343u, t, 0x04010400u); }
__device__ __forceinline__ uint32_t pair23(uint32_t t) { return __builtin_amdgcn_perm(0x43434343u, t, 0x04030402u); }
__device__ __forceinline__ u32x4 codes8(uint32_t ta, uint32_t tb) {
    return u32x4{pair01(ta), pair23(ta), pair01(tb), pair23(tb)};
}
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) { return (a & mask) | (b & ~mask); }

// Weight bytes one lane holds for one (tile, set).
template <uint32_t TYPE>
struct WT;
template <>
struct WT<kQ4K> {
    u32x4 q[4];  // qs pieces 4k4 + h of the set's two blocks (piece p: block p >> 3, bytes 16 + 16 (p & 7))
    u32x4 hd;    // header of block h >> 1 of the set
};
template <>
struct WT<kQ5K> {
    u32x4 q[4];   // qs pieces as Q4_K (piece p: block p >> 3, bytes 48 + 16 (p & 7))
    u32x4 hd;     // header of block h >> 1 of the set
    u32x4 qh[2];  // high-bit bytes 16 (h & 1) .. + 15 of blocks 0 and 1, shifted right by 2 (h >> 1)
};
template <>
struct WT<kQ6K> {
    u32x4 l[2];   // ql bytes 64k + 16h
    u32x4 qh[2];  // qh bytes 128 + 32k + 16 (h & 1)
    uint32_t sc;  // scales 4h .. 4h + 3
    uint32_t d;   // d (fp16 bits)
};

// This lane's MFMA pieces of row c, read from the wavefront's LDS tile.
template <uint32_t TYPE>
__device__ __forceinline__ void read_wt(WT<TYPE> &r, const uint8_t *tile, int c, int h) {
    const uint8_t *row = tile + c * Geo<TYPE>::kRowLds;
    if constexpr (TYPE == kQ4K) {
        r.q[0] = *reinterpret_cast<const u32x4 *>(row + 16 + 16 * h);
        r.q[1] = *reinterpret_cast<const u32x4 *>(row + 80 + 16 * h);
        r.q[2] = *reinterpret_cast<const u32x4 *>(row + 160 + 16 * h);
        r.q[3] = *reinterpret_cast<const u32x4 *>(row + 224 + 16 * h);
        r.hd = *reinterpret_cast<const u32x4 *>(row + 144 * (h >> 1));
    } else {
        r.l[0] = *reinterpret_cast<const u32x4 *>(row + 16 * h);
        r.l[1] = *reinterpret_cast<const u32x4 *>(row + 64 + 16 * h);
        r.qh[0] = *reinterpret_cast<const u32x4 *>(row + 128 + 16 * (h & 1));
        r.qh[1] = *reinterpret_cast<const u32x4 *>(row + 160 + 16 * (h & 1));
        r.sc = *reinterpret_cast<const uint32_t *>(row + 192 + 4 * h);
        r.d = *reinterpret_cast<const uint32_t *>(row + 208);
    }
}

// B operand of MFMA t: piece k = t >> 2, dword pair e = (t >> 1) & 1, nibble v = t & 1.
template <uint32_t TYPE, int T>
__device__ __forceinline__ u32x4 codes(const WT<TYPE> &r, uint32_t hmask, uint32_t sl, uint32_t sh) {
    constexpr int k = T >> 2, e = (T >> 1) & 1, v = T & 1;
    if constexpr (TYPE == kQ4K) {
        const uint32_t a = r.q[k][2 * e], b = r.q[k][2 * e + 1];
        if constexpr (v == 0) return codes8(a & 0x0f0f0f0fu, b & 0x0f0f0f0fu);
        else return codes8((a >> 4) & 0x0f0f0f0fu, (b >> 4) & 0x0f0f0f0fu);
    } else if constexpr (TYPE == kQ5K) {
        // Group 2 j + v of block k >> 1, j = 2 (k & 1) + (h >> 1): its fifth bit is bit
        // 4 (k & 1) + v of the high bytes already shifted right by 2 (h >> 1).
        constexpr int g0 = 4 * (k & 1) + v;
        const uint32_t a = r.q[k][2 * e], b = r.q[k][2 * e + 1];
        const uint32_t ha = r.qh[k >> 1][2 * e], hb = r.qh[k >> 1][2 * e + 1];
        const uint32_t fa = g0 <= 4 ? (ha << (4 - g0)) & 0x10101010u : (ha >> (g0 - 4)) & 0x10101010u;
        const uint32_t fb = g0 <= 4 ? (hb << (4 - g0)) & 0x10101010u : (hb >> (g0 - 4)) & 0x10101010u;
        if constexpr (v == 0) return codes8((a & 0x0f0f0f0fu) | fa, (b & 0x0f0f0f0fu) | fb);
        else return codes8(((a >> 4) & 0x0f0f0f0fu) | fa, ((b >> 4) & 0x0f0f0f0fu) | fb);
    } else {
        // Sub-block g = (h >> 1) + 2v of half k; its top bits sit at bits 2g, 2g + 1 of qh.
        const uint32_t ha = r.qh[k][2 * e] & hmask, hb = r.qh[k][2 * e + 1] & hmask;
        const uint32_t qa = r.l[k][2 * e], qb = r.l[k][2 * e + 1];
        if constexpr (v == 0) return codes8(bfi(0x0f0f0f0fu, qa, ha << sl), bfi(0x0f0f0f0fu, qb, hb << sl));
        else return codes8(bfi(0x0f0f0f0fu, qa >> 4, ha >> sh), bfi(0x0f0f0f0fu, qb >> 4, hb >> sh));
    }
}

// MFMA t's activation operand depends on t only through rho(t) = 2 (t >> 2) + (t & 1) (which
// A row each lane group feeds) and e(t) = (t >> 1) & 1 (which half of the slice). aptr[rho]
// points at the lane's own slice when its A row is fed in those MFMAs, else at the zero
// slots; e selects the 16-byte half.
template <uint32_t TYPE>
constexpr int kRho = TYPE == kQ6K ? 4 : 8;

template <uint32_t TYPE>
__device__ __forceinline__ bool a_match(int c, int rho) {
    if constexpr (TYPE != kQ6K) return (c >> 2) == (rho >> 1) && (c & 1) == (rho & 1);
    else return (c >> 3) == (rho >> 1) && ((c >> 2) & 1) == (rho & 1);
}

template <uint32_t TYPE, int T>
__device__ __forceinline__ void one_mfma(f32x4 &D, const WT<TYPE> &wt, const u32x4 *const (&aptr)[kRho<TYPE>],
                                         uint32_t hmask, uint32_t sl, uint32_t sh) {
    constexpr int rho = 2 * (T >> 2) + (T & 1), e = (T >> 1) & 1;
    D = mfma16(aptr[rho][e], codes<TYPE, T>(wt, hmask, sl, sh), D);
}

template <uint32_t TYPE, int... Ts>
__device__ __forceinline__ void all_mfmas(std::integer_sequence<int, Ts...>, f32x4 &D, const WT<TYPE> &wt,
                                          const u32x4 *const (&aptr)[kRho<TYPE>], uint32_t hmask, uint32_t sl,
                                          uint32_t sh) {
    (one_mfma<TYPE, Ts>(D, wt, aptr, hmask, sl, sh), ...);
}

// Staged loads (Q6_K): where load i of this lane goes: row r of the 16-row tile (4 bits per
// load in `rows`), byte offset j within the row's segment of the set, and the LDS byte
// address in the tile.
template <uint32_t TYPE>
struct ChunkMap {
    uint32_t roff[Geo<TYPE>::kLoads];  // r * pitch
    uint32_t j[Geo<TYPE>::kLoads];
    uint32_t l[Geo<TYPE>::kLoads];
    uint32_t rows;                     // r of load i in bits 4i .. 4i + 3
    uint32_t hi;                       // bit i: the chunk that carries d
};

// One pipeline stage: the raw chunks of one (tile, set) unit (Q4_K: the lane's pieces
// q[0..3] and header, as in WT) and the lane's activation slice (zero when it owns none).
template <uint32_t TYPE>
struct Stage {
    u32x4 ch[Geo<TYPE>::kLoads];
    u32x4 xa[2];
};

// Position of a unit: 16-row tile and K set.
struct Pos {
    int tile, set;
};

template <uint32_t TYPE>
__device__ __forceinline__ void issue(Stage<TYPE> &st, const ChunkMap<TYPE> &cm, __amdgpu_buffer_rsrc_t xr,
                                      const uint8_t *w, int64_t pitch, int N, Pos p, uint32_t xo, int nsb,
                                      int lane) {
    using G = Geo<TYPE>;
    const uint32_t vo = 2u * (uint32_t)(p.set * G::kSetK) + xo;
    st.xa[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, vo, 0, 0));
    st.xa[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, vo + 16u, 0, 0));
    if constexpr (!G::kStaged) {
        // Row c of the tile (rows past N re-read row N - 1); a Q4_K set past an odd block
        // count reads its first block again in place of the second.
        const int c = lane & 15, h = lane >> 4;
        const int row = min(16 * p.tile + c, N - 1);
        constexpr int kBytes = G::kSetBytes / 2, kQs = TYPE == kQ5K ? 48 : 16;
        const uint8_t *b0 = w + (int64_t)row * pitch + (int64_t)p.set * G::kSetBytes;
        const uint8_t *b1 = (2 * p.set + 1 >= nsb) ? b0 : b0 + kBytes;
        st.ch[0] = *reinterpret_cast<const u32x4a2 *>(b0 + kQs + 16 * h);
        st.ch[1] = *reinterpret_cast<const u32x4a2 *>(b0 + kQs + 64 + 16 * h);
        st.ch[2] = *reinterpret_cast<const u32x4a2 *>(b1 + kQs + 16 * h);
        st.ch[3] = *reinterpret_cast<const u32x4a2 *>(b1 + kQs + 64 + 16 * h);
        st.ch[4] = *reinterpret_cast<const u32x4a2 *>((h >> 1) ? b1 : b0);
        if constexpr (TYPE == kQ5K) {
            st.ch[5] = *reinterpret_cast<const u32x4a2 *>(b0 + 16 + 16 * (h & 1));
            st.ch[6] = *reinterpret_cast<const u32x4a2 *>(b1 + 16 + 16 * (h & 1));
        }
    } else {
        const int n0 = 16 * p.tile;
        const uint8_t *base = w + (int64_t)n0 * pitch + (int64_t)p.set * G::kSetBytes;
        const bool ragged = n0 + 16 > N;  // last tile: rows past N re-read row N - 1
#pragma unroll
        for (int i = 0; i < G::kLoads; ++i) {
            if (i < G::kLoads - 1 || 64 * i + lane < 16 * G::kChunks) {
                uint32_t roff = cm.roff[i];
                if (ragged) roff = (uint32_t)min((int)((cm.rows >> (4 * i)) & 15u), N - 1 - n0) * (uint32_t)pitch;
                st.ch[i] = *reinterpret_cast<const u32x4a2 *>(base + roff + cm.j[i]);
            }
        }
    }
    asm volatile("" ::: "memory");  // keep the loads here, a full stage ahead of their use
}

template <uint32_t TYPE>
__device__ __forceinline__ float compute(const Stage<TYPE> &st, const ChunkMap<TYPE> &cm, uint8_t *tile,
                                         u32x4 *xs_w, const u32x4 *const (&aptr)[kRho<TYPE>], int own, int c, int h,
                                         int lane, int set, int nsb, uint32_t hmask, uint32_t sl, uint32_t sh,
                                         uint32_t mA, uint32_t mB, uint32_t mC) {
    using G = Geo<TYPE>;
    if (own < G::kSlots) {
        xs_w[own] = st.xa[0];
        xs_w[own + 1] = st.xa[1];
    }
    WT<TYPE> r;
    if constexpr (G::kStaged) {
        // Stage the unit's rows in LDS (Q6_K: the 14th chunk of a row only carries d).
#pragma unroll
        for (int i = 0; i < G::kLoads; ++i) {
            if (i < G::kLoads - 1 || 64 * i + lane < 16 * G::kChunks) {
                if ((cm.hi >> i) & 1) *reinterpret_cast<uint32_t *>(tile + cm.l[i]) = st.ch[i].w >> 16;
                else *reinterpret_cast<u32x4 *>(tile + cm.l[i]) = st.ch[i];
            }
        }
        read_wt<TYPE>(r, tile, c, h);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) r.q[k] = st.ch[k];
        r.hd = st.ch[4];
        if constexpr (TYPE == kQ5K) {
            const uint32_t s = 2u * (uint32_t)(h >> 1);
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) r.qh[b][i] = st.ch[5 + b][i] >> s;
        }
    }
    const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    f32x4 X = mfma16(st.xa[0], ones, f32x4{0.f, 0.f, 0.f, 0.f});
    X = mfma16(st.xa[1], ones, X);
    f32x4 D = {0.f, 0.f, 0.f, 0.f};
    all_mfmas<TYPE>(std::make_integer_sequence<int, G::kMfma>{}, D, r, aptr, hmask, sl, sh);
    if constexpr (TYPE != kQ6K) {
        // Sub-blocks 4 (h & 1) + i of block 2 set + (h >> 1): 6-bit scales and mins (Q4_K and
        // Q5_K share the header and w = d sc q - dmin m; Q5_K codes run to 31).
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w;
        const uint32_t sc4 = (s0 & mA) | (s2 & mB) | ((s0 >> 2) & mC);
        const uint32_t m4 = (s1 & mA) | ((s2 >> 4) & mB) | ((s1 >> 2) & mC);
        const float d = half_to_float(r.hd.x), dmin = half_to_float(r.hd.x >> 16);
        float sd = 0.f, sx = 0.f, mx = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float fs = (float)((sc4 >> (8 * i)) & 255u), fm = (float)((m4 >> (8 * i)) & 255u);
            sd = __builtin_fmaf(fs, D[i], sd);
            sx = __builtin_fmaf(fs, X[i], sx);
            mx = __builtin_fmaf(fm, X[i], mx);
        }
        // The second block of the last set does not exist when the block count is odd.
        const float part = __builtin_fmaf(d, __builtin_fmaf(-128.f, sx, sd), -dmin * mx);
        return 2 * set + (h >> 1) < nsb ? part : 0.f;
    } else {
        float sd = 0.f, sx = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float fs = (float)(int8_t)(uint8_t)(r.sc >> (8 * i));
            sd = __builtin_fmaf(fs, D[i], sd);
            sx = __builtin_fmaf(fs, X[i], sx);
        }
        return half_to_float(r.d) * __builtin_fmaf(-160.f, sx, sd);
    }
}

// Workgroup: one 16-row tile, W wavefronts; wavefront w takes the sets w, w + W, ... (so at
// any time the workgroup reads W consecutive sets: long contiguous runs of each row), with
// two sets in flight (ping-pong stages). Partial row sums are added through LDS in
// wavefront order.
template <uint32_t TYPE>
__global__ __launch_bounds__(1024) void k_gemv1(const uint16_t *__restrict__ x, Gemv1Segments segs, int64_t pitch,
                                                 int nsb, int nks) {
    using G = Geo<TYPE>;
    // Dynamic LDS, per wavefront: the staged rows, then the A-operand slots; then the sums.
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int kTile = G::kStaged ? 16 * G::kRowLds : 0, kWaveLds = wave_lds_bytes<TYPE>();
    const int tid = (int)threadIdx.x, lane = tid & 63, h = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps the set loop scalar
    const int nw = (int)(blockDim.x >> 6);
    // Segment of this workgroup's tile: matrices sharing x (same K and type) are laid end to
    // end in tile order.
    int seg = 0;
    while (seg + 1 < segs.count && (int)blockIdx.x >= segs.tile_begin[seg + 1]) ++seg;
    const int tile_id = (int)blockIdx.x - segs.tile_begin[seg];
    const uint8_t *__restrict__ w = segs.w[seg];
    uint16_t *__restrict__ y = segs.y[seg];
    const uint16_t *__restrict__ bias = segs.bias[seg];
    const int N = segs.n[seg];
    uint8_t *tile = lds + wave * kWaveLds;
    u32x4 *xs_w = reinterpret_cast<u32x4 *>(tile + kTile);  // owned slices, a spare slot, two zero slots
    float *red = reinterpret_cast<float *>(lds + nw * kWaveLds);  // [nw][16]

    // Staged loads: chunk q = 64 i + lane of a (tile, set) unit is row q / kChunks, chunk
    // q % kChunks of the row.
    ChunkMap<TYPE> cm{};
    if constexpr (G::kStaged) {
#pragma unroll
        for (int i = 0; i < G::kLoads; ++i) {
            const int q = min(64 * i + lane, 16 * G::kChunks - 1), r = q / G::kChunks, j = q % G::kChunks;
            cm.rows |= (uint32_t)r << (4 * i);
            cm.roff[i] = (uint32_t)r * (uint32_t)pitch;
            cm.j[i] = j < 13 ? 16 * j : 194;  // the 14th chunk ends at the block end
            cm.l[i] = r * G::kRowLds + (j < 13 ? 16 * j : 208);
            cm.hi |= (uint32_t)(j == 13) << i;
        }
    }

    // As an A lane: which activation slice (two 8-element halves) this lane owns, if any.
    bool elig;
    int xoff, own;
    if constexpr (TYPE != kQ6K) {
        elig = ((c >> 1) & 1) == (h >> 1);  // sub-block c, positions 16 (h & 1) .. + 15
        xoff = 32 * c + 16 * (h & 1);
        own = 2 * (2 * c + (h & 1));
    } else {
        elig = (c & 3) == h;  // group c, all 16 positions
        xoff = 16 * c;
        own = 2 * c;
    }
    const uint32_t xo = elig ? 2u * (uint32_t)xoff : kOOR;
    if (!elig) own = G::kSlots;  // marks "owns no slice"
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(x), 0, 2 * 256 * nsb, 0x00020000);
    // Zero slots at an odd 16-byte index, so that they never share LDS banks with the owned
    // slot read in the same MFMA (owned slots of one MFMA all have the parity of e).
    if (lane < 2) xs_w[G::kSlots + 1 + lane] = u32x4{0, 0, 0, 0};
    const u32x4 *aptr[kRho<TYPE>];
#pragma unroll
    for (int rho = 0; rho < kRho<TYPE>; ++rho)
        aptr[rho] = xs_w + ((elig && a_match<TYPE>(c, rho)) ? own : G::kSlots + 1);

    // Q6_K code assembly constants for sub-blocks (h >> 1) and (h >> 1) + 2.
    const uint32_t sh = 2u * (uint32_t)(h >> 1), sl = 4u - sh, hmask = 0x33333333u << sh;
    // Q4_K scale/min field masks: lanes with h odd hold sub-blocks 4..7 of their block.
    const bool hi4 = (h & 1) != 0;
    const uint32_t mA = hi4 ? 0u : 0x3f3f3f3fu, mB = hi4 ? 0x0f0f0f0fu : 0u, mC = hi4 ? 0x30303030u : 0u;

    const int nmine = wave < nks ? (nks - 1 - wave) / nw + 1 : 0;
    float acc = 0.f;
    if (nmine > 0) {
        // Straight-line ping-pong: stage A holds set ks, stage B set ks + W.
        Stage<TYPE> A, B;
        int ks = wave;
        issue<TYPE>(A, cm, xr, w, pitch, N, Pos{tile_id, ks}, xo, nsb, lane);
        for (int i = (nmine - 1) >> 1; i > 0; --i, ks += 2 * nw) {
            issue<TYPE>(B, cm, xr, w, pitch, N, Pos{tile_id, ks + nw}, xo, nsb, lane);
            acc += compute<TYPE>(A, cm, tile, xs_w, aptr, own, c, h, lane, ks, nsb, hmask, sl, sh, mA, mB, mC);
            issue<TYPE>(A, cm, xr, w, pitch, N, Pos{tile_id, ks + 2 * nw}, xo, nsb, lane);
            acc += compute<TYPE>(B, cm, tile, xs_w, aptr, own, c, h, lane, ks + nw, nsb, hmask, sl, sh, mA, mB, mC);
        }
        if ((nmine & 1) == 0) {  // two sets left
            issue<TYPE>(B, cm, xr, w, pitch, N, Pos{tile_id, ks + nw}, xo, nsb, lane);
            acc += compute<TYPE>(A, cm, tile, xs_w, aptr, own, c, h, lane, ks, nsb, hmask, sl, sh, mA, mB, mC);
            acc += compute<TYPE>(B, cm, tile, xs_w, aptr, own, c, h, lane, ks + nw, nsb, hmask, sl, sh, mA, mB, mC);
        } else {
            acc += compute<TYPE>(A, cm, tile, xs_w, aptr, own, c, h, lane, ks, nsb, hmask, sl, sh, mA, mB, mC);
        }
    }

    // Row n = c: add the four lane groups, then the wavefronts (in order) through LDS.
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (h == 0) red[16 * wave + c] = acc;
    __syncthreads();
    if (tid < 16) {
        const int n = 16 * tile_id + tid;
        // N is even for kActSiluGlu, so lanes 2c and 2c + 1 (gate, up) pass this test together.
        if (n < N) {
            float v = 0.f;
            for (int k = 0; k < nw; ++k) v += red[16 * k + tid];
            uint32_t out = float_to_bf16_bits(v);
            if (bias) out = float_to_bf16_bits(bf16_to_float(out) + bf16_to_float(bias[n]));
            if (segs.act == kActSiluGlu) {
                const uint32_t up = (uint32_t)__shfl_xor((int)out, 1);
                if ((n & 1) == 0) y[n >> 1] = (uint16_t)silu_glu_bits(out, up);
            } else {
                y[n] = (uint16_t)(segs.act == kActGeluTanh ? gelu_tanh_bits(out) : out);
            }
        }
    }
}

template <uint32_t TYPE>
hipError_t launch_type(const uint16_t *x, const Gemv1Segments &segs, int K, hipStream_t stream, int force_w) {
    using G = Geo<TYPE>;
    const int nsb = K / 256, nks = (nsb + G::kBlocksPerSet - 1) / G::kBlocksPerSet;
    const int tiles = segs.tile_begin[segs.count];
    // Wavefronts per workgroup: Q6_K as many as keep the whole grid resident at once (about
    // 16 wavefronts per CU, 256 CUs), at most 16; Q4_K (direct loads, fewer registers) 4 to 8,
    // the best measured on MI355X for 7-76 MB matrices. At most one per set.
    int W = std::max(1, 4096 / tiles);
    if (!G::kStaged) W = std::min(8, std::max(4, W));
    if (force_w > 0) W = force_w;
    W = std::min(W, std::min(16, nks));
    const int64_t pitch = (int64_t)nsb * (TYPE == kQ4K ? kQ4KBytes : TYPE == kQ5K ? kQ5KBytes : kQ6KBytes);
    const size_t lds = (size_t)W * (wave_lds_bytes<TYPE>() + 16 * sizeof(float));
    hipLaunchKernelGGL((k_gemv1<TYPE>), dim3((unsigned)tiles), dim3((unsigned)(64 * W)), lds, stream, x, segs, pitch,
                       nsb, nks);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv1(uint32_t type, const uint16_t *x, const uint8_t *w, int N, int K, uint16_t *y,
                        const uint16_t *bias_bf16, hipStream_t stream, int force_waves, int act) {
    Gemv1Segments segs{};
    segs.count = 1;
    segs.act = act;
    segs.w[0] = w;
    segs.y[0] = y;
    segs.bias[0] = bias_bf16;
    segs.n[0] = N;
    segs.tile_begin[0] = 0;
    segs.tile_begin[1] = (N + 15) / 16;
    return launch_gemv1_segments(type, x, segs, K, stream, force_waves);
}

hipError_t launch_gemv1_segments(uint32_t type, const uint16_t *x, const Gemv1Segments &segs, int K,
                                 hipStream_t stream, int force_waves) {
    if (type == kQ4K) return launch_type<kQ4K>(x, segs, K, stream, force_waves);
    if (type == kQ5K) return launch_type<kQ5K>(x, segs, K, stream, force_waves);
    return launch_type<kQ6K>(x, segs, K, stream, force_waves);
}

}  // namespace tc
