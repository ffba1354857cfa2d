// Quantized linear for 9..64 activation rows (text-encoder prompts, short token runs), Q4_K /
// Q6_K: y[m, n] = bf16(sum_k x[m, k] * bf16(w[n, k])) (+ bias after the cast), w the exact
// dequantized weight rounded to bf16 (the reference pager's bf16 decode,
// gguf_weight_pager.cpp:347-349), fp32 accumulation. HBM-bound: every weight byte is read
// once per call.
//
// Replaces the mid-M side of mx::quantized_matmul (native/backends/mlx.cpp:678-679) for the
// Qwen text-encoder calls (components/text/qwen3_gguf.hpp:7-77, prompts of <= 256 tokens).
//
// Scheme (workgroup of 4 wavefronts, 64 weight rows; wavefront w owns rows 16 w .. 16 w + 15):
//   * for each super-block of K, the activation slab (16 RG rows x 256 columns, rows >= M read
//     as zero through the buffer range check) is copied global -> LDS by the buffer-load DMA
//     one super-block ahead into one of two LDS buffers, shared by the four wavefronts
//     (16-byte pieces XOR-swizzled by row so that fragment reads do not conflict);
//   * the raw weight bytes of the wavefront's 16 rows go straight into registers five
//     super-blocks ahead (buffer loads: each is exactly one instruction, which the explicit
//     vmcnt accounting below relies on);
//   * per 32-column group g: lane (n, h) dequantizes the 8 weights of row n at columns
//     32 g + 8 h .. + 7 to bf16 (fma(d sc, q, -dmin m) / (d sc)(q - 32), exact, one
//     rounding, then RNE) as the B operand of v_mfma_f32_16x16x32_bf16, and runs one MFMA per
//     16-row group of activations (A from LDS);
//   * K may be split into S slices (few weight tiles, long K): each slice writes fp32 partial
//     sums [S][M][N], which k_skinny_reduce adds in slice order (deterministic).
#include "tc_device.h"
#include "tc_kernels.h"

#include <algorithm>
#include <type_traits>

namespace tc {
namespace {

constexpr int kSkWaves = 4;
constexpr int kSkRows = 16 * kSkWaves;  // weight rows per workgroup
constexpr int kSlab = 512;              // bytes of one activation row of a super-block
// LDS slab buffers (DMA kBufs - 1 super-blocks ahead). Two (64 KB at 64 rows: two workgroups
// per CU) measured faster than three (96 KB: one workgroup per CU).
constexpr int kBufs = 2;
static_assert(kBufs == 2 || kBufs == 3, "slab buffers");
constexpr int kWSlots = 6;              // weight register stages (loads five super-blocks ahead)

typedef __attribute__((address_space(3))) void lds_void;

// Raw weight bytes of one super-block for one lane (n, h):
// Q4_K: q[j] = qs[32 j + 8 h .. + 7] (groups 2 j and 2 j + 1), hd = the block header;
// Q5_K: as Q4_K (qs at byte 48), and qh[0] = qh[8 h .. + 7]: bit g of byte c is the fifth code
//       bit of column 8 h + c of group g (gguf_decode.cpp:77-90);
// Q6_K: q[2 f + u] = ql[64 f + 32 u + 8 h .. + 7], qh[f] = qh[32 f + 8 h .. + 7],
//       hd = the 16 int8 scales, dw >> 16 = d (fp16 bits).
struct WStage {
    u32x2 q[4];
    u32x2 qh[2];
    u32x4 hd;
    uint32_t dw;
};
template <uint32_t TYPE>
constexpr int kWLoads = TYPE == kQ4K ? 5 : TYPE == kQ5K ? 6 : 8;  // buffer-load instructions per WStage
// Cache policy of the weight loads: the default (a non-temporal hint measured slower).
constexpr int kWeightPolicy = 0;

template <uint32_t TYPE>
__device__ __forceinline__ void load_stage(WStage &s, __amdgpu_buffer_rsrc_t wr, int rowoff, int sb, int h) {
    if constexpr (TYPE == kQ4K || TYPE == kQ5K) {
        constexpr int kQs = TYPE == kQ4K ? 16 : 48;  // the qs bytes (Q5_K: after the 32-byte qh plane)
        const int b = rowoff + sb * (int)(TYPE == kQ4K ? kQ4KBytes : kQ5KBytes);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            s.q[j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, b + kQs + 32 * j + 8 * h, 0, kWeightPolicy));
        if constexpr (TYPE == kQ5K)
            s.qh[0] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, b + 16 + 8 * h, 0, kWeightPolicy));
        s.hd = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, b, 0, kWeightPolicy));
    } else {
        // Q6_K blocks are 2-byte aligned: loads at 2-byte aligned offsets (the hardware's
        // unaligned access mode).
        const int b = rowoff + sb * (int)kQ6KBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            s.q[j] = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, b + 64 * (j >> 1) + 32 * (j & 1) + 8 * h, 0, kWeightPolicy));
#pragma unroll
        for (int f = 0; f < 2; ++f)
            s.qh[f] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, b + 128 + 32 * f + 8 * h, 0, kWeightPolicy));
        s.hd = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, b + 192, 0, kWeightPolicy));
        s.dw = __builtin_amdgcn_raw_buffer_load_b32(wr, b + 206, 0, kWeightPolicy);
    }
}

// Per-block scale terms of a Q4_K lane: a[g] = d * sc_g, b[g] = dmin * m_g for the 8 groups.
// The 6-bit unpack of get_scale_min_k4 (gguf_decode.cpp:48-54) for all 8 groups at once:
// sc[0..3] = s0 & 63, m[0..3] = s1 & 63, sc[4..7] = (s2 & 15) | (s0 >> 6) << 4,
// m[4..7] = (s2 >> 4) | (s1 >> 6) << 4, byte-wise.
struct Q4Scales {
    uint32_t sc_lo, m_lo, sc_hi, m_hi;
    float d, dmin;
};
__device__ __forceinline__ Q4Scales q4_scales(const u32x4 &hd) {
    Q4Scales s;
    s.d = half_to_float(hd.x);
    s.dmin = half_to_float(hd.x >> 16);
    s.sc_lo = hd.y & 0x3f3f3f3fu;
    s.m_lo = hd.z & 0x3f3f3f3fu;
    s.sc_hi = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
    s.m_hi = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
    return s;
}

// The 8 bf16 weights lane (n, h) feeds to the MFMA of group G (columns 32 G + 8 h .. + 7).
template <uint32_t TYPE, int G>
__device__ __forceinline__ bf16x8 dequant_group(const WStage &s, const Q4Scales &q4, float d6, int h) {
    uint32_t c0, c1;
    float a, b;
    if constexpr (TYPE == kQ4K || TYPE == kQ5K) {
        constexpr int j = G >> 1;
        const uint32_t w0 = s.q[j].x, w1 = s.q[j].y;
        uint32_t l0 = (G & 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu;
        uint32_t l1 = (G & 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu;
        if constexpr (TYPE == kQ5K) {  // fifth bit: bit G of each qh byte
            l0 |= ((s.qh[0].x >> G) & 0x01010101u) << 4;
            l1 |= ((s.qh[0].y >> G) & 0x01010101u) << 4;
        }
        c0 = launder(l0);
        c1 = launder(l1);
        const uint32_t scw = G < 4 ? q4.sc_lo : q4.sc_hi, mw = G < 4 ? q4.m_lo : q4.m_hi;
        constexpr int sh = 8 * (G & 3);
        a = q4.d * (float)((scw >> sh) & 0xffu);
        b = q4.dmin * (float)((mw >> sh) & 0xffu);
    } else {
        // Step G: half f = G / 4, quarter g = G % 4; scale sc[8 f + 2 g + h / 2].
        constexpr int f = G >> 2, g = G & 3;
        const u32x2 ql = s.q[2 * f + (g & 1)], qh = s.qh[f];
        const uint32_t l0 = g < 2 ? ql.x & 0x0f0f0f0fu : (ql.x >> 4) & 0x0f0f0f0fu;
        const uint32_t l1 = g < 2 ? ql.y & 0x0f0f0f0fu : (ql.y >> 4) & 0x0f0f0f0fu;
        c0 = launder(l0 | (((qh.x >> (2 * g)) & 0x03030303u) << 4));
        c1 = launder(l1 | (((qh.y >> (2 * g)) & 0x03030303u) << 4));
        constexpr int idx = 8 * f + 2 * g;  // + h / 2
        const uint32_t word = s.hd[idx >> 2] >> (8 * ((idx & 3) + (h >> 1)));
        a = d6 * (float)(int8_t)(uint8_t)word;
        b = 32.f * a;  // (code - 32) * a = code * a - 32 a, exact
    }
    const float v0 = __builtin_fmaf(a, (float)(c0 & 0xffu), -b), v1 = __builtin_fmaf(a, (float)((c0 >> 8) & 0xffu), -b);
    const float v2 = __builtin_fmaf(a, (float)((c0 >> 16) & 0xffu), -b), v3 = __builtin_fmaf(a, (float)(c0 >> 24), -b);
    const float v4 = __builtin_fmaf(a, (float)(c1 & 0xffu), -b), v5 = __builtin_fmaf(a, (float)((c1 >> 8) & 0xffu), -b);
    const float v6 = __builtin_fmaf(a, (float)((c1 >> 16) & 0xffu), -b), v7 = __builtin_fmaf(a, (float)(c1 >> 24), -b);
    const u32x4 packed = {pack_bf16x2(v0, v1), pack_bf16x2(v2, v3), pack_bf16x2(v4, v5), pack_bf16x2(v6, v7)};
    return __builtin_bit_cast(bf16x8, packed);
}

// Waits until at most VM of this wavefront's vector-memory operations are outstanding and its
// LDS reads have returned (the buffer a later DMA overwrites is then free), then joins the
// workgroup barrier.
template <int VM>
__device__ __forceinline__ void sk_wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

// Grid: tiles x S workgroups; workgroup b takes weight tile b % tiles and K slice b / tiles.
// The tiles may span several weight matrices of one type and K applied to the same x (fused
// projections, S = 1): segment s covers tiles [tile_begin[s], tile_begin[s + 1]).
template <uint32_t TYPE, int RG>
// x and w are deliberately not __restrict__: with it the compiler may move their loads across
// the ordering fences (asm memory clobbers) that the explicit vmcnt accounting depends on.
__global__ __launch_bounds__(256) void k_skinny(const uint16_t *x, int64_t x_stride, int M, Gemv1Segments segs,
                                                int64_t pitch, int nsb, int tiles, int splits,
                                                float *__restrict__ partials) {
    // The slab buffers. Fragments are read with inline-asm ds_read_b128 (the explicit vmcnt
    // wait + barrier below orders them after the DMA): the compiler's own DMA tracking would
    // otherwise wait for DMA issued for later blocks, and with it for the weight prefetch.
    constexpr int kBufBytes = 16 * RG * kSlab;
    __shared__ __attribute__((aligned(16))) uint8_t xs[kBufs * kBufBytes];
    auto xbuf = [&](auto btag) -> uint8_t * { return xs + decltype(btag)::value * kBufBytes; };
    const int gtile = (int)blockIdx.x % tiles, slice = (int)blockIdx.x / tiles;
    int seg = 0;
    while (seg + 1 < segs.count && gtile >= segs.tile_begin[seg + 1]) ++seg;
    const int tile = gtile - segs.tile_begin[seg];
    const uint8_t *w = segs.w[seg];
    uint16_t *__restrict__ y = segs.y[seg];
    const int64_t y_stride = segs.y_stride[seg];
    const uint16_t *__restrict__ bias = segs.bias[seg];
    const int N = segs.n[seg];
    const int sb0 = (int)((int64_t)slice * nsb / splits), sb1 = (int)((int64_t)(slice + 1) * nsb / splits);
    const int tid = (int)threadIdx.x, lane = tid & 63, n = lane & 15, h = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = kSkRows * tile;  // first weight row of the tile
    const int rows = min(kSkRows, N - row0);
    constexpr int kBlockBytes = TYPE == kQ4K ? (int)kQ4KBytes : TYPE == kQ5K ? (int)kQ5KBytes : (int)kQ6KBytes;

    // Weights: a buffer over the tile's rows; lane (n, h) reads row min(16 wave + n, rows - 1).
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w + (int64_t)row0 * pitch), (short)0, (int)((int64_t)rows * pitch), 0x00020000);
    const int rowoff = (int)((int64_t)min(16 * wave + n, rows - 1) * pitch);

    // Activation DMA: instruction J (0 .. 8 RG - 1; wavefront w issues J = 2 RG w + j) writes LDS
    // bytes [1024 J, 1024 J + 1024) = slab rows 2 J, 2 J + 1; lane L carries row 2 J + L / 32,
    // LDS slot L % 32, i.e. the row's 16-byte piece (L % 32) ^ (row & 15). Rows >= M are out of
    // the buffer's range and read as zero. The super-block's column base goes in soffset.
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(x), (short)0, (int)((int64_t)M * x_stride * 2), 0x00020000);
    int voff[8];  // first 2 RG used (a template-sized array captured by the lambdas below makes
                  // the host-side instantiation of the kernel invalid, dropping its launch stub)
#pragma unroll
    for (int j = 0; j < 2 * RG; ++j) {
        const int row = 2 * (2 * RG * wave + j) + (lane >> 5);
        voff[j] = (int)((int64_t)row * x_stride * 2) + 16 * ((lane & 31) ^ (row & 15));
    }
    auto dma = [&](auto btag, int sb) {
#pragma unroll
        for (int j = 0; j < 2 * RG; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void *)(xbuf(btag) + 1024 * (2 * RG * wave + j)), 16,
                                                     voff[j], kSlab * sb, 0, 0);
        asm volatile("" ::: "memory");  // keep each batch in issue order (the vmcnt accounting)
    };
    constexpr int kDma = 2 * RG, kW = kWLoads<TYPE>;

    WStage ws[kWSlots];
    f32x4 acc[4];  // first RG used (fixed size for the same reason)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto wload = [&](auto stag, int sb) {
        load_stage<TYPE>(ws[decltype(stag)::value], wr, rowoff, sb, h);
        asm volatile("" ::: "memory");
    };
    // Fragment reads: lane (r, hq) reads slab row 16 i + r, piece 4 g + hq (slot ^ (r & 15)): the 16
    // rows of a fragment read land on 16 different 16-byte bank groups (the 512-byte slab rows all
    // start on the same bank, and a swizzle by r & 7 left rows r and r + 8 colliding).
    const uint32_t frag = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)xs + n * kSlab;
    const int fswz = n & 15;

    // Issue order (iteration b, after its barrier): DMA of block b + kBufs - 1, then the weights
    // of block b + 5. The prologue issues what the iterations sb0 - 5 .. sb0 - 1 would have issued.
    // Every stage is issued unconditionally, with block indices past the slice clamped to its
    // last block (re-read, never used): the number of loads in flight is then the same on every
    // path, which keeps both the explicit waits below and the compiler's own exact.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    const int last = sb1 - 1;  // sb0 <= last: every slice holds at least one super-block
    wload(I0{}, sb0);
    wload(I1{}, min(sb0 + 1, last));
    wload(I2{}, min(sb0 + 2, last));
    if constexpr (kBufs == 3) dma(I0{}, sb0);
    wload(I3{}, min(sb0 + 3, last));
    if constexpr (kBufs == 3) dma(I1{}, min(sb0 + 1, last));
    else dma(I0{}, sb0);
    wload(I4{}, min(sb0 + 4, last));

    auto body = [&](auto ktag, int b) {
        constexpr int k = decltype(ktag)::value;  // (b - sb0) % 6
        constexpr int buf = k % kBufs;
        // This wavefront's DMA of block b is complete once no more than the loads issued after
        // it are outstanding: W(b + 6 - kBufs) (issued with it), then DMA and W of each later
        // iteration (three buffers: DMA(b + 1), W(b + 4)). The barrier then makes every
        // wavefront's part visible and frees the buffer of block b - 1.
        sk_wait_barrier<kW + (kBufs - 2) * (kDma + kW)>();
        dma(std::integral_constant<int, (k + kBufs - 1) % kBufs>{}, min(b + kBufs - 1, last));
        wload(std::integral_constant<int, (k + 5) % kWSlots>{}, min(b + 5, last));
        const WStage &s = ws[k];
        Q4Scales q4{};
        float d6 = 0.f;
        if constexpr (TYPE == kQ4K || TYPE == kQ5K) q4 = q4_scales(s.hd);
        else d6 = half_to_float(s.dw >> 16);
        const uint32_t xb = frag + buf * kBufBytes;
        // Fragment reads of group G + 2 are issued right after group G's wait, so that they
        // overlap two groups' MFMAs and dequant; the groups' fragments rotate through three
        // register sets (no copies of registers whose loads are in flight).
        u32x4 f0[4], f1[4];
        auto read = [&](auto gtag, u32x4(&dst)[4]) {
            constexpr int G = decltype(gtag)::value;
            const uint32_t addr = xb + 16 * ((4 * G + h) ^ fswz);
#pragma unroll
            for (int i = 0; i < RG; ++i)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst[i]) : "v"(addr), "i"(16 * i * kSlab));
        };
        // Fragments two groups ahead (three register sets): group G waits only for its own
        // reads (the RG reads of group G + 1 may still be in flight; LDS reads return in order).
        u32x4 f2[4];
        read(std::integral_constant<int, 0>{}, f0);
        read(std::integral_constant<int, 1>{}, f1);
        auto group = [&](auto gtag, u32x4(&a)[4], u32x4(&nxt)[4]) {
            constexpr int G = decltype(gtag)::value;
            const bf16x8 bw = dequant_group<TYPE, G>(s, q4, d6, h);
            constexpr int kAhead = G < 7 ? RG : 0;  // reads of group G + 1 left in flight
            if constexpr (RG == 1) asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a[0]) : "n"(kAhead));
            else if constexpr (RG == 2) asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a[0]), "+v"(a[1]) : "n"(kAhead));
            else asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]) : "n"(kAhead));
            if constexpr (G < 6) read(std::integral_constant<int, G + 2>{}, nxt);
#pragma unroll
            for (int i = 0; i < RG; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[i]), bw, acc[i], 0, 0, 0);
        };
        group(std::integral_constant<int, 0>{}, f0, f2);
        group(std::integral_constant<int, 1>{}, f1, f0);
        group(std::integral_constant<int, 2>{}, f2, f1);
        group(std::integral_constant<int, 3>{}, f0, f2);
        group(std::integral_constant<int, 4>{}, f1, f0);
        group(std::integral_constant<int, 5>{}, f2, f1);
        group(std::integral_constant<int, 6>{}, f0, f2);
        group(std::integral_constant<int, 7>{}, f1, f0);
    };
    for (int b = sb0; b < sb1; b += kWSlots) {
        body(I0{}, b);
        if (b + 1 >= sb1) break;
        body(I1{}, b + 1);
        if (b + 2 >= sb1) break;
        body(I2{}, b + 2);
        if (b + 3 >= sb1) break;
        body(I3{}, b + 3);
        if (b + 4 >= sb1) break;
        body(I4{}, b + 4);
        if (b + 5 >= sb1) break;
        body(std::integral_constant<int, 5>{}, b + 5);
    }

    // Lane (n, h) holds y[16 i + 4 h + v][row0 + 16 wave + n], v = 0..3 (MFMA output layout).
    const int col = row0 + 16 * wave + n;
    if (col >= N) return;
    const float bv = (splits == 1 && bias) ? bf16_to_float(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < RG; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = 16 * i + 4 * h + v;
            if (m >= M) continue;
            if (splits == 1) {
                uint32_t out = float_to_bf16_bits(acc[i][v]);
                if (bias) out = float_to_bf16_bits(bf16_to_float(out) + bv);
                if (segs.act == kActSiluGlu) {
                    // Lanes n and n ^ 1 hold the gate and up of one output (row0 and N even).
                    const uint32_t up = (uint32_t)__shfl_xor((int)out, 1);
                    if ((col & 1) == 0) y[(int64_t)m * y_stride + (col >> 1)] = (uint16_t)silu_glu_bits(out, up);
                } else {
                    y[(int64_t)m * y_stride + col] = (uint16_t)(segs.act == kActGeluTanh ? gelu_tanh_bits(out) : out);
                }
            } else {
                partials[((int64_t)slice * M + m) * N + col] = acc[i][v];
            }
        }
    }
}

// Sums the K slices in slice order, rounds to bf16, then adds the bias after the cast. One
// thread per four consecutive columns of a row: 16-byte partial loads when N % 4 == 0, 8-byte
// bf16 stores when y's rows and base are 8-byte aligned as well (`vec`).
__global__ __launch_bounds__(256) void k_skinny_reduce(const float *__restrict__ partials, int splits, int M, int N,
                                                       uint16_t *__restrict__ y, int64_t y_stride,
                                                       const uint16_t *__restrict__ bias, int vec, int act) {
    const int quads = (N + 3) / 4;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t)M * quads) return;
    const int m = (int)(t / quads), col = 4 * (int)(t % quads);
    const int64_t e = (int64_t)m * N + col;
    const bool full = col + 3 < N;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < splits; ++k) {
        const float *p = partials + (int64_t)k * M * N + e;
        if (full && (N & 3) == 0) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(p);
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] += v[c];
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (col + c < N) s[c] += p[c];
        }
    }
    uint32_t out[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        out[c] = float_to_bf16_bits(s[c]);
        if (bias && col + c < N) out[c] = float_to_bf16_bits(bf16_to_float(out[c]) + bf16_to_float(bias[col + c]));
    }
    store_out4(y + (int64_t)m * y_stride, col, N, out, vec, act);
}

int skinny_tiles(int N) { return (N + kSkRows - 1) / kSkRows; }

// K slices: about one workgroup per CU when the weight tiles are few, each slice at least two
// super-blocks.
int skinny_splits(int N, int K) {
    const int tiles = skinny_tiles(N), nsb = K / 256;
    if (tiles >= 160) return 1;
    return std::max(1, std::min(256 / tiles, nsb / 2));
}

}  // namespace

bool skinny_supports(uint32_t type, int M, int N, int K, int64_t x_stride) {
    if (type != kQ4K && type != kQ5K && type != kQ6K) return false;
    if (M < 1 || M > 64 || K % 256 || N < 1) return false;
    const int64_t pitch = (int64_t)(K / 256) * (type == kQ4K ? kQ4KBytes : type == kQ5K ? kQ5KBytes : kQ6KBytes);
    // 32-bit buffer offsets: the activation matrix and one 64-row weight tile.
    return (int64_t)M * x_stride * 2 < (1ll << 31) && (int64_t)kSkRows * pitch < (1ll << 31);
}

int skinny_tile_count(int N) { return skinny_tiles(N); }

int skinny_splits_within(int M, int N, int K, uint64_t capacity) {
    const uint64_t per = (uint64_t)M * (uint64_t)N * sizeof(float);
    const uint64_t fit = per ? capacity / per : 1;
    const int s = (int)std::min<uint64_t>((uint64_t)skinny_splits(N, K), fit);
    return s > 1 ? s : 1;
}

size_t skinny_workspace_bytes(int M, int N, int splits) {
    return splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
}

namespace {
hipError_t launch_skinny_impl(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const Gemv1Segments &segs,
                              int K, int splits, float *partials, hipStream_t stream) {
    const int nsb = K / 256, tiles = segs.tile_begin[segs.count];
    const int64_t pitch = (int64_t)nsb * (type == kQ4K ? kQ4KBytes : type == kQ5K ? kQ5KBytes : kQ6KBytes);
    const dim3 grid((unsigned)(tiles * splits)), block(256);
#define TC_SKINNY(T, R) \
    hipLaunchKernelGGL((k_skinny<T, R>), grid, block, 0, stream, x, x_stride, M, segs, pitch, nsb, tiles, splits, partials)
    if (type == kQ4K) {
        if (M <= 16) TC_SKINNY(kQ4K, 1); else if (M <= 32) TC_SKINNY(kQ4K, 2); else TC_SKINNY(kQ4K, 4);
    } else if (type == kQ5K) {
        if (M <= 16) TC_SKINNY(kQ5K, 1); else if (M <= 32) TC_SKINNY(kQ5K, 2); else TC_SKINNY(kQ5K, 4);
    } else {
        if (M <= 16) TC_SKINNY(kQ6K, 1); else if (M <= 32) TC_SKINNY(kQ6K, 2); else TC_SKINNY(kQ6K, 4);
    }
#undef TC_SKINNY
    return hipGetLastError();
}
}  // namespace

hipError_t launch_skinny(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                         uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, int splits, void *workspace,
                         hipStream_t stream, int act) {
    if (!skinny_supports(type, M, N, K, x_stride)) return hipErrorInvalidValue;
    if (act == kActSiluGlu && (N & 1)) return hipErrorInvalidValue;
    Gemv1Segments segs{};
    segs.count = 1;
    segs.act = act;
    segs.w[0] = w;
    segs.y[0] = y;
    segs.y_stride[0] = y_stride;
    segs.bias[0] = bias_bf16;
    segs.n[0] = N;
    segs.tile_begin[0] = 0;
    segs.tile_begin[1] = skinny_tiles(N);
    if (splits < 1 || (splits > 1 && !workspace)) return hipErrorInvalidValue;
    float *partials = static_cast<float *>(workspace);
    hipError_t e = launch_skinny_impl(type, x, x_stride, M, segs, K, splits, partials, stream);
    if (e != hipSuccess || splits == 1) return e;
    const int64_t quads = (int64_t)M * ((N + 3) / 4);
    // 8-byte stores of 4 outputs (4-byte stores of 2 for kActSiluGlu) when every row allows them.
    const int vec = act == kActSiluGlu ? (y_stride % 2) == 0 && (reinterpret_cast<uintptr_t>(y) & 3u) == 0
                                       : (y_stride % 4) == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0;
    hipLaunchKernelGGL(k_skinny_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, partials,
                       splits, M, N, y, y_stride, bias_bf16, vec, act);
    return hipGetLastError();
}

hipError_t launch_skinny_segments(uint32_t type, const uint16_t *x, int64_t x_stride, int M,
                                  const Gemv1Segments &segs, int K, hipStream_t stream) {
    for (int i = 0; i < segs.count; ++i)
        if (!skinny_supports(type, M, segs.n[i], K, x_stride)) return hipErrorInvalidValue;
    return launch_skinny_impl(type, x, x_stride, M, segs, K, 1, nullptr, stream);
}

}  // namespace tc
