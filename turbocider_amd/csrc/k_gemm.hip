// Dispatch of the fused K-quant dequant + bf16 MFMA GEMM (kernel: k_gemm_impl.h, compiled
// per variant from k_gemm_variant.hip): row-block count MT by M, split-K for grids with few
// output tiles, persistent grid size, and the deterministic split-K reduction.
//
// Replaces the reference's Metal quantized matmul (mx::quantized_matmul affine QMM,
// native/backends/mlx.cpp:678-679, and affine_gpu::projection_shared,
// native/backends/affine_gpu_shared.hpp:41-84).
#include "k_gemm.h"
#include "tc_device.h"
#include "tc_kernels.h"

#include <algorithm>
#include <atomic>

namespace tc {
namespace {

constexpr int kBN = 256;

// 32-row blocks per workgroup tile: 1 (M <= 32), 2 (M <= 64); 4 (128-row tiles) when 256-row
// tiles would leave the grid short of output tiles, for up to 512 rows at any K and up to 1024
// rows with K <= 8192 (measured at M = 256: N = K = 3584 32.5 -> 23.8 us; M = 1024,
// N = K = 3072 49 -> 42 us; with the 4-deep slice loads of the reduction, the M = 256 down
// projections at K = 12288 and 18944 are faster on 128-row tiles with fewer K slices: config 2
// block at M = 256 0.2934 -> 0.2906 ms, config 3 block (grouped streams) 0.448 -> 0.432 ms);
// else 8.
int gemm_mt(int M, int N, int K) {
    if (M <= 32) return 1;
    if (M <= 64) return 2;
    const int tiles8 = ((M + 255) / 256) * ((N + kBN - 1) / kBN);
    return (M <= 1024 && (K <= 8192 || M <= 512) && tiles8 < 160) ? 4 : 8;
}

// Sums the K slices of a split GEMM in slice order (a fixed order), rounds to bf16 and adds
// the bias after the cast (as the unsplit epilogue does). One thread per eight consecutive
// accumulator values of the kernel's MFMA-native partials layout (tile, wavefront, value
// v < 32 MT, lane): lanes 8q .. 8q + 7 hold the same output row and eight consecutive
// columns, so each slice is two 16-byte loads and the eight outputs one 16-byte store
// (`vec16`: y rows and base 16-byte aligned, no gated activation; otherwise two stores of
// four, 8-byte with `vec`, element stores at the N edge). The slices' loads are issued four
// slices at a time and added in slice order. Partial loads and the 16-byte output stores are
// non-temporal: each partial is read exactly once, and neither stream should displace the
// lines the next launch reuses. A launch reduces one problem, or both of a
// grouped launch: workgroups [0, p0.blocks) take p0, the rest p1. A part's tiles start `base`
// floats into each slice, and slices are `slice_stride` floats apart (a grouped launch's
// slices hold the tiles of both problems).
struct ReducePart {
    int64_t base;
    int tiles_m, tiles_n, M, N;
    uint16_t *y;
    int64_t y_stride;
    const uint16_t *bias;
    int vec, vec16, blocks;
};

__global__ __launch_bounds__(256) void k_splitk_reduce(const float *__restrict__ partials, int64_t slice_stride,
                                                       int splits, int mt, int act, ReducePart p0, ReducePart p1) {
    const bool second = (int)blockIdx.x >= p0.blocks;  // uniform per workgroup
    const int tiles_m = second ? p1.tiles_m : p0.tiles_m, tiles_n = second ? p1.tiles_n : p0.tiles_n;
    const int M = second ? p1.M : p0.M, N = second ? p1.N : p0.N;
    const int ntiles = tiles_m * tiles_n, vpl = 32 * mt;
    const int64_t per_part = (int64_t)ntiles * 4 * vpl * 64;
    const int64_t e = 8 * ((int64_t)((int)blockIdx.x - (second ? p0.blocks : 0)) * 256 + threadIdx.x);
    if (e >= per_part) return;
    const float *src = partials + (second ? p1.base : p0.base) + e;
    const int lane = (int)(e & 63);
    const int64_t q = e >> 6;
    const int v = (int)(q % vpl), wave = (int)((q / vpl) & 3), tile = (int)(q / vpl / 4);
    const int tm = tile / tiles_n, tn = tile % tiles_n;
    const int i = v >> 5, t = (v >> 4) & 1, j = v & 15, l32 = lane & 31, hh = lane >> 5;
    const int m = tm * 32 * mt + 32 * i + 8 * (j >> 2) + 4 * hh + (j & 3), n = tn * kBN + 64 * wave + 32 * t + l32;
    if (m >= M || n >= N) return;
    struct Oct {
        f32x4 lo, hi;
    };
    auto slice = [&](int k) {
        const float *p = src + (int64_t)k * slice_stride;
        return Oct{__builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p)),
                   __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p + 4))};
    };
    auto add = [](Oct &acc, const Oct &p) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            acc.lo[c] += p.lo[c];
            acc.hi[c] += p.hi[c];
        }
    };
    Oct s = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    int k = 0;
    for (; k + 4 <= splits; k += 4) {
        const Oct a = slice(k), b = slice(k + 1), c = slice(k + 2), d = slice(k + 3);
        add(s, a);
        add(s, b);
        add(s, c);
        add(s, d);
    }
    for (; k < splits; ++k) add(s, slice(k));
    const uint16_t *bias = second ? p1.bias : p0.bias;
    uint32_t out[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        out[c] = float_to_bf16_bits(c < 4 ? s.lo[c] : s.hi[c - 4]);
        if (bias && n + c < N) out[c] = float_to_bf16_bits(bf16_to_float(out[c]) + bf16_to_float(bias[n + c]));
    }
    uint16_t *yrow = (second ? p1.y : p0.y) + (int64_t)m * (second ? p1.y_stride : p0.y_stride);
    if ((second ? p1.vec16 : p0.vec16) && act != kActSiluGlu && n + 7 < N) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
            if (act == kActGeluTanh) out[c] = gelu_tanh_bits(out[c]);
        __builtin_nontemporal_store(
            u32x4{out[0] | (out[1] << 16), out[2] | (out[3] << 16), out[4] | (out[5] << 16), out[6] | (out[7] << 16)},
            reinterpret_cast<u32x4 *>(yrow + n));
    } else {
        const int vec = second ? p1.vec : p0.vec;
        store_out4(yrow, n, N, out, vec, act);
        store_out4(yrow, n + 4, N, out + 4, vec, act);
    }
}

// Workgroups per CU the persistent grid aims for: one for the large tile (one wavefront per
// SIMD, 256 accumulators per lane); for the skinny tiles, whose chunks are short, more, so
// that other workgroups' chunks cover the memory latency (measured best: two for 64-row
// tiles, four for 32-row tiles; more K slices also cost fp32 partial-sum traffic).
int gemm_occupancy(int mt) { return mt >= 4 ? 1 : mt == 2 ? 2 : 4; }

// One part of a slice reduction: a problem's tiles, `base` floats into each slice.
ReducePart reduce_part(int64_t base, int tiles_m, int tiles_n, int mt, int M, int N, uint16_t *y, int64_t y_stride,
                       const uint16_t *bias, int act) {
    ReducePart r;
    r.base = base;
    r.tiles_m = tiles_m;
    r.tiles_n = tiles_n;
    r.M = M;
    r.N = N;
    r.y = y;
    r.y_stride = y_stride;
    r.bias = bias;
    // 8-byte stores of 4 outputs (4-byte stores of 2 for kActSiluGlu) when every row allows them.
    r.vec = act == kActSiluGlu ? (y_stride % 2) == 0 && (reinterpret_cast<uintptr_t>(y) & 3u) == 0
                               : (y_stride % 4) == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0;
    r.vec16 = (y_stride % 8) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    const int64_t octets = (int64_t)tiles_m * tiles_n * 4 * (32 * mt) * 64 / 8;
    r.blocks = (int)((octets + 255) / 256);
    return r;
}

// The slice reduction (k_splitk_reduce) of one part, or of two in one launch.
hipError_t launch_reduce(const float *partials, int64_t slice_stride, int splits, int mt, int act, const ReducePart &p0,
                         const ReducePart *p1, hipStream_t stream) {
    ReducePart second{};
    if (p1) second = *p1;
    hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)(p0.blocks + (p1 ? p1->blocks : 0))), dim3(256), 0, stream,
                       partials, slice_stride, splits, mt, act, p0, second);
    return hipGetLastError();
}

int gemm_tiles(int M, int N, int K) {
    const int bm = 32 * gemm_mt(M, N, K);
    return ((M + bm - 1) / bm) * ((N + kBN - 1) / kBN);
}

// K slices for a grid of output tiles: enough to give about one (large tile) or two (skinny
// tiles) workgroups per CU, each slice at least two (large tile) or one super-block; 1 = no
// split.
int gemm_splits(int M, int N, int K) {
    const int mt = gemm_mt(M, N, K), occ = gemm_occupancy(mt), tiles = gemm_tiles(M, N, K), nsb = K / 256;
    if (mt >= 4) {
        if (tiles >= 160 || nsb < 4) return 1;
        return std::max(1, std::min(nsb / 2, 256 / tiles));
    }
    // Skinny tiles: slices of at least one super-block, up to `occ` workgroups per CU.
    if (tiles >= 160 * occ || nsb < 2) return 1;
    return std::max(1, std::min(nsb, 256 * occ / tiles));
}

// Compute units of the current device (the persistent grid size), queried once per device.
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace

int gemm_tail_rows(int M, int N, int K) {
    (void)K;
    const int rem = M % 256, full = M / 256;
    if (full < 1 || rem < 1 || rem > 64) return 0;
    const int tn = (N + kBN - 1) / kBN, cus = cu_count();
    if (gemm_mt(M - rem, N, K) != 8 || full * tn < 160) return 0;
    const int rounds_full = (full * tn + cus - 1) / cus, rounds_all = ((full + 1) * tn + cus - 1) / cus;
    return rounds_all > rounds_full ? rem : 0;
}

bool gemm_supports(int K, int64_t x_stride) { return 2 * (255 * x_stride + (int64_t)K) < (1ll << 31); }

// fp32 partials of one K slice: every tile's 4 wavefronts x 32 MT accumulator rows x 64 lanes.
static uint64_t gemm_slice_bytes(int M, int N, int K) {
    return (uint64_t)gemm_tiles(M, N, K) * 4 * (32 * gemm_mt(M, N, K)) * 64 * sizeof(float);
}

int gemm_splits_within(int M, int N, int K, uint64_t capacity) {
    const int s = (int)std::min<uint64_t>((uint64_t)gemm_splits(M, N, K), capacity / gemm_slice_bytes(M, N, K));
    return s > 1 ? s : 1;
}

size_t gemm_workspace_bytes(int M, int N, int K, int splits) {
    return splits > 1 ? (size_t)splits * gemm_slice_bytes(M, N, K) : 0;
}

hipError_t launch_gemm(uint32_t type, const uint16_t *x, int64_t x_stride, int M, const uint8_t *w, int N, int K,
                       uint16_t *y, int64_t y_stride, const uint16_t *bias_bf16, int splits, void *workspace,
                       hipStream_t stream, int act) {
    if (splits < 1 || (splits > 1 && !workspace)) return hipErrorInvalidValue;
    if (act == kActSiluGlu && (N & 1)) return hipErrorInvalidValue;
    const bool keep = act == kActNoneKeep;
    if (keep) act = kActNone;
    const int mt = gemm_mt(M, N, K), bm = 32 * mt;
    GemmArgs a;
    a.x = x;
    a.x_stride = x_stride;
    a.M = M;
    a.w = w;
    a.w_pitch = (int64_t)(K / 256) * (type == kQ4K ? kQ4KBytes : type == kQ5K ? kQ5KBytes : kQ6KBytes);
    a.N = N;
    a.K = K;
    a.y = y;
    a.y_stride = y_stride;
    a.tiles_m = (M + bm - 1) / bm;
    a.tiles_n = (N + kBN - 1) / kBN;
    a.splits = splits;
    a.partials = static_cast<float *>(workspace);
    a.act = act;
    const bool split = a.splits > 1;
    a.bias = split ? nullptr : bias_bf16;
    const int items = a.tiles_m * a.tiles_n * a.splits;
    a.grid = std::min(items, cu_count() * gemm_occupancy(mt));
    hipError_t e;
#define TC_GEMM_CALL(T, MT)                                                                      \
    (split                    ? TC_GEMM_VARIANT_NAME(T, 1, MT, 0)(a, stream)                     \
        : act == kActGeluTanh ? TC_GEMM_VARIANT_NAME(T, 0, MT, 1)(a, stream)                     \
        : act == kActSiluGlu  ? TC_GEMM_VARIANT_NAME(T, 0, MT, 2)(a, stream)                     \
                              : TC_GEMM_VARIANT_NAME(T, 0, MT, 0)(a, stream))
#define TC_GEMM_PICK(T, MT) e = TC_GEMM_CALL(T, MT)
#define TC_GEMM_PICK_KEEP(T, MT) e = !split && keep ? TC_GEMM_VARIANT_NAME(T, 0, MT, 3)(a, stream) : TC_GEMM_CALL(T, MT)
    if (type == kQ4K) {
        if (mt == 1) TC_GEMM_PICK(12, 1); else if (mt == 2) TC_GEMM_PICK(12, 2);
        else if (mt == 4) TC_GEMM_PICK_KEEP(12, 4); else TC_GEMM_PICK_KEEP(12, 8);
    } else if (type == kQ5K) {
        if (mt == 1) TC_GEMM_PICK(13, 1); else if (mt == 2) TC_GEMM_PICK(13, 2);
        else if (mt == 4) TC_GEMM_PICK_KEEP(13, 4); else TC_GEMM_PICK_KEEP(13, 8);
    } else {
        if (mt == 1) TC_GEMM_PICK(14, 1); else if (mt == 2) TC_GEMM_PICK(14, 2);
        else if (mt == 4) TC_GEMM_PICK_KEEP(14, 4); else TC_GEMM_PICK_KEEP(14, 8);
    }
#undef TC_GEMM_PICK_KEEP
#undef TC_GEMM_PICK
#undef TC_GEMM_CALL
    if (e != hipSuccess || !split) return e;
    const int64_t per_slice = (int64_t)a.tiles_m * a.tiles_n * 4 * bm * 64;
    return launch_reduce(a.partials, per_slice, a.splits, mt, act,
                         reduce_part(0, a.tiles_m, a.tiles_n, mt, M, N, y, y_stride, bias_bf16, act), nullptr, stream);
}

namespace {
// Row-block count and K slices of a grouped launch: the single-problem rules applied to the
// two problems' tiles together.
struct GroupGeometry {
    int mt, tiles_m0, tiles_n0, tiles_m1, tiles_n1, splits;
    int tiles() const { return tiles_m0 * tiles_n0 + tiles_m1 * tiles_n1; }
};
GroupGeometry group_geometry(int M0, int N0, int M1, int N1, int K) {
    GroupGeometry g;
    g.tiles_n0 = (N0 + kBN - 1) / kBN;
    g.tiles_n1 = (N1 + kBN - 1) / kBN;
    const int tiles8 = (M0 + 255) / 256 * g.tiles_n0 + (M1 + 255) / 256 * g.tiles_n1;
    const int mmax = std::max(M0, M1);
    g.mt = (mmax <= 1024 && (K <= 8192 || mmax <= 512) && tiles8 < 160) ? 4 : 8;
    const int bm = 32 * g.mt, nsb = K / 256;
    g.tiles_m0 = (M0 + bm - 1) / bm;
    g.tiles_m1 = (M1 + bm - 1) / bm;
    const int tiles = g.tiles();
    g.splits = (tiles >= 160 || nsb < 4) ? 1 : std::max(1, std::min(nsb / 2, 256 / tiles));
    return g;
}
uint64_t group_slice_bytes(const GroupGeometry &g) { return (uint64_t)g.tiles() * 4 * (32 * g.mt) * 64 * sizeof(float); }
}  // namespace

bool gemm_group_supports(int M0, int M1, int K, int64_t x_stride) {
    return M0 >= 65 && M1 >= 65 && gemm_supports(K, x_stride);
}

int gemm_group_splits_within(int M0, int N0, int M1, int N1, int K, uint64_t capacity) {
    const GroupGeometry g = group_geometry(M0, N0, M1, N1, K);
    const int s = (int)std::min<uint64_t>((uint64_t)g.splits, capacity / group_slice_bytes(g));
    return s > 1 ? s : 1;
}

size_t gemm_group_workspace_bytes(int M0, int N0, int M1, int N1, int K, int splits) {
    return splits > 1 ? (size_t)splits * group_slice_bytes(group_geometry(M0, N0, M1, N1, K)) : 0;
}

hipError_t launch_gemm_group(uint32_t type, const uint16_t *const x[2], int64_t x_stride, const int M[2],
                             const uint8_t *const w[2], const int N[2], int K, uint16_t *const y[2],
                             const int64_t y_stride[2], const uint16_t *const bias_bf16[2], int splits,
                             void *workspace, hipStream_t stream, int act) {
    if (splits < 1 || (splits > 1 && !workspace)) return hipErrorInvalidValue;
    if (act != kActNone && splits == 1) return hipErrorInvalidValue;  // only the reduction applies it
    if (act == kActSiluGlu && ((N[0] & 1) || (N[1] & 1))) return hipErrorInvalidValue;
    if (!gemm_group_supports(M[0], M[1], K, x_stride)) return hipErrorInvalidValue;
    const GroupGeometry g = group_geometry(M[0], N[0], M[1], N[1], K);
    const bool split = splits > 1;
    GemmArgs a;
    a.x = x[0];
    a.x_stride = x_stride;
    a.M = M[0];
    a.w = w[0];
    a.w_pitch = (int64_t)(K / 256) * (type == kQ4K ? kQ4KBytes : type == kQ5K ? kQ5KBytes : kQ6KBytes);
    a.N = N[0];
    a.K = K;
    a.y = y[0];
    a.y_stride = y_stride[0];
    a.bias = split ? nullptr : bias_bf16[0];
    a.tiles_m = g.tiles_m0;
    a.tiles_n = g.tiles_n0;
    a.splits = splits;
    a.partials = static_cast<float *>(workspace);
    a.act = kActNone;
    a.grid = std::min(g.tiles() * splits, cu_count());
    GemmSecond b;
    b.x = x[1];
    b.M = M[1];
    b.w = w[1];
    b.N = N[1];
    b.y = y[1];
    b.y_stride = y_stride[1];
    b.bias = split ? nullptr : bias_bf16[1];
    b.tiles_m = g.tiles_m1;
    b.tiles_n = g.tiles_n1;
    hipError_t e;
#define TC_GEMMG_PICK(T)                                                                          \
    e = g.mt == 4 ? (split ? TC_GEMMG_VARIANT_NAME(T, 1, 4)(a, b, stream) : TC_GEMMG_VARIANT_NAME(T, 0, 4)(a, b, stream)) \
                  : (split ? TC_GEMMG_VARIANT_NAME(T, 1, 8)(a, b, stream) : TC_GEMMG_VARIANT_NAME(T, 0, 8)(a, b, stream))
    if (type == kQ4K) TC_GEMMG_PICK(12);
    else if (type == kQ5K) TC_GEMMG_PICK(13);
    else TC_GEMMG_PICK(14);
#undef TC_GEMMG_PICK
    if (e != hipSuccess || !split) return e;
    const int bm = 32 * g.mt;
    const int64_t stride = (int64_t)g.tiles() * 4 * bm * 64, base1 = (int64_t)g.tiles_m0 * g.tiles_n0 * 4 * bm * 64;
    const ReducePart r1 =
        reduce_part(base1, g.tiles_m1, g.tiles_n1, g.mt, M[1], N[1], y[1], y_stride[1], bias_bf16[1], act);
    return launch_reduce(a.partials, stride, splits, g.mt, act,
                         reduce_part(0, g.tiles_m0, g.tiles_n0, g.mt, M[0], N[0], y[0], y_stride[0], bias_bf16[0], act),
                         &r1, stream);
}

}  // namespace tc
