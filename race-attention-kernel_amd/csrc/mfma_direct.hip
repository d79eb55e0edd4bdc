// mfma_direct.hip -- register-direct MFMA kernels for gfx950.
//
// Operands go from global memory straight into MFMA operand registers, with
// no LDS staging: a lane (group g, row lr) of a wave loads, for the 32 tokens
// of a sub-chunk, the 8 rows j = 4 g + r + 16 h (r < 4, h < 2) -- exactly the
// contraction rows that lane supplies in the permuted-k order of
// mfma_common.h -- and, of each 64-column group, the 4 consecutive columns
// 4 lr .. 4 lr + 3.  Column 4 lr + c of a group then feeds MFMA block c at
// row (or column) lr, so the feature index inside a group is permuted as
//     block c, row m  <->  column 4 m + c,
// which the kernels undo when they write results.  One load instruction of a
// wave still covers four whole 256-byte rows, so global reads stay coalesced.
//
// tile_sums_direct_kernel: per-tile totals B_tile = K^T V and A_tile =
// colsum(K) (the K1 of the causal decomposition, src/causal_v2/kernels/
// race_causal_fwd.h:23-27), one wave per tile; tile_sums_quad_kernel: the
// same for fp32 S = d = 64 with four waves per tile.
#include "mfma_common.h"

namespace race {
namespace {

using namespace mfma;

constexpr int kDirC = 32;  // tokens per sub-chunk
// tile_sums_quad_kernel reads the first RACE_SUMS_F32_ALLOC_EIGHTHS eighths
// of each tile (the part the output pass reads first, and K1 last) with the
// cache-allocating policy, the rest `nt`: what the output pass reaches last
// would have left the memory-side cache by then.  Measured at cfg2 (20 steps
// after the settling phase, one box): 6/8 3795 M tokens/s, 8/8 3688, 4/8 3745,
// 2/8 3705 with the same inputs every step; 3476, 3465, 3478, 3442 with two
// input sets alternating.  On another box, three alternating runs each: 6/8
// 3810-3843, 5/8 3763-3791, 7/8 3742-3770.
#ifndef RACE_SUMS_F32_ALLOC_EIGHTHS
#define RACE_SUMS_F32_ALLOC_EIGHTHS 6
#endif

// Eight floats (permuted-k order) to bf16 hi/lo fragments.
template <bool kSplit>
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
    uint2 h0, l0, h1, l1;
    split4<kSplit>(v[0], v[1], v[2], v[3], h0, l0);
    split4<kSplit>(v[4], v[5], v[6], v[7], h1, l1);
    hi = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
    if constexpr (kSplit) lo = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
}

// One sub-chunk of a [tokens][W] tensor in the lane layout above.
template <typename TIn, int W, int P>
struct DRows {
    static constexpr int NG = W / 64;
    f32x4 x[NG][2][4];  // [column group][h][r]: columns 64 gg + 4 lr .. + 3 of row 16 h + 4 g + r

    template <int PP = P>
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int r0, int g, int lr) {
#pragma unroll
        for (int gg = 0; gg < NG; ++gg)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    x[gg][h][r] = load_q4<TIn, PP>(
                        rs, ((r0 + 16 * h + 4 * g + r) * W + 64 * gg + 4 * lr) * int(sizeof(TIn)));
    }
    // The 8 rows of column 64 gg + 4 lr + c, in permuted-k order.
    __device__ __forceinline__ void col(int gg, int c, float (&v)[8]) const {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[4 * h + r] = x[gg][h][r][c];
    }
};

__device__ __forceinline__ bool direct_tile(int64_t total_tiles, int64_t tiles, int w, int64_t* n,
                                            int64_t* ti) {
    const int64_t id = int64_t(blockIdx.x) * 4 + w;
    if (id >= total_tiles) return false;
    *n = id / tiles;
    *ti = id - *n * tiles;
    return true;
}

// ---------------------------------------------------------------------------
// K1: one wave per tile.  Accumulator (sg, sb, dg, cb) holds, at lane
// (g, lr), B[64 sg + 4 (4 g + r) + sb][64 dg + 4 lr + cb], r = 0..3.
template <typename TIn, int S, int D, int kMinBlocks>
__global__ __launch_bounds__(kThreads, kMinBlocks) void tile_sums_direct_kernel(
    const TIn* __restrict__ k, const TIn* __restrict__ v, float* __restrict__ records, int64_t T,
    int tile, int64_t tiles, int64_t rec, int64_t total_tiles) {
    constexpr bool kSplit = std::is_same<TIn, float>::value;
    constexpr int C = kDirC, NSG = S / 64, NDG = D / 64;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, g = l >> 4, lr = l & 15;
    int64_t n, ti;
    if (!direct_tile(total_tiles, tiles, w, &n, &ti)) return;
    const int64_t t_begin = ti * tile;
    const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + (n * T + t_begin) * S, int64_t(rows) * S * sizeof(TIn));
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * sizeof(TIn));

    f32x4 acc[NSG][4][NDG][4];
#pragma unroll
    for (int sg = 0; sg < NSG; ++sg)
#pragma unroll
        for (int sb = 0; sb < 4; ++sb)
#pragma unroll
            for (int dg = 0; dg < NDG; ++dg)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) acc[sg][sb][dg][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float asum[NSG][4];
#pragma unroll
    for (int sg = 0; sg < NSG; ++sg)
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) asum[sg][sb] = 0.f;

    auto chunk = [&](DRows<TIn, S, kSumsLoadPolicy>& kx, DRows<TIn, D, kSumsLoadPolicy>& vx, int r0) {
        bf16x8 vh[NDG][4], vl[NDG][4];
#pragma unroll
        for (int dg = 0; dg < NDG; ++dg)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                float e[8];
                vx.col(dg, cb, e);
                split8<kSplit>(e, vh[dg][cb], vl[dg][cb]);
            }
        // Past the tile the loads read zeros, so the prefetch needs no bound.
        vx.load(vr, r0 + 2 * C, g, lr);
#pragma unroll
        for (int sg = 0; sg < NSG; ++sg)
#pragma unroll
            for (int sb = 0; sb < 4; ++sb) {
                float e[8];
                kx.col(sg, sb, e);
                asum[sg][sb] += (((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7])));
                bf16x8 kh, kl;
                split8<kSplit>(e, kh, kl);
#pragma unroll
                for (int dg = 0; dg < NDG; ++dg)
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb)
                        acc[sg][sb][dg][cb] =
                            mfma3<kSplit>(kh, kl, vh[dg][cb], vl[dg][cb], acc[sg][sb][dg][cb]);
            }
        kx.load(kr, r0 + 2 * C, g, lr);
    };

    DRows<TIn, S, kSumsLoadPolicy> k0, k1;
    DRows<TIn, D, kSumsLoadPolicy> v0, v1;
    k0.load(kr, 0, g, lr);
    v0.load(vr, 0, g, lr);
    k1.load(kr, C, g, lr);
    v1.load(vr, C, g, lr);
    for (int r0 = 0; r0 < rows; r0 += 2 * C) {
        chunk(k0, v0, r0);
        chunk(k1, v1, r0 + C);  // past the tile: zeros, adds nothing
    }

    // B [S][D]: lane writes 4 consecutive columns 64 dg + 4 lr .. + 3 of row
    // 64 sg + 16 g + 4 r + sb.
    float* rp = records + (n * tiles + ti) * rec;
#pragma unroll
    for (int sg = 0; sg < NSG; ++sg)
#pragma unroll
        for (int sb = 0; sb < 4; ++sb)
#pragma unroll
            for (int dg = 0; dg < NDG; ++dg)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const f32x4 x = {acc[sg][sb][dg][0][r], acc[sg][sb][dg][1][r], acc[sg][sb][dg][2][r],
                                     acc[sg][sb][dg][3][r]};
                    *reinterpret_cast<f32x4*>(rp + (64 * sg + 16 * g + 4 * r + sb) * D + 64 * dg + 4 * lr) = x;
                }
    // A [S]: the four token groups g hold partial sums; add them in a fixed order.
#pragma unroll
    for (int sg = 0; sg < NSG; ++sg) {
        f32x4 a;
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            float x = asum[sg][sb];
            x = x + __shfl_xor(x, 16);
            x = x + __shfl_xor(x, 32);
            a[sb] = x;
        }
        if (g == 0) *reinterpret_cast<f32x4*>(rp + S * D + 64 * sg + 4 * lr) = a;
    }
}

// ---------------------------------------------------------------------------
// K1 for fp32 S = d = 64: one workgroup per tile, so the launch spreads over
// every CU (one wave per tile left half of them idle at cfg2).  The tile's
// sub-chunk pairs (64 tokens) are dealt to the four waves round-robin from
// the last pair down: at each step the workgroup reads the 256 tokens below
// the previous step's, so it walks the tile from its end to its start, with
// cache-allocating loads (kSumsF32LoadPolicy).  The start of every tile is
// then what the 256 MB memory-side cache holds most recently when the output
// pass, which walks each tile from its start, begins.  The four partial sums
// meet in LDS and are added in wave order, so the record is the same bit for
// bit on every run.
template <int S, int D>
__global__ __launch_bounds__(kThreads, 2) void tile_sums_quad_kernel(
    const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ records, int64_t T,
    int tile, int64_t tiles, int64_t rec) {
    static_assert(S == 64 && D == 64, "one 64 x 64 block per wave");
    constexpr int C = kDirC, LP = kSumsF32LoadPolicy;
    constexpr int kPart = S * D + S;  // floats of one wave's partial record in LDS
    extern __shared__ __align__(16) float part[];  // [4][kPart]
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, g = l >> 4, lr = l & 15;
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + (n * T + t_begin) * S, int64_t(rows) * S * 4);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * 4);

    f32x4 acc[4][4];  // [sb][cb]: B[4 (4 g + r) + sb][4 lr + cb] at element r
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[sb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float asum[4] = {0.f, 0.f, 0.f, 0.f};

    // Consume the sub-chunk held in (kx, vx), then refill them from row
    // `next` (past the tile the loads read zeros, which are never consumed).
    auto chunk = [&](auto pol, DRows<float, S, LP>& kx, DRows<float, D, LP>& vx, int next) {
        constexpr int PP = decltype(pol)::value;
        bf16x8 vh[4], vl[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            float e[8];
            vx.col(0, cb, e);
            split8<true>(e, vh[cb], vl[cb]);
        }
        vx.template load<PP>(vr, next, g, lr);
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            float e[8];
            kx.col(0, sb, e);
            asum[sb] += (((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7])));
            bf16x8 kh, kl;
            split8<true>(e, kh, kl);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) acc[sb][cb] = mfma3<true>(kh, kl, vh[cb], vl[cb], acc[sb][cb]);
        }
        kx.template load<PP>(kr, next, g, lr);
    };

    // Pair p covers rows 2 C p .. 2 C p + 2 C - 1 (the second half may lie
    // past the tile and read zeros).  Wave w takes pairs P-1-w, P-5-w, ...
    const int pairs = (rows + 2 * C - 1) / (2 * C);
    int p = pairs - 1 - w;
    const int first = p >= 0 ? 2 * C * p : rows;
    // Pairs from `pcut` up are read `nt`, the rest with the allocating policy.
    const int pcut = int((int64_t(pairs) * RACE_SUMS_F32_ALLOC_EIGHTHS + 7) / 8);
    const int cut = 2 * C * pcut;
    DRows<float, S, LP> k0, k1;
    DRows<float, D, LP> v0, v1;
    if (first < cut) {
        k0.load(kr, first, g, lr);
        v0.load(vr, first, g, lr);
        k1.load(kr, first + C, g, lr);
        v1.load(vr, first + C, g, lr);
    } else {
        k0.template load<kPolicyStream>(kr, first, g, lr);
        v0.template load<kPolicyStream>(vr, first, g, lr);
        k1.template load<kPolicyStream>(kr, first + C, g, lr);
        v1.template load<kPolicyStream>(vr, first + C, g, lr);
    }
    using Alloc = std::integral_constant<int, LP>;
    using Stream = std::integral_constant<int, kPolicyStream>;
    for (; p - 4 >= pcut; p -= 4) {
        const int nx = 2 * C * (p - 4);
        chunk(Stream{}, k0, v0, nx);
        chunk(Stream{}, k1, v1, nx + C);
    }
    for (; p >= 0; p -= 4) {
        const int nx = 2 * C * (p - 4);  // below row 0 (last round): outside the range, zeros
        chunk(Alloc{}, k0, v0, nx);
        chunk(Alloc{}, k1, v1, nx + C);
    }

    // Partial record of wave w: B row 16 g + 4 r + sb, columns 4 lr .. + 3,
    // then A (the token groups g added in a fixed order).
    float* mine = part + w * kPart;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<f32x4*>(mine + (16 * g + 4 * r + sb) * D + 4 * lr) =
                f32x4{acc[sb][0][r], acc[sb][1][r], acc[sb][2][r], acc[sb][3][r]};
    {
        f32x4 a;
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            float x = asum[sb];
            x = x + __shfl_xor(x, 16);
            x = x + __shfl_xor(x, 32);
            a[sb] = x;
        }
        if (g == 0) *reinterpret_cast<f32x4*>(mine + S * D + 4 * lr) = a;
    }
    __syncthreads();
    // record = ((part0 + part1) + part2) + part3, 16-byte pieces.
    float* rp = records + (n * tiles + ti) * rec;
    for (int i = threadIdx.x; i < kPart / 4; i += kThreads) {
        f32x4 x = *reinterpret_cast<const f32x4*>(part + 4 * i);
#pragma unroll
        for (int j = 1; j < 4; ++j) x += *reinterpret_cast<const f32x4*>(part + j * kPart + 4 * i);
        *reinterpret_cast<f32x4*>(rp + 4 * i) = x;
    }
}

// ---------------------------------------------------------------------------
// K3: causal output pass for S = d = 64, one wave per tile, every operand in
// registers.  Per sub-chunk of C = 32 tokens the lane (g, lr) loads
//   k1, v1: K / V rows 16 h + 4 g + r, columns 4 lr .. + 3     (k = token order)
//   k2, q2: K / Q rows 16 b + lr, columns 16 g .. 16 g + 15    (rows = tokens)
// and the products are (M x N, contraction):
//   1. Abar^T = A0 + K^T tril(1)  (bucket block sb: s = 4 m + sb) x (token i), over j
//      -> lane holds Abar[16 bi + lr][16 g + 4 r + sb]; Q is loaded at the same spots
//   2. W = Q / (Abar + eps) in registers, at the same spots
//   3. P^T = K W^T  (token j) x (token i), over s in the order s = 16 g + 8 kk + e,
//      masked j > i -> lane holds P^T[16 bj + 4 g + r][16 bi + lr]
//   4. O^T = B0^T W^T + V^T P^T  (column block cb: c = 4 m + cb) x (token i)
//      -> lane holds O[16 bi + lr][16 g + 4 r + cb]: 16 consecutive columns
//   5. B0 += K^T V  (s block sb) x (c block cb) over j
//      -> lane holds B0[16 g + 4 r + sb][4 lr + cb], which is the A operand of
//         step 4 for s = 16 g + 8 kk + e without any data movement.
template <typename TIn>
struct DStage {
    f32x4 k1[2][4], v1[2][4];  // [h][r]
    f32x4 k2[2][4], q2[2][4];  // [row block][u]: columns 16 g + 4 u .. + 3

    __device__ __forceinline__ void load_kv(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                            int r0, int g, int lr) {
        constexpr int es = int(sizeof(TIn));
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = r0 + 16 * h + 4 * g + r;
                k1[h][r] = load_q4<TIn, kPolicyDefault>(kr, (row * 64 + 4 * lr) * es);
                v1[h][r] = load_q4<TIn, kOutKVPolicy>(vr, (row * 64 + 4 * lr) * es);
            }
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int u = 0; u < 4; ++u) k2[b][u] = load_q4<TIn, kPolicyDefault>(kr, ((r0 + 16 * b + lr) * 64 + 16 * g + 4 * u) * es);
    }
    __device__ __forceinline__ void load_q(__amdgpu_buffer_rsrc_t qr, int r0, int g, int lr) {
        constexpr int es = int(sizeof(TIn));
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int u = 0; u < 4; ++u) q2[b][u] = load_q4<TIn, kOutQPolicy>(qr, ((r0 + 16 * b + lr) * 64 + 16 * g + 4 * u) * es);
    }
};

// Two consecutive output values at byte offset `off` of a buffer.
template <typename TIn>
__device__ __forceinline__ void store2(__amdgpu_buffer_rsrc_t r, int off, float x0, float x1) {
    if constexpr (std::is_same<TIn, float>::value) {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(x0), __float_as_uint(x1)}, r, off, 0, kOutStorePolicy);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32(pack2(x0, x1), r, off, 0, kOutStorePolicy);
    }
}

template <typename TIn, int kMinBlocks>
__global__ __launch_bounds__(kThreads, kMinBlocks) void causal_output_direct_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    TIn* __restrict__ out, const float* __restrict__ records, int64_t T, int tile, int64_t tiles,
    int64_t rec, int64_t total_tiles) {
    constexpr bool kSplit = std::is_same<TIn, float>::value;
    constexpr int C = kDirC, S = 64, D = 64;
    constexpr int es = int(sizeof(TIn));
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, g = l >> 4, lr = l & 15;
    int64_t n, ti;
    if (!direct_tile(total_tiles, tiles, w, &n, &ti)) return;
    const int64_t t_begin = ti * tile;
    const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + (n * T + t_begin) * S, int64_t(rows) * S * es);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + (n * T + t_begin) * S, int64_t(rows) * S * es);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * es);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(out + (n * T + t_begin) * D, int64_t(rows) * D * es);

    // Carried state from the tile's exclusive prefix record.
    const float* rp = records + (n * tiles + ti) * rec;
    f32x4 b0[4][4];  // [sb][cb]: B0[16 g + 4 r + sb][4 lr + cb]
    f32x4 a0[4];     // [sb]:     A0[16 g + 4 r + sb]
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(rp + (16 * g + 4 * r + sb) * D + 4 * lr);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) b0[sb][cb][r] = x[cb];
            a0[sb][r] = rp[S * D + 16 * g + 4 * r + sb];
        }
    }
    const bf16x8 tri0 = tril_frag(0, g, lr), tri1 = tril_frag(16, g, lr);

    // The raw registers of a sub-chunk are loaded at the end of the previous
    // one; two resident waves per SIMD cover each other's load latency.
    DStage<TIn> st;
    st.load_kv(kr, vr, 0, g, lr);
    st.load_q(qr, 0, g, lr);
    for (int r0 = 0; r0 < rows; r0 += C) {
        // 1 + 2: running mass and W (lane: W[16 bi + lr][16 g + 4 r + sb] = wv[bi][sb][r]).
        bf16x8 kh[4], kl[4];
        f32x4 wv[2][4];
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            float e[8];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) e[4 * h + r] = st.k1[h][r][sb];
            split8<kSplit>(e, kh[sb], kl[sb]);
            f32x4 m0 = a0[sb], m1 = a0[sb];
            if constexpr (kSplit) {
                m0 = mfma16(kl[sb], tri0, m0);
                m1 = mfma16(kl[sb], tri1, m1);
            }
            m0 = mfma16(kh[sb], tri0, m0);
            m1 = mfma16(kh[sb], tri1, m1);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                wv[0][sb][r] = st.q2[0][r][sb] * __builtin_amdgcn_rcpf(m0[r] + kEps);
                wv[1][sb][r] = st.q2[1][r][sb] * __builtin_amdgcn_rcpf(m1[r] + kEps);
                // Inclusive mass at the sub-chunk's last row (rows past the tile are zero).
                a0[sb][r] = __shfl(m1[r], 16 * g + 15);
            }
        }
        // W fragments over s = 16 g + 8 kk + e: e < 4 -> (r = 2 kk, sb = e), else (r = 2 kk + 1, sb = e - 4).
        bf16x8 wh[2][2], wl[2][2];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const float e[8] = {wv[bi][0][2 * kk], wv[bi][1][2 * kk], wv[bi][2][2 * kk], wv[bi][3][2 * kk],
                                    wv[bi][0][2 * kk + 1], wv[bi][1][2 * kk + 1], wv[bi][2][2 * kk + 1],
                                    wv[bi][3][2 * kk + 1]};
                split8<kSplit>(e, wh[bi][kk], wl[bi][kk]);
            }

        // 3: P^T blocks (j-block, i-block) = (0,0), (0,1), (1,1).
        f32x4 p00 = {0.f, 0.f, 0.f, 0.f}, p01 = p00, p11 = p00;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8 a0h, a0l, a1h, a1l;
            {
                const f32x4 x0 = st.k2[0][2 * kk], x1 = st.k2[0][2 * kk + 1];
                const float e[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                split8<kSplit>(e, a0h, a0l);
            }
            {
                const f32x4 x0 = st.k2[1][2 * kk], x1 = st.k2[1][2 * kk + 1];
                const float e[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                split8<kSplit>(e, a1h, a1l);
            }
            p00 = mfma3<kSplit>(a0h, a0l, wh[0][kk], wl[0][kk], p00);
            p01 = mfma3<kSplit>(a0h, a0l, wh[1][kk], wl[1][kk], p01);
            p11 = mfma3<kSplit>(a1h, a1l, wh[1][kk], wl[1][kk], p11);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r > lr) {
                p00[r] = 0.f;
                p11[r] = 0.f;
            }
        // P^T as the B operand over j in permuted order: e < 4 -> block 0, else block 1.
        bf16x8 ph[2], pl[2];
        {
            const float e0[8] = {p00[0], p00[1], p00[2], p00[3], 0.f, 0.f, 0.f, 0.f};
            split8<kSplit>(e0, ph[0], pl[0]);
            const float e1[8] = {p01[0], p01[1], p01[2], p01[3], p11[0], p11[1], p11[2], p11[3]};
            split8<kSplit>(e1, ph[1], pl[1]);
        }

        // 4 + 5 per pair of column blocks: O^T = B0^T W^T + V^T P^T, then B0 += K^T V.
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            f32x4 o[2][2];
            bf16x8 vh[2], vl[2];
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int cb = 2 * half + cc;
                float e[8];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) e[4 * h + r] = st.v1[h][r][cb];
                split8<kSplit>(e, vh[cc], vl[cc]);
                o[cc][0] = f32x4{0.f, 0.f, 0.f, 0.f};
                o[cc][1] = o[cc][0];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const float b[8] = {b0[0][cb][2 * kk], b0[1][cb][2 * kk], b0[2][cb][2 * kk], b0[3][cb][2 * kk],
                                        b0[0][cb][2 * kk + 1], b0[1][cb][2 * kk + 1], b0[2][cb][2 * kk + 1],
                                        b0[3][cb][2 * kk + 1]};
                    bf16x8 bh, bl;
                    split8<kSplit>(b, bh, bl);
                    o[cc][0] = mfma3<kSplit>(bh, bl, wh[0][kk], wl[0][kk], o[cc][0]);
                    o[cc][1] = mfma3<kSplit>(bh, bl, wh[1][kk], wl[1][kk], o[cc][1]);
                }
                o[cc][0] = mfma3<kSplit>(vh[cc], vl[cc], ph[0], pl[0], o[cc][0]);
                o[cc][1] = mfma3<kSplit>(vh[cc], vl[cc], ph[1], pl[1], o[cc][1]);
            }
            // Lane holds O[16 bi + lr][16 g + 4 r + cb]; this half writes cb = 2 half, 2 half + 1.
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    store2<TIn>(orr, ((r0 + 16 * bi + lr) * D + 16 * g + 4 * r + 2 * half) * es,
                                o[0][bi][r], o[1][bi][r]);
#pragma unroll
            for (int sb = 0; sb < 4; ++sb)
#pragma unroll
                for (int cc = 0; cc < 2; ++cc)
                    b0[sb][2 * half + cc] =
                        mfma3<kSplit>(kh[sb], kl[sb], vh[cc], vl[cc], b0[sb][2 * half + cc]);
        }
        // Next sub-chunk (past the tile the loads read zeros and stores are dropped).
        st.load_kv(kr, vr, r0 + C, g, lr);
        st.load_q(qr, r0 + C, g, lr);
    }
}


}  // namespace

bool direct_sums_supported(int S, int d) {
    return (S == 64 && (d == 64 || d == 128)) || (S == 128 && d == 64);
}

hipError_t launch_tile_sums_direct(const void* k, const void* v, float* records, const Problem& p,
                                   hipStream_t stream) {
    if (p.tile % (2 * kDirC) != 0) return hipErrorInvalidValue;
    if (p.dtype == RACE_F32 && p.S == 64 && p.d == 64) {
        constexpr size_t kLds = 4 * (64 * 64 + 64) * sizeof(float);
        tile_sums_quad_kernel<64, 64><<<dim3(unsigned(p.tiles), unsigned(p.N)), kThreads, kLds, stream>>>(
            static_cast<const float*>(k), static_cast<const float*>(v), records, p.T, p.tile, p.tiles, p.rec);
        return hipGetLastError();
    }
    const int64_t total = p.N * p.tiles;
    const dim3 grid(unsigned((total + 3) / 4));
#define RACE_SUMS(TIN, S_, D_, MB)                                                                 \
    tile_sums_direct_kernel<TIN, S_, D_, MB><<<grid, kThreads, 0, stream>>>(                       \
        static_cast<const TIN*>(k), static_cast<const TIN*>(v), records, p.T, p.tile, p.tiles, p.rec, \
        total)
    if (p.dtype == RACE_F32) {
        if (p.S == 64 && p.d == 64) RACE_SUMS(float, 64, 64, 1);
        else if (p.S == 64 && p.d == 128) RACE_SUMS(float, 64, 128, 1);
        else if (p.S == 128 && p.d == 64) RACE_SUMS(float, 128, 64, 1);
        else return hipErrorInvalidValue;
    } else {
        if (p.S == 64 && p.d == 64) RACE_SUMS(bf16_t, 64, 64, 1);
        else if (p.S == 64 && p.d == 128) RACE_SUMS(bf16_t, 64, 128, 1);
        else if (p.S == 128 && p.d == 64) RACE_SUMS(bf16_t, 128, 64, 1);
        else return hipErrorInvalidValue;
    }
#undef RACE_SUMS
    return hipGetLastError();
}


bool direct_output_supported(int S, int d, int dtype) {
    // fp32 operands need three products per contraction and more registers than
    // two waves per SIMD allow; the LDS-staged workgroup kernel is faster there.
    return S == 64 && d == 64 && dtype == RACE_BF16;
}

// Four tiles per compute unit (one wave per SIMD): measured faster at cfg3
// than eight (1.15 against 1.21 ms), with half the tile records.
int direct_output_tiles_per_cu() { return 4; }

hipError_t launch_causal_output_direct(const void* q, const void* k, const void* v, void* out,
                                       const float* records, const Problem& p, hipStream_t stream) {
    if (p.S != 64 || p.d != 64 || p.tile % kDirC != 0) return hipErrorInvalidValue;
    const int64_t total = p.N * p.tiles;
    const dim3 grid(unsigned((total + 3) / 4));
    if (p.dtype != RACE_BF16) return hipErrorInvalidValue;
    causal_output_direct_kernel<bf16_t, 2><<<grid, kThreads, 0, stream>>>(
        static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k), static_cast<const bf16_t*>(v),
        static_cast<bf16_t*>(out), records, p.T, p.tile, p.tiles, p.rec, total);
    return hipGetLastError();
}

}  // namespace race
