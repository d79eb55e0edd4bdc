// hashed_kernels.h -- the causal per-bucket op with the hashing inside, on
// gfx950 matrix cores: BatchedACE.forward's lines 41-51
// (src/race_baseline.py) in three launches, and the fused forward of
// src/race_fused_fwd.cu:80-146, which hashes the Q and K rows in the same pass
// as the state update and the blend.  The bucket probabilities never go
// through HBM: each kernel hashes the token rows it needs (hash_stage.h) into
// the same LDS plane tiles the probability-input kernels (mfma_causal.hip)
// stage from memory, and from there the contractions are theirs:
//   1. hashed_sums_kernel   per (tile, stream): Phi_K of the tile's key rows,
//                           B_tile = Phi_K^T V, A_tile = colsum Phi_K
//   2. tile_scan_kernel     exclusive scan of the tile records
//   3. hashed_output_kernel per (tile, stream): per sub-chunk of C tokens,
//                             Phi_K (plane tile), Phi_Q (read from the plane
//                             values as the query-side weights are formed),
//                             Abar = A0 + tril(1) Phi_K, W = Phi_Q / (Abar + eps),
//                             O = W B0 + tril(W Phi_K^T) V,
//                             A0 += colsum Phi_K, B0 += Phi_K^T V.
// Per stream-token the kernels read the Q, K and V rows (3 D values) and
// write the output row (D values), against 2 S + 2 D for the probability
// inputs: at S = D the same bytes, and the hashing's own round trip through
// HBM (writing and re-reading S values per token for each of Q and K) is
// gone.  The kernels are templates on the planes per table KP (so every loop
// over planes, tables and corners unrolls); hashed_causal.hip and
// hashed_causal_bf16.hip instantiate them for fp32 and bf16 rows.
#pragma once

#include "causal_geo.h"
#include "hash_stage.h"

#ifndef RACE_HASHED_SUMS_ALLOC_EIGHTHS
#define RACE_HASHED_SUMS_ALLOC_EIGHTHS 6
#endif
// Resident fp32 tile-sum workgroups per CU (S = d = 64, the lean layout):
// the automatic 1024-token tiles start two per CU at cfg2, and the
// end-to-start walk spills at the four-per-CU register bound.
#ifndef RACE_HASHED_SUMS_F32_BLOCKS
#define RACE_HASHED_SUMS_F32_BLOCKS 2
#endif

namespace race {
namespace hashed {

using namespace mfma;

// Planes per table KP fixes the tables L = S / 2^KP of an (S, KP) kernel and
// the 16-plane blocks its projection needs.
constexpr int tables_of(int S, int KP) { return S >> KP; }
constexpr int npb_of(int S, int KP) { return ((S >> KP) * KP + 15) / 16; }
// Whether (S, KP) is a shape the hashed kernels take: 2 <= KP, L >= 1,
// L * KP <= 64.
constexpr bool kp_ok(int S, int KP) { return KP >= 2 && (S >> KP) >= 1 && (S >> KP) * KP <= 64; }

// Token rows [C][Wd] of one sub-chunk in registers (blocks of kRows rows x
// one 16-byte vector, kRows = 4, 2 or 1: the most that still gives every one
// of the NT threads a block), then stored as a plane tile.  The V part of
// KVStage for a workgroup of NT threads.
template <typename TIn, int Wd, int C, int P, int NT>
struct RowStage {
    static constexpr int E = Elem<TIn>::kPerVec;
    static constexpr bool kSplit = std::is_same<TIn, float>::value;
    static constexpr int kVecs = C * (Wd / E);
    static constexpr int kRows = kVecs >= 4 * NT ? 4 : kVecs >= 2 * NT ? 2 : 1;
    static constexpr int kBlk = (C / kRows) * (Wd / E);
    static constexpr int kPer = (kBlk + NT - 1) / NT;
    static_assert(C % kRows == 0, "whole blocks of rows");
    uint4 x[kPer][kRows];

    template <int PP = P>
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int r0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int blk = tid + p * NT;
            const int a = blk / (Wd / E), b = blk % (Wd / E);
            if (kBlk % NT == 0 || blk < kBlk) {
#pragma unroll
                for (int rr = 0; rr < kRows; ++rr)
                    x[p][rr] = buf_load16<PP>(r, ((r0 + kRows * a + rr) * Wd + b * E) * int(sizeof(TIn)));
            }
        }
    }

    __device__ __forceinline__ void store(unsigned char* t) const {
        using PL = Plane<kSplit, Wd>;
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int blk = tid + p * NT;
            if (blk >= kBlk) continue;
            const int a = blk / (Wd / E), b = blk % (Wd / E);
#pragma unroll
            for (int h = 0; h < E / 4; ++h)
#pragma unroll
                for (int rr = 0; rr < kRows; ++rr) {
                    uint2 hi, lo;
                    if constexpr (kSplit) {
                        split4<true>(Elem<TIn>::get(x[p][rr], 4 * h), Elem<TIn>::get(x[p][rr], 4 * h + 1),
                                     Elem<TIn>::get(x[p][rr], 4 * h + 2),
                                     Elem<TIn>::get(x[p][rr], 4 * h + 3), hi, lo);
                    } else {
                        hi = make_uint2(h ? x[p][rr].z : x[p][rr].x, h ? x[p][rr].w : x[p][rr].y);
                        lo = hi;
                    }
                    PL::put4(t, kRows * a + rr, b * E + 4 * h, hi, lo);
                }
        }
    }
};

// Projection, plane values and features of one 16-token block (rows t0 ..
// t0 + 15 of the sub-chunk), all by the one wave that projects it: its lanes
// write the block's plane values to U and read them back as items (token,
// table), so the exchange needs only a wavefront-scope fence, not a
// workgroup barrier.  Each item decodes its table's sigma pairs once and
// writes the R / 4 corner quads: keys into the token-row plane tile (rows at
// or past `valid` zero: zero rows hash to 1/R, which would add mass), queries
// into the float tile Qf (OutTile layout), or with kQInPlane into the plane
// tile W will occupy: the four floats of a quad as the raw bits of its hi
// (two) and lo (two) slots, which the thread that forms W there reads back
// before it overwrites them.
template <typename TIn, int D, int S, int KP, int C, bool kQuery, typename PW, bool kQInPlane = false>
__device__ __forceinline__ void hash_block(const Projector<TIn, D, npb_of(S, KP)>& pj, const PW& wp, float* U,
                                           int t0, unsigned char* dst, int valid, float scale2, int g,
                                           int lr) {
    constexpr int NPB = npb_of(S, KP), L = tables_of(S, KP), R = 1 << KP;
    static_assert(!kQInPlane || std::is_same<TIn, float>::value, "fp32 plane slots hold a float each");
    using PS = Plane<std::is_same<TIn, float>::value, S>;
    using QT = OutTile<float, S, C>;
    constexpr int kUP = 16 * NPB + 1;
    f32x4 acc[NPB];
    pj.project(wp, g, lr, acc);
    hs_write_sigmas<NPB>(U, kUP, t0 + lr, acc, scale2, g);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < (16 * L + 63) / 64; ++i) {
        const int it = 16 * g + lr + 64 * i;
        if (16 * L % 64 != 0 && it >= 16 * L) break;
        const int t = t0 + (it & 15), l = it >> 4;
        CornerTable<KP> ct;
        ct.decode(U + t * kUP + l * KP);
        const float live = (kQuery || t < valid) ? 1.f : 0.f;
#pragma unroll
        for (int m = 0; m < R / 4; ++m) {
            const f32x4 q = live * ct.quad(m);
            if constexpr (kQuery && kQInPlane) {
                PS::put4(dst, t, l * R + 4 * m, make_uint2(__float_as_uint(q[0]), __float_as_uint(q[1])),
                         make_uint2(__float_as_uint(q[2]), __float_as_uint(q[3])));
            } else if constexpr (kQuery) {
                QT::put(dst, t, l * R + 4 * m, q);
            } else {
                uint2 hi, lo;
                split4<std::is_same<TIn, float>::value>(q[0], q[1], q[2], q[3], hi, lo);
                PS::put4(dst, t, l * R + 4 * m, hi, lo);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// K1: per (tile, stream) B_tile = Phi_K^T V, A_tile = colsum Phi_K into the
// tile record (B [S][D] then A [S]).  Wave w hashes 16-token block w of
// each sub-chunk (when C / 16 > w) and owns the V columns of c-blocks w,
// w + 4, .. for B and the buckets of s-blocks w, w + 4, .. for A.
//
// Where a wave's plane values fit its own 16 rows of the K plane tile and
// one pass over (token, table) items decodes them all (16 L <= 64), they are
// kept there (sums_u_in_k): every lane of the wave reads its items' values
// before the wave writes those rows, and only this wave writes them.
template <typename TIn, int S, int KP>
constexpr bool sums_u_in_k() {
    return 16 * tables_of(S, KP) <= 64 &&
           (16 * npb_of(S, KP) + 1) * 4 <= Plane<std::is_same<TIn, float>::value, S>::kPitch;
}

template <typename TIn, int S, int D, int C, int KP, int kMinBlocks, bool kDB>
__global__ __launch_bounds__(kThreads, kMinBlocks) void hashed_sums_kernel(
    const TIn* __restrict__ kx, const TIn* __restrict__ v, const float* __restrict__ planes,
    float* __restrict__ records, int64_t T, int tile, int64_t tiles, int64_t rec) {
    constexpr int NPB = npb_of(S, KP), LK = tables_of(S, KP) * KP;
    using G = Geo<TIn, S, D, C>;
    using PS = typename G::PS;
    using PD = typename G::PD;
    constexpr bool kSplit = G::kSplit;
    constexpr int NSB = S / 16, NKC = C / 32, CBW = D / 64, SBW = S / 64;
    constexpr int kUP = 16 * NPB + 1;
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr bool kUInK = sums_u_in_k<TIn, S, KP>();
    // fp32 rows at S = d = 64 (the cfg2 module): the memory-side cache
    // ordering of the probability-fed tile sums (mfma_direct.hip).
    constexpr bool kEndFirst = std::is_same<TIn, float>::value && S == 64 && D == 64 && kDB;
    unsigned char* Ks = lds;
    unsigned char* Vs = Ks + G::kKBytes;
    unsigned char* Ue = Vs + G::kVBytes;                     // [C][kUP] (not kUInK)
    unsigned char* Wl = Ue + (kUInK ? 0 : C * kUP * 4);      // the staged planes

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min(T, t_begin + tile) - t_begin);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(kx + (n * T + t_begin) * D, int64_t(rows) * D * sizeof(TIn));
    (void)l;
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * sizeof(TIn));
    const float scale2 = 2.0f * __builtin_amdgcn_rsqf(float(D));
    const bool projects = w < C / 16;
    // This wave's plane values: token t at U + t kUP.
    float* U = reinterpret_cast<float*>(kUInK ? Ks + 16 * w * (PS::kPitch - 4 * kUP) : Ue);
    // fp32 planes swizzled: the padding would keep S = d = 64 from four
    // workgroups per CU (40 KB of LDS each).
    using PW = std::conditional_t<std::is_same<TIn, float>::value, PlanesLdsT<true>, PlanesB3>;
    PW wp;
    if constexpr (std::is_same<TIn, float>::value) {
        stage_planes<D, NPB, kThreads, true>(reinterpret_cast<float*>(Wl), planes, LK);
        wp.w = reinterpret_cast<const float*>(Wl);
    } else {
        stage_planes_b3<D, NPB, kThreads>(Wl, planes, LK);
        wp.w = Wl;
        wp.rows = 16 * NPB;
    }

    f32x4 bacc[NSB][CBW], aacc[SBW];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) bacc[sb][cbw] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < SBW; ++j) aacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = __bf16(1.0f);

    // Wave w owns 16-token block w of every sub-chunk (C / 16 blocks); its
    // rows are double-buffered so the next sub-chunk's loads are issued
    // before this one's projection.
    RowStage<TIn, D, C, kSumsLoadPolicy, kThreads> vst;
    Projector<TIn, D, NPB> pjA;
    std::conditional_t<kDB, Projector<TIn, D, NPB>, Projector<TIn, D, NPB>&> pjB = pjA;
    using Stream = std::integral_constant<int, kSumsLoadPolicy>;
    using Alloc = std::integral_constant<int, kPolicyDefault>;
    // One sub-chunk at r0; the next one the walk takes (at rn, past either
    // end of the tile: zeros, never used) is loaded with policy `pol`.
    auto step = [&](auto pol, int r0, int rn, const Projector<TIn, D, NPB>& cur, Projector<TIn, D, NPB>& nxt) {
        constexpr int PP = decltype(pol)::value;
        __syncthreads();  // the previous sub-chunk's tiles have been read
        vst.store(Vs);
        vst.template load<PP>(vr, rn);
        if (projects) {
            if constexpr (kDB) nxt.template load<PP>(kr, rn + 16 * w, g, lr);
            hash_block<TIn, D, S, KP, C, false>(cur, wp, U, 16 * w, Ks, rows - r0, scale2, g, lr);
            if constexpr (!kDB) nxt.template load<PP>(kr, rn + 16 * w, g, lr);
        }
        __syncthreads();
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) {
            bf16x8 vh[NKC], vl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) PD::frag_tr(Vs, 32 * kk, 16 * (w + 4 * cbw), g, lr, vh[kk], vl[kk]);
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    bf16x8 kh, kl;
                    PS::frag_tr(Ks, 32 * kk, 16 * sb, g, lr, kh, kl);
                    bacc[sb][cbw] = mfma3<kSplit>(kh, kl, vh[kk], vl[kk], bacc[sb][cbw]);
                }
        }
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) {
                bf16x8 kh, kl;
                PS::frag_tr(Ks, 32 * kk, 16 * (w + 4 * j), g, lr, kh, kl);
                if constexpr (kSplit) aacc[j] = mfma16(kl, ones, aacc[j]);
                aacc[j] = mfma16(kh, ones, aacc[j]);
            }
        }
    };
    if constexpr (kEndFirst) {
        // End to start, the streamed part first; the first
        // RACE_HASHED_SUMS_ALLOC_EIGHTHS eighths of the tile (what the output
        // pass reads first) with the cache-allocating policy, last.
        const int last = ((rows - 1) / C) * C;
        const int cut = C * int((int64_t(tile / C) * RACE_HASHED_SUMS_ALLOC_EIGHTHS + 7) / 8);
        if (last < cut) {
            vst.template load<Alloc::value>(vr, last);
            if (projects) pjA.template load<Alloc::value>(kr, last + 16 * w, g, lr);
        } else {
            vst.template load<Stream::value>(vr, last);
            if (projects) pjA.template load<Stream::value>(kr, last + 16 * w, g, lr);
        }
        int r0 = last;
        for (; r0 - 2 * C >= cut; r0 -= 2 * C) {
            step(Stream{}, r0, r0 - C, pjA, pjB);
            step(Stream{}, r0 - C, r0 - 2 * C, pjB, pjA);
        }
        for (; r0 >= C; r0 -= 2 * C) {
            step(Alloc{}, r0, r0 - C, pjA, pjB);
            step(Alloc{}, r0 - C, r0 - 2 * C, pjB, pjA);
        }
        if (r0 >= 0) step(Alloc{}, r0, r0 - C, pjA, pjB);
    } else {
        vst.load(vr, 0);
        if (projects) pjA.template load<kSumsLoadPolicy>(kr, 16 * w, g, lr);
        for (int r0 = 0; r0 < rows; r0 += 2 * C) {
            step(Stream{}, r0, r0 + C, pjA, pjB);
            if (r0 + C < rows) step(Stream{}, r0 + C, r0 + 2 * C, pjB, pjA);
        }
    }

    float* r = records + (n * tiles + ti) * rec;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                r[(16 * sb + 4 * g + rr) * D + 16 * (w + 4 * cbw) + lr] = bacc[sb][cbw][rr];
    if (lr == 0) {
#pragma unroll
        for (int j = 0; j < SBW; ++j)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) r[S * D + 16 * (w + 4 * j) + 4 * g + rr] = aacc[j][rr];
    }
}

// ---------------------------------------------------------------------------
// K3: the output pass of mfma_causal.hip's causal_output_mfma_kernel with the
// hashing in front.  Per sub-chunk (barriers numbered):
//   (1) flush the previous output tile; stage V; issue the next sub-chunk's
//       loads; hash jobs (Q or K, 16-token block; hash_block): Phi_Q into
//       its float tile, Phi_K into the K plane tile (plane values in the P
//       tile's space)
//   (2) running mass, W = Phi_Q / (Abar + eps)
//   (3) P^T blocks = masked K W^T into the P tile
//   then output and state update as in the probability-input kernel.
// kLean (fp32 rows): Phi_Q goes into the W plane's own slots and each lane
// stores its output quad straight from the accumulators, so neither the
// query-feature tile nor the output tile takes LDS (37 KB at S = d = 64, C =
// 32: four workgroups per CU where 53 KB allowed three).
template <typename TIn, int S, int D, int C, int KP, int kMinBlocks, int NW, bool kWl, bool kDB, bool kLean>
__global__ __launch_bounds__(64 * NW, kMinBlocks) void hashed_output_kernel(
    const TIn* __restrict__ qx, const TIn* __restrict__ kx, const TIn* __restrict__ v,
    const float* __restrict__ planes, TIn* __restrict__ out, const float* __restrict__ records,
    int64_t T, int tile, int64_t tiles, int64_t rec) {
    constexpr int NPB = npb_of(S, KP), LK = tables_of(S, KP) * KP;
    static_assert(kWl || std::is_same<TIn, float>::value, "bf16 rows project against staged planes");
    using G = Geo<TIn, S, D, C, NW>;
    using PS = typename G::PS;
    using PC = typename G::PC;
    using PD = typename G::PD;
    constexpr bool kSplit = G::kSplit;
    static_assert(!kLean || kSplit, "the lean layout keeps fp32 Phi_Q in the hi/lo plane slots");
    constexpr int NSB = S / 16, NBI = C / 16, NKS = S / 32, NKC = C / 32;
    constexpr int SBW = S / (16 * NW), CBW = D / (16 * NW);
    constexpr int NLB = NBI * (NBI + 1) / 2;
    constexpr int PBW = (NLB + NW - 1) / NW;
    constexpr int kUP = 16 * NPB + 1;
    constexpr int kUBytes = C * kUP * 4;
    constexpr int kPU = G::kPBytes > 2 * kUBytes ? G::kPBytes : 2 * kUBytes;
    constexpr int kJobs = 2 * NBI;  // (Q or K, 16-token block)
    constexpr int kJobsW = (kJobs + NW - 1) / NW;
    constexpr int kStoreP = std::is_same<TIn, float>::value ? kOutWgStorePolicyF32 : kOutStorePolicy;
    // fp32 rows at S = d = 64: Q streams past the memory-side cache, which
    // holds the K and V rows the tile sums left there.
    constexpr int kQP = (std::is_same<TIn, float>::value && S == 64 && D == 64) ? kOutQPolicyF32 : kOutQPolicy;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Ws = lds;
    unsigned char* Ks = Ws + G::kWBytes;
    unsigned char* Ps = Ks + G::kKBytes;  // P; earlier in a sub-chunk U_Q then U_K
    float* Uq = reinterpret_cast<float*>(Ps);
    float* Uk = Uq + C * kUP;
    unsigned char* Vs = Ps + kPU;
    unsigned char* Os = Vs + G::kVBytes;                                  // out (not kLean)
    unsigned char* Qf = Os + (kLean ? 0 : C * D * int(sizeof(TIn)));      // Phi_Q [C][S] fp32 (not kLean)
    unsigned char* Wl = Qf + (kLean ? 0 : C * S * 4);                     // the staged planes (kWl)
    using OT = OutTile<TIn, D, C>;
    using QT = OutTile<float, S, C>;

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min(T, t_begin + tile) - t_begin);
    const int64_t row_bytes = int64_t(rows) * D * sizeof(TIn);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(qx + (n * T + t_begin) * D, row_bytes);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(kx + (n * T + t_begin) * D, row_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, row_bytes);
    const __amdgpu_buffer_rsrc_t or_ = make_rsrc(out + (n * T + t_begin) * D, row_bytes);
    const float scale2 = 2.0f * __builtin_amdgcn_rsqf(float(D));
    // The planes: staged in LDS (read after the first barrier) when the
    // workgroup's LDS has room, else read through the cache.
    using PW = std::conditional_t<!kWl, PlanesGlobal,
                                  std::conditional_t<std::is_same<TIn, float>::value, PlanesLds, PlanesB3>>;
    PW wp;
    if constexpr (!kWl) {
        wp.r = make_rsrc(planes, int64_t(LK) * D * 4);
    } else if constexpr (std::is_same<TIn, float>::value) {
        stage_planes<D, NPB, 64 * NW>(reinterpret_cast<float*>(Wl), planes, LK);
        wp.w = reinterpret_cast<const float*>(Wl);
    } else {
        stage_planes_b3<D, NPB, 64 * NW>(Wl, planes, LK);
        wp.w = Wl;
        wp.rows = 16 * NPB;
    }

    // Carried state from the tile's exclusive prefix record.
    const float* rec_p = records + (n * tiles + ti) * rec;
    f32x4 b0[NSB][CBW];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                b0[sb][cbw][rr] = rec_p[(16 * sb + 4 * g + rr) * D + 16 * (w + NW * cbw) + lr];
    float a0[SBW][4];
#pragma unroll
    for (int sbw = 0; sbw < SBW; ++sbw)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) a0[sbw][rr] = rec_p[S * D + 16 * (w + NW * sbw) + 4 * g + rr];

    const bf16x8 tri0 = tril_frag(0, g, lr), tri1 = tril_frag(16, g, lr);
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = __bf16(1.0f);

    // Wave w hashes jobs w, w + NW, ..: job j < NBI is query block j, the
    // others key block j - NBI.  With kDB their rows are double-buffered, so
    // the next sub-chunk's loads are issued before this one's projections;
    // without it (where the registers are short) they are issued after.
    struct Jobs {
        Projector<TIn, D, NPB> j[kJobsW];
    };
    RowStage<TIn, D, C, kOutKVPolicy, 64 * NW> vst;
    Jobs pjA;
    std::conditional_t<kDB, Jobs, Jobs&> pjB = pjA;
    auto load_rows = [&](Jobs& dst, int r0) {
#pragma unroll
        for (int j = 0; j < kJobsW; ++j) {
            const int job = w + NW * j;
            if (job < kJobs) {
                if (job < NBI)
                    dst.j[j].template load<kQP>(qr, r0 + 16 * job, g, lr);
                else
                    dst.j[j].template load<kOutKVPolicy>(kr, r0 + 16 * (job - NBI), g, lr);
            }
        }
    };

    auto sub_chunk = [&](int r0, const Jobs& cur, Jobs& nxt) {
        __syncthreads();
        // Unconditional flush (at r0 = 0 the offsets fall outside the buffer
        // range and the stores are dropped), as in the probability kernel.
        if constexpr (!kLean) OT::template flush<kStoreP, G::kT>(Os, or_, r0 - C);
        vst.store(Vs);
        vst.load(vr, r0 + C);  // prefetch (past the tile: zeros, never used)
        if constexpr (kDB) load_rows(nxt, r0 + C);
#pragma unroll
        for (int j = 0; j < kJobsW; ++j) {
            const int job = w + NW * j;
            if (job < NBI)
                hash_block<TIn, D, S, KP, C, true, PW, kLean>(cur.j[j], wp, Uq, 16 * job, kLean ? Ws : Qf,
                                                              rows - r0, scale2, g, lr);
            else if (job < kJobs)
                hash_block<TIn, D, S, KP, C, false>(cur.j[j], wp, Uk, 16 * (job - NBI), Ks, rows - r0,
                                                    scale2, g, lr);
        }
        if constexpr (!kDB) load_rows(nxt, r0 + C);
        __syncthreads();

        // Running mass, Phi_Q and W.
#pragma unroll
        for (int sbw = 0; sbw < SBW; ++sbw) {
            const int sb = w + NW * sbw;
            bf16x8 kh[NKC], kl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) PS::frag_tr(Ks, 32 * kk, 16 * sb, g, lr, kh[kk], kl[kk]);
            f32x4 last;
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
                f32x4 acc = {a0[sbw][0], a0[sbw][1], a0[sbw][2], a0[sbw][3]};
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    const int off = 16 * bi - 32 * kk;
                    if (off < 0) continue;
                    const bf16x8& lf = off == 0 ? tri0 : off == 16 ? tri1 : ones;
                    if constexpr (kSplit) acc = mfma16(kl[kk], lf, acc);
                    acc = mfma16(kh[kk], lf, acc);
                }
                f32x4 qv;
                if constexpr (kLean) {
                    const int at = PS::off4(16 * bi + lr, 16 * sb + 4 * g);
                    const uint2 h = *reinterpret_cast<const uint2*>(Ws + at);
                    const uint2 lo = *reinterpret_cast<const uint2*>(Ws + at + PS::kLoOff);
                    qv = f32x4{__uint_as_float(h.x), __uint_as_float(h.y), __uint_as_float(lo.x),
                               __uint_as_float(lo.y)};
                } else {
                    qv = QT::get4(Qf, 16 * bi + lr, 16 * sb + 4 * g);
                }
                uint2 hi, lo;
                split4<kSplit>(qv[0] * __builtin_amdgcn_rcpf(acc[0] + kEps),
                               qv[1] * __builtin_amdgcn_rcpf(acc[1] + kEps),
                               qv[2] * __builtin_amdgcn_rcpf(acc[2] + kEps),
                               qv[3] * __builtin_amdgcn_rcpf(acc[3] + kEps), hi, lo);
                PS::put4(Ws, 16 * bi + lr, 16 * sb + 4 * g, hi, lo);
                last = acc;
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) a0[sbw][rr] = __shfl(last[rr], 16 * g + 15);
        }
        __syncthreads();

        // P^T blocks of the lower triangle, round robin over the waves.
        f32x4 pacc[PBW];
        int pbi[PBW], pbj[PBW];
#pragma unroll
        for (int pb = 0; pb < PBW; ++pb) {
            const int idx = w + NW * pb;
            int bi = 0, rem = idx;
            while (rem > bi) { rem -= bi + 1; ++bi; }
            pbi[pb] = bi;
            pbj[pb] = rem;
            pacc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (idx >= NLB) continue;
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                bf16x8 ah, al, bh, bl;
                PS::frag(Ks, 16 * rem + lr, kk, g, ah, al);
                PS::frag(Ws, 16 * bi + lr, kk, g, bh, bl);
                pacc[pb] = mfma3<kSplit>(ah, al, bh, bl, pacc[pb]);
            }
            if (rem == bi) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (4 * g + rr > lr) pacc[pb][rr] = 0.f;
            }
        }
#pragma unroll
        for (int pb = 0; pb < PBW; ++pb) {
            if (w + NW * pb >= NLB) continue;
            uint2 hi, lo;
            split4<kSplit>(pacc[pb][0], pacc[pb][1], pacc[pb][2], pacc[pb][3], hi, lo);
            PC::put4(Ps, 16 * pbi[pb] + lr, 16 * pbj[pb] + 4 * g, hi, lo);
        }
        __syncthreads();

        // Output and state update for this wave's c-blocks.
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) {
            const int cb = w + NW * cbw;
            bf16x8 vh[NKC], vl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) PD::frag_tr(Vs, 32 * kk, 16 * cb, g, lr, vh[kk], vl[kk]);
            f32x4 o[NBI];
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) o[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                const f32x4 x0 = b0[2 * kk][cbw], x1 = b0[2 * kk + 1][cbw];
                uint2 h0, l0, h1, l1;
                split4<kSplit>(x0[0], x0[1], x0[2], x0[3], h0, l0);
                split4<kSplit>(x1[0], x1[1], x1[2], x1[3], h1, l1);
                const bf16x8 bh = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                bf16x8 bl;
                if constexpr (kSplit) bl = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi) {
                    bf16x8 wh, wl;
                    PS::frag(Ws, 16 * bi + lr, kk, g, wh, wl);
                    o[bi] = mfma3<kSplit>(bh, bl, wh, wl, o[bi]);
                }
            }
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    if (32 * kk > 16 * bi) continue;
                    bf16x8 ph, pl;
                    PC::frag(Ps, 16 * bi + lr, kk, g, ph, pl);
                    if (32 * kk == 16 * bi) {
#pragma unroll
                        for (int e = 4; e < 8; ++e) {
                            ph[e] = __bf16(0.0f);
                            if constexpr (kSplit) pl[e] = __bf16(0.0f);
                        }
                    }
                    o[bi] = mfma3<kSplit>(vh[kk], vl[kk], ph, pl, o[bi]);
                }
                // Lean: rows past the tile fall outside or_ and are dropped.  The
                // default (write-back) policy lets the two 64-byte halves of a
                // 128-byte line, stored by two waves, meet in L2; streamed, lines
                // left half written and reached HBM twice (1.23x the bytes).
                if constexpr (kLean)
                    store4<TIn, kOutStorePolicy>(or_, ((r0 + 16 * bi + lr) * D + 16 * cb + 4 * g) * 4, o[bi]);
                else
                    OT::put(Os, 16 * bi + lr, 16 * cb + 4 * g, o[bi]);
            }
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    bf16x8 kh, kl;
                    PS::frag_tr(Ks, 32 * kk, 16 * sb, g, lr, kh, kl);
                    b0[sb][cbw] = mfma3<kSplit>(kh, kl, vh[kk], vl[kk], b0[sb][cbw]);
                }
                if constexpr (kSplit && S * D >= 128 * 128) __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    vst.load(vr, 0);
    load_rows(pjA, 0);
    int r0 = 0;
    for (; r0 < rows; r0 += 2 * C) {
        sub_chunk(r0, pjA, pjB);
        if (r0 + C < rows) sub_chunk(r0 + C, pjB, pjA);
    }
    r0 = ((rows + C - 1) / C) * C;  // one past the last sub-chunk
    if constexpr (!kLean) {
        __syncthreads();
        if (r0 > 0) OT::template flush<kStoreP, G::kT>(Os, or_, r0 - C);
    }
}

// LDS of the output pass, with (kWl) or without the staged planes.
template <typename TIn, int S, int D, int C, int KP, int NW, bool kWl, bool kLean = false>
constexpr int hashed_output_lds() {
    using G = Geo<TIn, S, D, C, NW>;
    constexpr int NPB = npb_of(S, KP);
    constexpr int kUBytes = C * (16 * NPB + 1) * 4;
    constexpr int kPU = G::kPBytes > 2 * kUBytes ? G::kPBytes : 2 * kUBytes;
    return G::kWBytes + G::kKBytes + kPU + G::kVBytes + (kLean ? 0 : C * D * int(sizeof(TIn)) + C * S * 4) +
           (kWl ? planes_lds_bytes<TIn, D, NPB>() : 0);
}
constexpr int kMaxLds = 160 * 1024;  // gfx950: LDS per workgroup

template <typename TIn, int S, int D, int C, int KP>
constexpr int hashed_sums_lds() {
    using G = Geo<TIn, S, D, C>;
    constexpr int NPB = npb_of(S, KP);
    return G::kKBytes + G::kVBytes + (sums_u_in_k<TIn, S, KP>() ? 0 : C * (16 * NPB + 1) * 4) +
           planes_lds_bytes<TIn, D, NPB, true>();
}

// C: the output pass's sub-chunk; CS: the tile sums' (a multiple of C); kDB:
// double-buffered row registers (where they fit); kLean: the output pass's
// fp32 layout without the query-feature and output tiles; kSumsBlocks and
// kSumsDB: the tile sums' workgroups per CU and row buffering.
template <typename TIn, int S, int D, int C, int KP, int kMinBlocks, int NW = 4, int CS = C,
          bool kDB = false, bool kLean = false, int kSumsBlocks = kMinBlocks, bool kSumsDB = kDB>
hipError_t launch_hashed_family(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks) {
    if (p.tile % C != 0 || p.tile % CS != 0) return hipErrorInvalidValue;
    // The planes go to LDS when the output pass has room for them (not at
    // fp32, S = d = 128).  gfx950 gives a workgroup at most 160 KB.
    constexpr bool kWl = hashed_output_lds<TIn, S, D, C, KP, NW, true, kLean>() <= kMaxLds;
    constexpr int kOutLds = hashed_output_lds<TIn, S, D, C, KP, NW, kWl, kLean>();
    static_assert(kOutLds <= kMaxLds, "output pass LDS");
    static_assert(hashed_sums_lds<TIn, S, D, CS, KP>() <= kMaxLds, "tile sums LDS");
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    hipError_t err;
    hashed_sums_kernel<TIn, S, D, CS, KP, kSumsBlocks, kSumsDB>
        <<<grid, kThreads, hashed_sums_lds<TIn, S, D, CS, KP>(), stream>>>(
            static_cast<const TIn*>(a.k), static_cast<const TIn*>(a.v), a.planes, a.records, p.T, p.tile,
            p.tiles, p.rec);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    if ((err = launch_tile_scan(a.records, a.state, p, stream)) != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    hashed_output_kernel<TIn, S, D, C, KP, kMinBlocks, NW, kWl, kDB, kLean>
        <<<grid, 64 * NW, kOutLds, stream>>>(
            static_cast<const TIn*>(a.q), static_cast<const TIn*>(a.k), static_cast<const TIn*>(a.v),
            a.planes, static_cast<TIn*>(a.out), a.records, p.T, p.tile, p.tiles, p.rec);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    return marks ? marks->mark(stream) : hipSuccess;
}

template <typename TIn, int S, int D, int KP>
hipError_t launch_hashed_shape(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks) {
    if constexpr (!kp_ok(S, KP)) {
        return hipErrorInvalidValue;
    } else if constexpr (S == 64 && D == 64) {
        // Four workgroups per CU where the output pass fits 40 KB of LDS (bf16
        // rows in the ordinary layout, fp32 rows in the lean one), rows
        // single-buffered (double-buffered they would spill).  Else (fewer
        // planes per table: more tables, larger hash scratch and planes)
        // three, rows double-buffered.  64-token sub-chunks for the tile sums.
        constexpr bool kLean = std::is_same<TIn, float>::value;
        constexpr bool kFour = hashed_output_lds<TIn, 64, 64, 32, KP, 4, true, kLean>() <= kMaxLds / 4;
        if constexpr (kFour)
            return launch_hashed_family<TIn, 64, 64, 32, KP, 4, 4, 64, false, kLean,
                                        kLean ? RACE_HASHED_SUMS_F32_BLOCKS : 4, kLean>(a, p, stream, marks);
        else
            return launch_hashed_family<TIn, 64, 64, 32, KP, 3, 4, 64, true>(a, p, stream, marks);
    } else if constexpr (S == 256 && D == 128) {
        return launch_hashed_family<TIn, 256, 128, 32, KP, 1, 8>(a, p, stream, marks);
    } else {
        // 32-token sub-chunks: with the query features' own tile, 64 would not
        // fit fp32 S = d = 128 in 160 KB of LDS.
        return launch_hashed_family<TIn, S, D, 32, KP, 1>(a, p, stream, marks);
    }
}

template <typename TIn, int S, int D>
hipError_t dispatch_kp(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks) {
    switch (a.K) {
        case 2: return launch_hashed_shape<TIn, S, D, 2>(a, p, stream, marks);
        case 3: return launch_hashed_shape<TIn, S, D, 3>(a, p, stream, marks);
        case 4: return launch_hashed_shape<TIn, S, D, 4>(a, p, stream, marks);
        case 5: return launch_hashed_shape<TIn, S, D, 5>(a, p, stream, marks);
        case 6: return launch_hashed_shape<TIn, S, D, 6>(a, p, stream, marks);
        case 7: return launch_hashed_shape<TIn, S, D, 7>(a, p, stream, marks);
        case 8: return launch_hashed_shape<TIn, S, D, 8>(a, p, stream, marks);
        default: return hipErrorInvalidValue;
    }
}

// The (S, d) specializations of the probability kernels (mfma_causal.hip).
template <typename TIn>
hipError_t dispatch_hashed(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks) {
    if (p.S == 64 && p.d == 64) return dispatch_kp<TIn, 64, 64>(a, p, stream, marks);
    if (p.S == 64 && p.d == 128) return dispatch_kp<TIn, 64, 128>(a, p, stream, marks);
    if (p.S == 128 && p.d == 64) return dispatch_kp<TIn, 128, 64>(a, p, stream, marks);
    if (p.S == 128 && p.d == 128) return dispatch_kp<TIn, 128, 128>(a, p, stream, marks);
    if (p.S == 256 && p.d == 64) return dispatch_kp<TIn, 256, 64>(a, p, stream, marks);
    if (p.S == 256 && p.d == 128) return dispatch_kp<TIn, 256, 128>(a, p, stream, marks);
    return hipErrorInvalidValue;
}

}  // namespace hashed

// The bf16 instantiation (hashed_causal_bf16.hip).
hipError_t launch_hashed_causal_bf16(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks);

}  // namespace race
