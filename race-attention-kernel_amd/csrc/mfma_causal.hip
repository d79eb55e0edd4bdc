// mfma_causal.hip -- matrix-core (MFMA) causal forward for gfx950.
//
// The per-bucket causal function of src/race_baseline.py:45-51 through the
// chunk identity (docs/causal_v2_design.md:70-77, restated per bucket):
// for a sub-chunk of C tokens with carried state (A0 [S], B0 [S][d]),
//     Abar = A0 + tril(1) K          (inclusive running mass per query row)
//     W    = Q / (Abar + eps)
//     O    = W B0 + tril(W K^T) V
//     A0  += 1^T K,   B0 += K^T V.
// Every product runs on v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
// fp32 inputs are carried as bf16 hi/lo pairs (x = hi + lo, hi = bf16(x),
// lo = bf16(x - hi)) and each product takes the three terms hi*hi + hi*lo +
// lo*hi, which leaves a relative error of about 2^-17 per product; bf16
// inputs take the single hi*hi product.
//
// Launch sequence (the decomposition of the reference's v2,
// src/causal_v2/kernels/race_causal_fwd.h:23-27, for the per-bucket function):
//   1. tile_sums_mfma_kernel     per (tile, stream): B_tile = K^T V, A_tile = 1^T K
//   2. tile_scan_kernel          exclusive scan of the tile records (VALU file)
//   3. causal_output_mfma_kernel per (tile, stream): walks the tile's
//      sub-chunks from its exclusive prefix state.
//
// Layout conventions.  Workgroups are 4 wave64s.  A lane l of a wave has
// group g = l / 16 and row lr = l % 16.  For the MFMA A operand a lane supplies
// row m = lr of a 16-row block and 8 values of the contraction index k; for the
// B operand column n = lr and the same 8 k values; the accumulator gives lane
// l the 4 values D[4g + r][lr], r = 0..3.  The contraction index of one
// 32-wide step kk is permuted: lane group g, element e carries
//     k = 32 kk + 4 g + (e % 4) + 16 (e / 4),
// which is exactly the set of rows an accumulator of two stacked 16-row blocks
// gives a lane; so the carried state B0, held in accumulators, feeds the next
// product without a trip through LDS.
//
// LDS operand tiles are stored in that "fragment order": a row of K elements
// holds the bf16 high parts of all its elements in fragment order, then (with
// hi/lo) the low parts, so element k sits at position
//     fpos(k) = 32 (k / 32) + 8 ((k / 4) % 4) + 4 ((k / 16) % 2) + k % 4
// of each plane and one fragment is a single 16-byte read per plane (the
// chunk swizzle of Plane keeps those reads and the staging stores spread over
// the banks).  Tiles are stored with tokens as rows only; the operands that
// contract over tokens (K^T, V^T) are read transposed from the same tiles with
// ds_read_b64_tr_b16 (Plane::frag_tr), two reads per fragment and plane.
#include "causal_geo.h"

// fp32 S = d = 64 output pass: two sub-chunks of operands in flight in
// registers ahead of the one in LDS, at two workgroups per CU (the launch
// bound that leaves room for them).  With the automatic 1024-token tiles two
// workgroups per CU is what the launch holds anyway; measured at cfg2
// (20 steps after the settling phase, one box): 3755 -> 3794 M tokens/s with
// the same inputs every step, 3469 -> 3510 with two input sets alternating.
#ifndef RACE_OUT_F32_DEPTH
#define RACE_OUT_F32_DEPTH 2
#endif
#ifndef RACE_OUT_F32_6464_MINBLOCKS
#define RACE_OUT_F32_6464_MINBLOCKS 2
#endif

namespace race {
namespace {

using namespace mfma;


// ---------------------------------------------------------------------------
// K1: per (tile, stream) totals B_tile = K^T V and A_tile = colsum(K) into the
// tile record (B [S][D] then A [S]).  Wave w owns the V columns of c-blocks
// w, w + 4, ...; its accumulators hold B[16 sb + 4 g + r][16 cb + lr].
template <typename TIn, int S, int D, int C, int kMinBlocks>
__global__ __launch_bounds__(kThreads, kMinBlocks) void tile_sums_mfma_kernel(
    const TIn* __restrict__ k, const TIn* __restrict__ v, float* __restrict__ records, int64_t T,
    int tile, int64_t tiles, int64_t rec) {
    using G = Geo<TIn, S, D, C>;
    using PS = typename G::PS;
    using PK = typename G::PK;
    using PD = typename G::PD;
    constexpr bool kSplit = G::kSplit;
    constexpr int NSB = S / 16, NKC = C / 32, CBW = D / 64;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Ks = lds;
    unsigned char* Vs = Ks + G::kKBytes;
    float* Apart = reinterpret_cast<float*>(Vs + G::kVBytes);  // [16][S]

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const int rows = int(t_end - t_begin);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + (n * T + t_begin) * S, int64_t(rows) * S * sizeof(TIn));
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * sizeof(TIn));

    f32x4 acc[NSB][CBW];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) acc[sb][cbw] = f32x4{0.f, 0.f, 0.f, 0.f};
    float asum[G::kKPer * G::E];
#pragma unroll
    for (int i = 0; i < G::kKPer * G::E; ++i) asum[i] = 0.f;

    KVStage<TIn, S, D, C, kSumsLoadPolicy> st;
    st.load(kr, vr, 0);
    for (int r0 = 0; r0 < rows; r0 += C) {
        __syncthreads();
        st.store(Ks, Vs, asum);
        st.load(kr, vr, r0 + C);  // past the tile: zeros, never used
        __syncthreads();
        bf16x8 vh[CBW][NKC], vl[CBW][NKC];
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) PD::frag_tr(Vs, 32 * kk, 16 * (w + 4 * cbw), g, lr, vh[cbw][kk], vl[cbw][kk]);
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) {
                bf16x8 kh, kl;
                PK::frag_tr(Ks, 32 * kk, 16 * sb, g, lr, kh, kl);
#pragma unroll
                for (int cbw = 0; cbw < CBW; ++cbw)
                    acc[sb][cbw] = mfma3<kSplit>(kh, kl, vh[cbw][kk], vl[cbw][kk], acc[sb][cbw]);
            }
    }

    float* r = records + (n * tiles + ti) * rec;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                r[(16 * sb + 4 * g + rr) * D + 16 * (w + 4 * cbw) + lr] = acc[sb][cbw][rr];

    // Column sums: thread partials per 4-row group a, then a fixed-order sum over a.
    __syncthreads();
    for (int e = tid; e < 16 * S; e += kThreads) Apart[e] = 0.f;
    __syncthreads();
#pragma unroll
    for (int p = 0; p < G::kKPer; ++p) {
        const int blk = tid + p * kThreads;
        if (blk >= G::kKBlk) continue;
        const int a = blk / (S / G::E), b = blk % (S / G::E);
#pragma unroll
        for (int c = 0; c < G::E; ++c) Apart[(a & 15) * S + b * G::E + c] += asum[p * G::E + c];
    }
    __syncthreads();
    if (tid < S) {
        float sum = 0.f;
        for (int a = 0; a < 16; ++a) sum += Apart[a * S + tid];
        r[S * D + tid] = sum;
    }
}

// ---------------------------------------------------------------------------
// K3: causal output pass, one workgroup per (tile, stream), walking the tile
// in sub-chunks of C tokens from the tile's exclusive prefix record.
//
// Per sub-chunk:
//   1. Abar^T [S][C] = A0 + K^T tril(1)       wave w: s-blocks w, w+4, ..
//   2. W [C][S] = Q / (Abar + eps)             Q read from global memory in
//      the accumulator layout, W written as a plane tile
//   3. P^T blocks (j-block <= i-block) = K W^T, masked j > i, written as the
//      plane tile P [C][C]
//   4. O^T [D][C] = B0^T W^T + V^T P^T         wave w: c-blocks w, w+NW, ..
//   5. B0 += K^T V                             same c-blocks, all s-blocks
// NW waves per workgroup (4, or 8 where the carried state would otherwise
// fill the register file: two waves per SIMD then share the CU's work).
template <typename TIn, int S, int D, int C, int kMinBlocks, int NW, bool kPrecise>
__global__ __launch_bounds__(64 * NW, kMinBlocks) void causal_output_mfma_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    TIn* __restrict__ out, const float* __restrict__ records, int64_t T, int tile, int64_t tiles,
    int64_t rec) {
    using G = Geo<TIn, S, D, C, NW, kPrecise>;
    using PS = typename G::PS;
    using PK = typename G::PK;
    using PC = typename G::PC;
    using PD = typename G::PD;
    constexpr bool kSplit = G::kSplit;
    constexpr int NSB = S / 16, NBI = C / 16, NKS = S / 32, NKC = C / 32;
    constexpr int SBW = S / (16 * NW), CBW = D / (16 * NW);
    constexpr int NLB = NBI * (NBI + 1) / 2;       // lower-triangular P blocks
    constexpr int PBW = (NLB + NW - 1) / NW;       // P blocks per wave
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Ws = lds;
    unsigned char* Ks = Ws + G::kWBytes;
    unsigned char* Ps = Ks + G::kKBytes;
    unsigned char* Vs = Ps + G::kPBytes;
    unsigned char* Os = Vs + G::kVBytes;
    unsigned char* Qs = Os + G::kOBytes;
    using OT = OutTile<TIn, D, C>;
    using QT = OutTile<TIn, S, C>;
    constexpr bool kQStage = G::kQStage;
    constexpr int kQChunks = C * QT::kChunks;
    constexpr int kQPer = (kQChunks + G::kT - 1) / G::kT;
    constexpr int kStoreP = std::is_same<TIn, float>::value ? kOutWgStorePolicyF32 : kOutStorePolicy;
    constexpr int kQP = std::is_same<TIn, float>::value ? kOutQPolicyF32 : kOutQPolicy;
    // Sub-chunks of operands in flight in registers ahead of the one in LDS.
    constexpr int kDepth = (std::is_same<TIn, float>::value && S == 64 && D == 64) ? RACE_OUT_F32_DEPTH : 1;

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const int rows = int(t_end - t_begin);
    const __amdgpu_buffer_rsrc_t qr_ = make_rsrc(q + (n * T + t_begin) * S, int64_t(rows) * S * sizeof(TIn));
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + (n * T + t_begin) * S, int64_t(rows) * S * sizeof(TIn));
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * sizeof(TIn));
    const __amdgpu_buffer_rsrc_t or_ = make_rsrc(out + (n * T + t_begin) * D, int64_t(rows) * D * sizeof(TIn));

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

    // The two partial triangles of the running-mass operand (i - j offset 0 or 16).
    const bf16x8 tri0 = tril_frag(0, g, lr), tri1 = tril_frag(16, g, lr);
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = __bf16(1.0f);

    // Q of a sub-chunk: staged (bf16) as 16-byte chunks of whole rows, or in
    // the layout of step 2, lane (g, lr) holding Q[16 bi + lr][16 (w + NW sbw)
    // + 4 g .. + 3].
    using QRegs = std::conditional_t<kQStage, uint4[kQPer], f32x4[SBW][NBI]>;
    auto load_q = [&](QRegs& qr, int r0) {
        if constexpr (kQStage) {
#pragma unroll
            for (int i = 0; i < kQPer; ++i) {
                const int qi = tid + i * G::kT;
                if (kQChunks % G::kT == 0 || qi < kQChunks)
                    qr[i] = buf_load16<kQP>(qr_, r0 * S * int(sizeof(TIn)) + 16 * qi);
            }
        } else {
#pragma unroll
            for (int sbw = 0; sbw < SBW; ++sbw)
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi)
                    qr[sbw][bi] = load_q4<TIn, kQP>(
                        qr_, ((r0 + 16 * bi + lr) * S + 16 * (w + NW * sbw) + 4 * g) * int(sizeof(TIn)));
        }
    };

    // One sub-chunk from the raw registers `st` / `qr`, which are then
    // refilled with the next sub-chunk (a deeper prefetch measured slower).
    // The previous sub-chunk's output tile is flushed after the first barrier
    // (measured: issuing it after the prefetch instead was slower at cfg5).
    auto sub_chunk = [&](KVStage<TIn, S, D, C, kOutKVPolicy, NW, kPrecise>& st, QRegs& qr, int r0) {
        __syncthreads();
        // Unconditional: at r0 = 0 the offsets are negative, outside the
        // buffer range, so those stores are dropped.  (A conditional flush
        // gives the compiler a peeled first iteration; in the backward's bf16
        // dQ kernel that peel produced wrong values.)
        OT::template flush<kStoreP, G::kT>(Os, or_, r0 - C);
        st.store(Ks, Vs, nullptr);
        f32x4 qc[SBW][NBI];
        if constexpr (kQStage) {
#pragma unroll
            for (int i = 0; i < kQPer; ++i) {
                const int qi = tid + i * G::kT;
                if (kQChunks % G::kT == 0 || qi < kQChunks)
                    *reinterpret_cast<uint4*>(Qs + QT::chunk_at(qi)) = qr[i];
            }
        } else {
#pragma unroll
            for (int sbw = 0; sbw < SBW; ++sbw)
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi) qc[sbw][bi] = qr[sbw][bi];
        }
        // Prefetch (past the tile: zeros, never used).
        st.load(kr, vr, r0 + kDepth * C);
        load_q(qr, r0 + kDepth * C);
        __syncthreads();

        // 1 + 2: running mass and W.
#pragma unroll
        for (int sbw = 0; sbw < SBW; ++sbw) {
            const int sb = w + NW * sbw;
            bf16x8 kh[NKC], kl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) PK::frag_tr(Ks, 32 * kk, 16 * sb, g, lr, kh[kk], kl[kk]);
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
                const f32x4 qv = kQStage ? QT::get4(Qs, 16 * bi + lr, 16 * sb + 4 * g) : qc[sbw][bi];
                uint2 hi, lo;
                split4<kSplit>(qv[0] * __builtin_amdgcn_rcpf(acc[0] + kEps),
                               qv[1] * __builtin_amdgcn_rcpf(acc[1] + kEps),
                               qv[2] * __builtin_amdgcn_rcpf(acc[2] + kEps),
                               qv[3] * __builtin_amdgcn_rcpf(acc[3] + kEps), hi, lo);
                PS::put4(Ws, 16 * bi + lr, 16 * sb + 4 * g, hi, lo);
                last = acc;
            }
            // Inclusive mass at the chunk's last row (zero rows past the tile add nothing).
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) a0[sbw][rr] = __shfl(last[rr], 16 * g + 15);
        }
        __syncthreads();

        // 3: P^T blocks of the lower triangle, round robin over the waves.
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
                PK::frag(Ks, 16 * rem + lr, kk, g, ah, al);
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

        // 4 + 5: output and state update for this wave's c-blocks.
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
                        // The upper half of this step is the block above the
                        // diagonal: zero, and never written to the P tile.
#pragma unroll
                        for (int e = 4; e < 8; ++e) {
                            ph[e] = __bf16(0.0f);
                            if constexpr (kSplit) pl[e] = __bf16(0.0f);
                        }
                    }
                    o[bi] = mfma3<kSplit>(vh[kk], vl[kk], ph, pl, o[bi]);
                }
                OT::put(Os, 16 * bi + lr, 16 * cb + 4 * g, o[bi]);
            }
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    bf16x8 kh, kl;
                    PK::frag_tr(Ks, 32 * kk, 16 * sb, g, lr, kh, kl);
                    b0[sb][cbw] = mfma3<kSplit>(kh, kl, vh[kk], vl[kk], b0[sb][cbw]);
                }
                // Where the carried state fills the register file, keep the
                // scheduler from hoisting every s-block's operand reads.
                if constexpr (kSplit && S * D >= 128 * 128) __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    KVStage<TIn, S, D, C, kOutKVPolicy, NW, kPrecise> st[kDepth];
    QRegs qr[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        st[d].load(kr, vr, d * C);
        load_q(qr[d], d * C);
    }
    int r0 = 0;
    for (; r0 < rows; r0 += kDepth * C) {
        // A sub-chunk past a ragged tile end reads zeros and stores nothing.
#pragma unroll
        for (int d = 0; d < kDepth; ++d) sub_chunk(st[d], qr[d], r0 + d * C);
    }
    __syncthreads();
    if (r0 > 0) OT::template flush<kStoreP, G::kT>(Os, or_, r0 - C);
}

// K1 alone: the register-direct kernel where it applies, else the workgroup one.
template <typename TIn, int S, int D, int C, int kMinBlocks>
hipError_t launch_sums_family(const void* k, const void* v, float* records, const Problem& p,
                              hipStream_t stream) {
    using G = Geo<TIn, S, D, C>;
    // Tiles are whole sub-chunks, and a tile's bytes fit a 32-bit buffer range.
    if (p.tile % C != 0) return hipErrorInvalidValue;
    if (int64_t(p.tile) * (S > D ? S : D) * int64_t(sizeof(TIn)) >= (int64_t(1) << 31))
        return hipErrorInvalidValue;
    if (direct_sums_supported(S, D)) return launch_tile_sums_direct(k, v, records, p, stream);
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    tile_sums_mfma_kernel<TIn, S, D, C, kMinBlocks><<<grid, kThreads, G::kSumsLds, stream>>>(
        static_cast<const TIn*>(k), static_cast<const TIn*>(v), records, p.T, p.tile, p.tiles, p.rec);
    return hipGetLastError();
}

template <typename TIn, bool kPrecise, int S, int D, int C, int kMinBlocks, int NW = 4>
hipError_t launch_mfma_family(const void* q, const void* k, const void* v, void* out, float* records,
                              float* state, const Problem& p, hipStream_t stream, Marks* marks) {
    using GO = Geo<TIn, S, D, C, NW, kPrecise>;
    static_assert(GO::kOutputLds <= 160 * 1024, "gfx950 gives a workgroup at most 160 KB of LDS");
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    hipError_t err = launch_sums_family<TIn, S, D, C, kMinBlocks>(k, v, records, p, stream);
    if (err != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    if ((err = launch_tile_scan(records, state, p, stream)) != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    causal_output_mfma_kernel<TIn, S, D, C, kMinBlocks, NW, kPrecise><<<grid, GO::kT, GO::kOutputLds, stream>>>(
        static_cast<const TIn*>(q), static_cast<const TIn*>(k), static_cast<const TIn*>(v),
        static_cast<TIn*>(out), records, p.T, p.tile, p.tiles, p.rec);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (marks) return marks->mark(stream);
    return hipSuccess;
}

template <typename TIn, bool kPrecise = false>
hipError_t dispatch_mfma(const void* q, const void* k, const void* v, void* out, float* records,
                         float* state, const Problem& p, hipStream_t stream, Marks* marks) {
    // S = d = 64: 32-token sub-chunks halve every LDS plane (32 KB per
    // workgroup) so four workgroups share a CU and keep four times the loads
    // in flight; the output pass there is bound by bytes in flight, not math.
    if (p.S == 64 && p.d == 64)
        return launch_mfma_family<TIn, kPrecise, 64, 64, 32,
                                  std::is_same<TIn, float>::value ? RACE_OUT_F32_6464_MINBLOCKS : 4>(
            q, k, v, out, records, state, p, stream, marks);
    if (p.S == 64 && p.d == 128)
        return launch_mfma_family<TIn, kPrecise, 64, 128, 64, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 128 && p.d == 64)
        return launch_mfma_family<TIn, kPrecise, 128, 64, 64, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 128 && p.d == 128)
        return launch_mfma_family<TIn, kPrecise, 128, 128, 64, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 256 && p.d == 64)
        return launch_mfma_family<TIn, kPrecise, 256, 64, 32, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 256 && p.d == 128)
        return launch_mfma_family<TIn, kPrecise, 256, 128, 32, 1, 8>(q, k, v, out, records, state, p, stream,
                                                                       marks);
    return hipErrorInvalidValue;
}

template <typename TIn>
hipError_t dispatch_sums(const void* k, const void* v, float* records, const Problem& p,
                         hipStream_t stream) {
    // The K1 launches of dispatch_mfma, shape for shape.
    if (p.S == 64 && p.d == 64)
        return launch_sums_family<TIn, 64, 64, 32, std::is_same<TIn, float>::value ? RACE_OUT_F32_6464_MINBLOCKS : 4>(
            k, v, records, p, stream);
    if (p.S == 64 && p.d == 128) return launch_sums_family<TIn, 64, 128, 64, 1>(k, v, records, p, stream);
    if (p.S == 128 && p.d == 64) return launch_sums_family<TIn, 128, 64, 64, 1>(k, v, records, p, stream);
    if (p.S == 128 && p.d == 128) return launch_sums_family<TIn, 128, 128, 64, 1>(k, v, records, p, stream);
    if (p.S == 256 && p.d == 64) return launch_sums_family<TIn, 256, 64, 32, 1>(k, v, records, p, stream);
    if (p.S == 256 && p.d == 128) return launch_sums_family<TIn, 256, 128, 32, 1>(k, v, records, p, stream);
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_tile_sums_mfma(const void* k, const void* v, float* records, const Problem& p,
                                 hipStream_t stream) {
    if (p.dtype == RACE_BF16) return dispatch_sums<bf16_t>(k, v, records, p, stream);
    return dispatch_sums<float>(k, v, records, p, stream);
}

int mfma_tiles_per_cu(int S, int d, int dtype, int kernel) {
    if (kernel == RACE_KERNEL_MFMA && direct_output_supported(S, d, dtype))
        return direct_output_tiles_per_cu();
    // fp32 S = d = 64 (the workgroup output pass, four resident per CU):
    // two tiles per CU.  Measured over 2000-step windows at cfg2 (T = 65536):
    // 1024-token tiles 3536 M tokens/s against 3351 for 512 and 2337 for 2048;
    // the hashed module 3051 against 3003.  The longer tiles halve the
    // records and the scan and start half as many workgroups on the same
    // loads.  The others run one or two per CU over two or more rounds; S =
    // 256 prefers longer tiles (fewer 132 KB records to scan).
    if (S == 64 && d == 64 && dtype == RACE_F32) return 2;
    return S >= 256 ? 2 : 4;
}

bool mfma_causal_supported(int S, int d) {
    return (S == 64 || S == 128 || S == 256) && (d == 64 || d == 128);
}

hipError_t launch_causal_mfma(const void* q, const void* k, const void* v, void* out,
                              float* records, float* state, const Problem& p, hipStream_t stream,
                              Marks* marks) {
    if (!mfma_causal_supported(p.S, p.d)) return hipErrorInvalidValue;
    // The register-direct output pass runs when asked for (RACE_KERNEL_MFMA);
    // the automatic choice is the workgroup pass everywhere: at cfg3 (bf16, S
    // = d = 64, T = 2^20, 8192-token tiles) it measured 844 against 864 us,
    // 7286 against 7174 M tokens/s over the whole op.
    if (p.kernel == RACE_KERNEL_MFMA && direct_output_supported(p.S, p.d, p.dtype) &&
        p.tile % 64 == 0) {
        hipError_t err = launch_tile_sums_direct(k, v, records, p, stream);
        if (err != hipSuccess) return err;
        if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
        if ((err = launch_tile_scan(records, state, p, stream)) != hipSuccess) return err;
        if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
        if ((err = launch_causal_output_direct(q, k, v, out, records, p, stream)) != hipSuccess)
            return err;
        return marks ? marks->mark(stream) : hipSuccess;
    }
    if (p.dtype == RACE_BF16 && p.kernel == RACE_KERNEL_MFMA_PRECISE)
        return dispatch_mfma<bf16_t, true>(q, k, v, out, records, state, p, stream, marks);
    if (p.dtype == RACE_BF16)
        return dispatch_mfma<bf16_t>(q, k, v, out, records, state, p, stream, marks);
    return dispatch_mfma<float>(q, k, v, out, records, state, p, stream, marks);
}

}  // namespace race
