// mfma_bwd.hip -- matrix-core (MFMA) kernels of the causal backward for
// S = d = 64 on gfx950, in sub-chunks of 32 tokens.
//
// The function and its VJP are those of causal_bwd.hip (per stream;
// r = 1 / (Abar + eps), W = Q r, g = dOut; in a sub-chunk with prefix state
// (A0, B0) and suffix state (Z1, Y1)):
//     Abar = A0 + tril(1) K,  M = tril(G V^T),  P = tril(W K^T)
//     dQ = r (G B0^T + M K),  alpha = -W dQ
//     dK = V Z1^T + 1 Y1^T + M^T W + triu(1) alpha,   dV = K Z1 + P^T G
//     Z1 += W^T G,  Y1 += 1^T alpha,  B0 += K^T V,  A0 += 1^T K.
// These kernels write exactly the buffers of the vector-ALU ones (dQ, the fp32
// copy of dQ, the running mass per sub-chunk, the suffix records), so the two
// families are interchangeable launch by launch.
//
// Blocks.  The per-bucket function is a sum over buckets of independent
// per-bucket terms, and each term is linear in the value columns, so a
// problem with S and d multiples of 64 is the sum of (S / 64) (d / 64)
// independent S = d = 64 problems: bucket group m (columns 64 m .. of probsQ
// and probsK) with value group h (columns 64 h .. of V and dOut).  Block
// (m, h) gives dQ and dK of bucket group m summed over h, and dV of value
// group h summed over m.  The kernels take one block through BwdBlock: row
// strides of the full tensors and where the block's state sits in the full
// forward records; race_api.hip runs the blocks in a fixed order and the
// kernels add each block's part to fp32 running sums (BwdBlock).  For bf16
// tokens with d = 128 and S = 128 or 256 the walks instead take 128-bucket x
// 128-column blocks with eight waves (causal_bwd_dq_wide_kernel,
// causal_bwd_dkv_wide_kernel): dQ and dK of a block whole, dV summed over the
// blocks; one launch takes the forward walks of every block, with the
// workgroups that read the same V and dOut rows on the same XCD.
//
// Layout.  Workgroups are 4 wave64s; wave w owns bucket block w
// (s = 16 w .. 16 w + 15).  Products use v_mfma_f32_16x16x32_bf16 with the
// permuted contraction order of mfma_common.h, fp32 operands as bf16 hi/lo.
// The running mass is computed with tokens as rows (Abar[i][s]: M = tokens,
// N = buckets), so a lane holds r, W, dQ and alpha at
//     i = 16 bi + 4 g + rr,  s = 16 w + lr        (bi < 2, rr < 4),
// which is also the B operand (column s, contraction over tokens) of
// Z^T += G^T W.  The carried B0 is held transposed, B0^T[c][s] at
// c = 16 cb + 4 g + rr, s = 16 w + lr, which is the B operand (column s,
// contraction over c) of G B0^T; Z^T is held the same way.
// The token tiles K, V, G are staged through LDS as bf16 "R" planes (rows =
// tokens, contraction over features); products that contract over tokens
// read them transposed (ds_read_b64_tr_b16, Plane::frag_tr).  W and Z1 are
// stored the same way, with their first index as rows: W^T [s][i], Z1 [s][c].
#include "mfma_common.h"

namespace race {
namespace {

using namespace mfma;

constexpr int kBC = 32;  // tokens per sub-chunk
constexpr int kBS = 64;  // buckets (S) and value columns (d)
#ifndef RACE_BWD_DQ_BLOCKS
#define RACE_BWD_DQ_BLOCKS 2
#endif
// Resident B1 workgroups per CU: two since dQ is staged through LDS (three
// spill registers there; measured 139 against 170 us at cfg2).
constexpr int kDqBlocks = RACE_BWD_DQ_BLOCKS;
// B1 takes Q's rows of a sub-chunk as whole 16-byte rows into an LDS tile
// (read in the accumulator layout there) rather than 4 (fp32) or 2 (bf16)
// bytes per lane and row straight from global memory: 132 -> 130 us at cfg2,
// 1535 -> 1520 us at the cfg3 shape.  The same in B3 measured no faster at
// cfg2 and 1.5% slower at the cfg3 shape (the Q tile on top of 66 KB of LDS).
#ifndef RACE_BWD_STAGE_Q
#define RACE_BWD_STAGE_Q 1
#endif
constexpr bool kStageQ = RACE_BWD_STAGE_Q != 0;

template <typename TIn>
struct BwdGeo {
    static constexpr bool kSplit = std::is_same<TIn, float>::value;
    static constexpr int E = Elem<TIn>::kPerVec;  // elements per 16-byte load
    using PR = Plane<kSplit, kBS>;                // rows = tokens, k = features
    using PM = Plane<kSplit, kBC>;                // rows = tokens or features, k = tokens
    static constexpr int kRBytes = kBC * PR::kPitch;
    static constexpr int kMBytes = kBC * PM::kPitch;
    static constexpr int kWTBytes = kBS * PM::kPitch;  // W^T [s][i]
    static constexpr int kZBytes = kBS * PR::kPitch;   // Z1 [s][c]
    // B1's dQ tile [kBC][kBS] fp32 staged in LDS (OutTile) and stored as
    // whole rows, as the fp32 copy and (bf16 tokens) converted to dQ at the
    // store (164 -> 139 us at cfg2).  B3 stores dK and dV from registers:
    // staged the same way it measured slower (196 -> 260 us).
    static constexpr int kT32Bytes = kBC * kBS * 4;
    static constexpr int kDqLds = 3 * kRBytes + kMBytes + kT32Bytes;
    // B1 over DV value columns (64, or all 128 of a d = 128 problem at once):
    // V and G planes of DV columns, staged as (kBC / 4) (DV / E) blocks each.
    template <int DV>
    using PV = Plane<kSplit, DV>;
    template <int DV>
    static constexpr int kVBytes = kBC * PV<DV>::kPitch;
    // ... and, staged, Q's rows of the sub-chunk (whole 16-byte rows in,
    // read in the accumulator layout).
    using QT = OutTile<TIn, kBS, kBC>;
    static constexpr int kQTBytes = kBC * QT::kRowBytes;
    template <int DV>
    static constexpr int kDqLdsV = kRBytes + 2 * kVBytes<DV> + kMBytes + kT32Bytes + (kStageQ ? kQTBytes : 0);
    template <int DV>
    static constexpr int kBlkV = (kBC / 4) * (DV / E);
    static constexpr int kDkvLds = 3 * kRBytes + kWTBytes + 2 * kMBytes + kZBytes;
    // Staging: blocks of 4 tokens x E features per tensor.
    static constexpr int kBlk = (kBC / 4) * (kBS / E);   // 128 (fp32) or 64 (bf16)
    static constexpr int kWavesPerTensor = kBlk / 64;    // 2 or 1
    static_assert(kBlk % 64 == 0, "a tensor's blocks fill whole waves");
};

// Raw registers of one staging block: rows 4 a + rr, features b E .. b E + E - 1
// of a tensor whose rows are `ld` elements apart.
template <typename TIn>
struct StageBlock {
    uint4 x[4];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int r0, int a, int b, int ld) {
        constexpr int E = BwdGeo<TIn>::E;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            x[rr] = buf_load16<kPolicyDefault>(rs, ((r0 + 4 * a + rr) * ld + b * E) * int(sizeof(TIn)));
    }
    // R plane: row = token, 4 consecutive features.
    template <typename P>
    __device__ __forceinline__ void store_r(unsigned char* t, int a, int b) const {
        constexpr int E = BwdGeo<TIn>::E;
        constexpr bool kSplit = BwdGeo<TIn>::kSplit;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
            for (int h = 0; h < E / 4; ++h) {
                uint2 hi, lo;
                split4<kSplit>(Elem<TIn>::get(x[rr], 4 * h), Elem<TIn>::get(x[rr], 4 * h + 1),
                               Elem<TIn>::get(x[rr], 4 * h + 2), Elem<TIn>::get(x[rr], 4 * h + 3), hi,
                               lo);
                P::put4(t, 4 * a + rr, b * E + 4 * h, hi, lo);
            }
    }
};

template <typename TIn>
__device__ __forceinline__ float load1(__amdgpu_buffer_rsrc_t r, int elem) {
    if constexpr (std::is_same<TIn, float>::value) {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, elem * 4, 0, 0));
    } else {
        return __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b16(r, elem * 2, 0, 0)) << 16);
    }
}

template <typename TIn>
__device__ __forceinline__ void store1(__amdgpu_buffer_rsrc_t r, int elem, float x) {
    if constexpr (std::is_same<TIn, float>::value) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, elem * 4, 0, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b16(uint16_t(pack2(x, 0.f) & 0xffffu), r, elem * 2, 0, 0);
    }
}

// Eight fp32 values (permuted-k order) to bf16 hi/lo fragments.
template <bool kSplit>
__device__ __forceinline__ void split8v(const f32x4& a, const f32x4& b, bf16x8& hi, bf16x8& lo) {
    uint2 h0, l0, h1, l1;
    split4<kSplit>(a[0], a[1], a[2], a[3], h0, l0);
    split4<kSplit>(b[0], b[1], b[2], b[3], h1, l1);
    hi = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
    if constexpr (kSplit) lo = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
}

// ---------------------------------------------------------------------------
// B1, forward walk of one (tile, stream): dQ, its fp32 copy, the running mass
// at every sub-chunk start, and the tile's suffix totals Z = sum W (x) g,
// Y = sum alpha into its record.  For fp32 tokens the fp32 copy is the only
// dQ output (the caller passes its dQ as dq32 and no dQ).
template <typename TIn, bool kSums, int DV>
__global__ __launch_bounds__(kThreads, kDqBlocks) void causal_bwd_dq_mfma_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    const TIn* __restrict__ g, TIn* __restrict__ dQ, float* __restrict__ dq32,
    float* __restrict__ apre, const float* __restrict__ fwd_records,
    float* __restrict__ bwd_records, int64_t T, int tile, int64_t tiles, int64_t rec,
    BwdBlock blk) {
    using G = BwdGeo<TIn>;
    using PR = typename G::PR;
    using PM = typename G::PM;
    using PV = typename G::template PV<DV>;  // V and G planes: DV value columns
    constexpr bool kSplit = G::kSplit;
    constexpr int NCB = DV / 16;             // value column blocks
    constexpr int NKV = DV / 32;             // contraction steps over the value columns
    static_assert(DV == kBS || DV == 2 * kBS, "64 or 128 value columns");
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Ks = lds;
    unsigned char* Vs = Ks + G::kRBytes;
    unsigned char* Gs = Vs + G::template kVBytes<DV>;
    unsigned char* Ms = Gs + G::template kVBytes<DV>;
    unsigned char* D32s = Ms + G::kMBytes;
    unsigned char* Qt = D32s + G::kT32Bytes;  // Q rows (kStageQ)
    using T32 = OutTile<float, kBS, kBC>;
    using QT = typename G::QT;

    const int tid = threadIdx.x, l = tid & 63, gq = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
    const int64_t base = n * T + t_begin;
    constexpr int es = int(sizeof(TIn));
    const int ldq = blk.ldq, ldv = blk.ldv;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + base * ldq, int64_t(rows) * ldq * es);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + base * ldq, int64_t(rows) * ldq * es);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + base * ldv, int64_t(rows) * ldv * es);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(g + base * ldv, int64_t(rows) * ldv * es);
    const __amdgpu_buffer_rsrc_t dqr = make_rsrc(dQ ? dQ + base * kBS : nullptr,
                                                 dQ ? int64_t(rows) * kBS * es : 0);
    const __amdgpu_buffer_rsrc_t d32r = make_rsrc(dq32 + base * kBS, int64_t(rows) * kBS * 4);
    // Several blocks: dQ's running sum and, for the last addend of bf16
    // tokens, the caller's dQ (rows of ldq).
    const __amdgpu_buffer_rsrc_t aqr =
        make_rsrc(blk.acc_q ? blk.acc_q + base * ldq : nullptr, blk.acc_q ? int64_t(rows) * ldq * 4 : 0);
    const __amdgpu_buffer_rsrc_t fqr = make_rsrc(
        blk.fin_q ? static_cast<TIn*>(blk.fin_q) + base * ldq : nullptr, blk.fin_q ? int64_t(rows) * ldq * es : 0);

    // Prefix state at the tile start, transposed: B0^T[16 cb + 4 g + rr][16 w + lr]
    // (the block's rows and columns of the forward record).
    const float* fr = fwd_records + (n * tiles + ti) * blk.fwd_rec;
    f32x4 b0t[NCB], zt[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            b0t[cb][rr] = fr[int64_t(blk.s0 + 16 * w + lr) * blk.fwd_d + blk.c0 + 16 * cb + 4 * gq + rr];
            zt[cb][rr] = 0.f;
        }
    float a0 = fr[blk.fwd_a + blk.s0 + 16 * w + lr];
    float ypart = 0.f;
    const bf16x8 tri0 = tril_frag(0, gq, lr), tri1 = tril_frag(16, gq, lr);

    // Staging: this wave's tensor (K, V or G) and block.  Slot e = tid +
    // 256 s counts K's blocks, then V's, then G's (kBlkV each, DV wide);
    // every boundary is a multiple of 64, so a wave stages one tensor.
    constexpr int kBlkK = G::kBlk, kBlkV = G::template kBlkV<DV>;
    constexpr int kSlots = (kBlkK + 2 * kBlkV + kThreads - 1) / kThreads;
    static_assert(kBlkK % 64 == 0 && kBlkV % 64 == 0, "a wave stages one tensor");
    auto slot_tensor = [&](int s) {
        const int e = __builtin_amdgcn_readfirstlane(tid + s * kThreads - l);
        return e < kBlkK ? 0 : e < kBlkK + kBlkV ? 1 : e < kBlkK + 2 * kBlkV ? 2 : 3;
    };
    auto slot_block = [&](int s, int tensor) {
        const int e = tid + s * kThreads;
        return tensor == 0 ? e : tensor == 1 ? e - kBlkK : e - kBlkK - kBlkV;
    };
    StageBlock<TIn> st[kSlots];
    auto stage_load = [&](int r0) {
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            const int tensor = slot_tensor(s);
            if (tensor >= 3) continue;
            const int blk = slot_block(s, tensor);
            // One call per tensor: choosing the buffer and the row stride
            // with conditional expressions put the captured locals (and the
            // staging registers) in scratch memory, 3x slower.
            if (tensor == 0)
                st[s].load(kr, r0, blk / (kBS / G::E), blk % (kBS / G::E), ldq);
            else if (tensor == 1)
                st[s].load(vr, r0, blk / (DV / G::E), blk % (DV / G::E), ldv);
            else
                st[s].load(gr, r0, blk / (DV / G::E), blk % (DV / G::E), ldv);
        }
    };
    auto stage_store = [&]() {
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            const int tensor = slot_tensor(s);
            if (tensor >= 3) continue;
            const int blk = slot_block(s, tensor);
            if (tensor == 0)
                st[s].template store_r<PR>(Ks, blk / (kBS / G::E), blk % (kBS / G::E));
            else
                st[s].template store_r<PV>(tensor == 1 ? Vs : Gs, blk / (DV / G::E), blk % (DV / G::E));
        }
    };
    // Q at this lane's (i, s) positions, or (kStageQ) the sub-chunk's rows
    // as 16-byte chunks: chunk c = tid + i kThreads is row c / QT::kChunks.
    constexpr int kQC = kBC * QT::kChunks;
    constexpr int kQPer = (kQC + kThreads - 1) / kThreads;
    static_assert(kQC % kThreads == 0, "whole chunks per thread");
    float qreg[2][4];
    uint4 qx[kQPer];
    auto load_q = [&](int r0) {
        if constexpr (kStageQ) {
#pragma unroll
            for (int i = 0; i < kQPer; ++i) {
                const int c = tid + i * kThreads;
                qx[i] = buf_load16<kPolicyDefault>(
                    qr, ((r0 + c / QT::kChunks) * ldq + (c % QT::kChunks) * G::E) * int(sizeof(TIn)));
            }
        } else {
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    qreg[bi][rr] = load1<TIn>(qr, (r0 + 16 * bi + 4 * gq + rr) * ldq + 16 * w + lr);
        }
    };

    const int subs = tile / kBC;
    float* ap = apre + (n * tiles + ti) * int64_t(subs) * kBS;
    // The previous sub-chunk's gradient tiles are stored after the first
    // barrier of the next one (and after the loop).
    // The fp32 tile's 16-byte chunks go to dq32 as they are and, for bf16
    // tokens, to dQ as 8-byte bf16 chunks (chunk q holds elements 4 q .. 4 q + 3
    // of the row-major tile).
    // dQ's running sum over the rows of the sub-chunk being computed,
    // requested with its tokens and added at the flush one sub-chunk later
    // (read where it is added, every flush waited a full memory round trip).
    constexpr int kAccPer = T32::template Chunks<kThreads>::kPer;
    f32x4 aq_next[kAccPer], aq_cur[kAccPer];
    // (The first addend reads nothing: an empty view returns zeros.)
    const __amdgpu_buffer_rsrc_t aq_rd = make_rsrc(blk.acc_q && !blk.q_first ? blk.acc_q + base * ldq : nullptr,
                                                   blk.acc_q && !blk.q_first ? int64_t(rows) * ldq * 4 : 0);
    auto load_acc_q = [&](int r0) {
#pragma unroll
        for (int i = 0; i < kAccPer; ++i) {
            const int qi = tid + i * kThreads;
            const int off = (r0 + (qi >> 4)) * ldq + 4 * (qi & 15);
            aq_next[i] = __builtin_bit_cast(f32x4, buf_load16<kPolicyDefault>(aq_rd, off * 4));
        }
    };
#pragma unroll
    for (int i = 0; i < kAccPer; ++i) aq_next[i] = aq_cur[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto flush = [&](int r0) {
        typename T32::template Chunks<kThreads> c32;
        T32::template read<kThreads>(D32s, c32);
        if constexpr (!kSplit) {
            if (dQ) {
#pragma unroll
                for (int i = 0; i < T32::template Chunks<kThreads>::kPer; ++i) {
                    const int qi = tid + i * kThreads;
                    const uint4 x = c32.x[i];
                    __builtin_amdgcn_raw_buffer_store_b64(
                        u32x2{pack2(__uint_as_float(x.x), __uint_as_float(x.y)),
                              pack2(__uint_as_float(x.z), __uint_as_float(x.w))},
                        dqr, r0 * kBS * 2 + 8 * qi, 0, kPolicyDefault);
                }
            }
        }
        T32::template write<kPolicyDefault, kThreads>(c32, d32r, r0);
        if (kSums && (blk.acc_q || blk.fin_q)) {
            // The block's part into dQ's running sum (rows outside the tile,
            // and all rows of the first flush, fall outside the views); a
            // first addend with fin_q (a walk over every value column) is
            // dQ itself.
#pragma unroll
            for (int i = 0; i < T32::template Chunks<kThreads>::kPer; ++i) {
                const int qi = tid + i * kThreads;
                const int off = (r0 + (qi >> 4)) * ldq + 4 * (qi & 15);
                f32x4 t = __builtin_bit_cast(f32x4, c32.x[i]);
                if (!blk.q_first) t = t + aq_cur[i];
                if (blk.fin_q)
                    store4<TIn, kPolicyDefault>(fqr, off * es, t);
                else
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, t), aqr, off * 4, 0,
                                                           kPolicyDefault);
            }
        }
    };
    stage_load(0);
    load_q(0);
    int r0 = 0;
    for (; r0 < rows; r0 += kBC) {
        __syncthreads();
        stage_store();
        float qc[2][4];
        if constexpr (kStageQ) {
#pragma unroll
            for (int i = 0; i < kQPer; ++i) *reinterpret_cast<uint4*>(Qt + QT::chunk_at(tid + i * kThreads)) = qx[i];
        } else {
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) qc[bi][rr] = qreg[bi][rr];
        }
        stage_load(r0 + kBC);  // past the tile: zeros, never used
        load_q(r0 + kBC);
        if constexpr (kSums) {
#pragma unroll
            for (int i = 0; i < kAccPer; ++i) aq_cur[i] = aq_next[i];
            load_acc_q(r0);
        }
        // After the prefetch: a wait for those loads then leaves these stores
        // in flight (one counter covers both, in issue order).  Unconditional:
        // at r0 = 0 the offsets are negative, outside the buffer ranges, and
        // the stores are dropped.  With `if (r0 > 0)` the compiler peeled the
        // first iteration, and the bf16 build of that peel returned wrong dQ
        // rows 16..31 (tests/test_gpu_causal_bwd.py covers it).
        flush(r0 - kBC);
        if (gq == 0) ap[(r0 / kBC) * kBS + 16 * w + lr] = a0;
        __syncthreads();

        // 1: Abar[i][s] = A0[s] + sum_{j <= i} K[j][s], r and W.
        if constexpr (kStageQ) {
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const unsigned char* qp = Qt + QT::at(16 * bi + 4 * gq + rr, (16 * w + lr) * int(sizeof(TIn)));
                    if constexpr (std::is_same<TIn, float>::value)
                        qc[bi][rr] = *reinterpret_cast<const float*>(qp);
                    else
                        qc[bi][rr] = to_f32(*reinterpret_cast<const bf16_t*>(qp));
                }
        }
        bf16x8 kh, kl;
        PR::frag_tr(Ks, 0, 16 * w, gq, lr, kh, kl);
        f32x4 ab[2];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            f32x4 acc = {a0, a0, a0, a0};
            const bf16x8& tf = bi == 0 ? tri0 : tri1;
            if constexpr (kSplit) acc = mfma16(tf, kl, acc);
            ab[bi] = mfma16(tf, kh, acc);
        }
        a0 = __shfl(ab[1][3], 48 + lr);  // inclusive mass at the last token
        f32x4 rv[2], wv[2];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                rv[bi][rr] = __builtin_amdgcn_rcpf(ab[bi][rr] + kEps);
                wv[bi][rr] = qc[bi][rr] * rv[bi][rr];
            }

        // 2: M^T blocks (j-block, i-block) = V G^T, j <= i: (0,0), (0,1), (1,1) on waves 0..2.
        f32x4 mt = {0.f, 0.f, 0.f, 0.f};
        const int mbj = w == 2 ? 1 : 0, mbi = w >= 1 ? 1 : 0;
        if (w < 3) {
#pragma unroll
            for (int kk = 0; kk < NKV; ++kk) {
                bf16x8 ah, al, bh, bl;
                PV::frag(Vs, 16 * mbj + lr, kk, gq, ah, al);
                PV::frag(Gs, 16 * mbi + lr, kk, gq, bh, bl);
                mt = mfma3<kSplit>(ah, al, bh, bl, mt);
            }
            if (mbj == mbi) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (4 * gq + rr > lr) mt[rr] = 0.f;
            }
        }
        if (w < 3) {
            uint2 hi, lo;
            split4<kSplit>(mt[0], mt[1], mt[2], mt[3], hi, lo);
            PM::put4(Ms, 16 * mbi + lr, 16 * mbj + 4 * gq, hi, lo);
        }
        __syncthreads();

        // 3: U = G B0^T + M K;  dQ = r U;  alpha = -W dQ.
        f32x4 u[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int kk = 0; kk < NKV; ++kk) {
            bf16x8 bh, bl;
            split8v<kSplit>(b0t[2 * kk], b0t[2 * kk + 1], bh, bl);
#pragma unroll
            for (int bi = 0; bi < 2; ++bi) {
                bf16x8 gh, gl;
                PV::frag(Gs, 16 * bi + lr, kk, gq, gh, gl);
                u[bi] = mfma3<kSplit>(gh, gl, bh, bl, u[bi]);
            }
        }
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            bf16x8 mh, ml;
            PM::frag(Ms, 16 * bi + lr, 0, gq, mh, ml);
            if (bi == 0) {
                // Tokens 16..31 of the first block's row are above the diagonal.
#pragma unroll
                for (int e = 4; e < 8; ++e) {
                    mh[e] = __bf16(0.0f);
                    if constexpr (kSplit) ml[e] = __bf16(0.0f);
                }
            }
            u[bi] = mfma3<kSplit>(mh, ml, kh, kl, u[bi]);
        }
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const float dqv = rv[bi][rr] * u[bi][rr];
                T32::put1(D32s, 16 * bi + 4 * gq + rr, 16 * w + lr, dqv);
                ypart += -wv[bi][rr] * dqv;
            }

        // 4: Z^T += G^T W (contraction over the sub-chunk's tokens).
        bf16x8 wh, wl;
        split8v<kSplit>(wv[0], wv[1], wh, wl);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            bf16x8 gh, gl;
            PV::frag_tr(Gs, 0, 16 * cb, gq, lr, gh, gl);
            zt[cb] = mfma3<kSplit>(gh, gl, wh, wl, zt[cb]);
        }
        // 5: B0^T += V^T K.
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            bf16x8 vh, vl;
            PV::frag_tr(Vs, 0, 16 * cb, gq, lr, vh, vl);
            b0t[cb] = mfma3<kSplit>(vh, vl, kh, kl, b0t[cb]);
        }
    }
    __syncthreads();
    if constexpr (kSums) {
#pragma unroll
        for (int i = 0; i < kAccPer; ++i) aq_cur[i] = aq_next[i];
    }
    if (r0 > 0) flush(r0 - kBC);

    // Suffix totals of this tile: Z[s][c] (record layout B[s][c]) and Y[s],
    // one 64 x 64 record per value group h (records of group h start h N
    // tiles records in); Y, the totals of alpha over all DV columns, goes to
    // group 0's record and group 1's holds zero.
    float y = ypart + __shfl_xor(ypart, 16);
    y = y + __shfl_xor(y, 32);
#pragma unroll
    for (int h = 0; h < DV / kBS; ++h) {
        float* br = bwd_records + (int64_t(h) * gridDim.y * tiles + n * tiles + ti) * rec;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                br[(16 * w + lr) * kBS + 16 * cb + 4 * gq + rr] = zt[4 * h + cb][rr];
        if (gq == 0) br[kBS * kBS + 16 * w + lr] = h == 0 ? y : 0.f;
    }
}

// Upper-triangular ones as an A operand: element e of lane (g, lr) is
// (i' >= j') with i' = 4 g + e % 4 + 16 (e / 4) (contraction index) and row
// j' = off + lr.
__device__ __forceinline__ bf16x8 triu_frag(int off, int g, int lr) {
    bf16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (4 * g + (e & 3) + 16 * (e >> 2) >= off + lr) ? __bf16(1.0f) : __bf16(0.0f);
    return f;
}

// ---------------------------------------------------------------------------
// B3, backward walk of one (tile, stream) from the suffix state at the tile
// end: dK (wave w: buckets 16 w ..) and dV (wave w: value columns 16 w ..).
// Per sub-chunk, with the suffix state Z1 after it:
//   1. Abar, r, W (as B1, from the running mass saved by B1); alpha = -W dQ;
//      W also goes to an R plane (rows = tokens) for P
//   2. M = tril(G V^T) and P = tril(W K^T) into T-oriented planes (rows = j)
//   3. dK = V Z1^T + M^T W + triu(1) alpha + Y1        (Z1^T from registers)
//   4. dV = K Z1 + P^T G                                (Z1 from an LDS plane)
//   5. Z1^T += G^T W, Y1 += 1^T alpha
template <typename TIn, bool kSums>
__global__ __launch_bounds__(kThreads, 2) void causal_bwd_dkv_mfma_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    const TIn* __restrict__ g, const float* __restrict__ dq32, const float* __restrict__ apre,
    const float* __restrict__ suffix_records, TIn* __restrict__ dK, TIn* __restrict__ dV,
    int64_t T, int tile, int64_t tiles, int64_t rec, BwdBlock blk) {
    using G = BwdGeo<TIn>;
    using PR = typename G::PR;
    using PM = typename G::PM;
    constexpr bool kSplit = G::kSplit;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Ks = lds;
    unsigned char* Vs = Ks + G::kRBytes;
    unsigned char* Gs = Vs + G::kRBytes;
    unsigned char* WT = Gs + G::kRBytes;     // W^T: rows s, elements i
    unsigned char* MT = WT + G::kWTBytes;    // rows j, contraction over i
    unsigned char* PTp = MT + G::kMBytes;    // rows j, contraction over i
    unsigned char* Zr = PTp + G::kMBytes;    // Z1: rows s, elements c

    const int tid = threadIdx.x, l = tid & 63, gq = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
    const int64_t base = n * T + t_begin;
    constexpr int es = int(sizeof(TIn));
    const int ldq = blk.ldq, ldv = blk.ldv;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + base * ldq, int64_t(rows) * ldq * es);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + base * ldq, int64_t(rows) * ldq * es);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v + base * ldv, int64_t(rows) * ldv * es);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(g + base * ldv, int64_t(rows) * ldv * es);
    // Without the alpha terms dQ is not read: an empty view returns zeros.
    const __amdgpu_buffer_rsrc_t d32r =
        make_rsrc(blk.alpha ? dq32 + base * kBS : nullptr, blk.alpha ? int64_t(rows) * kBS * 4 : 0);
    const __amdgpu_buffer_rsrc_t dkr = make_rsrc(dK ? dK + base * kBS : nullptr,
                                                 dK ? int64_t(rows) * kBS * es : 0);
    const __amdgpu_buffer_rsrc_t dvr = make_rsrc(dV ? dV + base * kBS : nullptr,
                                                 dV ? int64_t(rows) * kBS * es : 0);
    // Several blocks: the running sums of dK (rows of ldq) and dV (rows of
    // ldv), and the caller's gradients for the last addend of bf16 tokens.
    const __amdgpu_buffer_rsrc_t akr =
        make_rsrc(blk.acc_k ? blk.acc_k + base * ldq : nullptr, blk.acc_k ? int64_t(rows) * ldq * 4 : 0);
    const __amdgpu_buffer_rsrc_t avr =
        make_rsrc(blk.acc_v ? blk.acc_v + base * ldv : nullptr, blk.acc_v ? int64_t(rows) * ldv * 4 : 0);
    const __amdgpu_buffer_rsrc_t fkr = make_rsrc(
        blk.fin_k ? static_cast<TIn*>(blk.fin_k) + base * ldq : nullptr, blk.fin_k ? int64_t(rows) * ldq * es : 0);
    const __amdgpu_buffer_rsrc_t fvr = make_rsrc(
        blk.fin_v ? static_cast<TIn*>(blk.fin_v) + base * ldv : nullptr, blk.fin_v ? int64_t(rows) * ldv * es : 0);
    // One gradient value at (row, col): as it is (one block), or added to its
    // running sum (blocks).
    // `sum` is the running sum at (row, col), prefetched with the sub-chunk's
    // tokens (read where it is added, the loads waited a full memory round
    // trip in every sub-chunk).
    auto put_grad = [&](__amdgpu_buffer_rsrc_t own, __amdgpu_buffer_rsrc_t accr, __amdgpu_buffer_rsrc_t finr,
                        bool has_acc, bool first, bool has_fin, int ld, int row, int col, float x,
                        float sum) {
        if (!kSums) {
            store1<TIn>(own, row * kBS + col, x);
        } else if (has_acc) {
            const int off = row * ld + col;
            if (!first) x += sum;
            if (has_fin)
                store1<TIn>(finr, off, x);
            else
                store1<float>(accr, off, x);
        }
    };
    // Read views of the running sums (empty for a first addend: zeros).
    const __amdgpu_buffer_rsrc_t ak_rd = make_rsrc(blk.acc_k && !blk.k_first ? blk.acc_k + base * ldq : nullptr,
                                                   blk.acc_k && !blk.k_first ? int64_t(rows) * ldq * 4 : 0);
    const __amdgpu_buffer_rsrc_t av_rd = make_rsrc(blk.acc_v && !blk.v_first ? blk.acc_v + base * ldv : nullptr,
                                                   blk.acc_v && !blk.v_first ? int64_t(rows) * ldv * 4 : 0);
    float ksum_n[2][4], vsum_n[2][4];
    auto load_sums = [&](int r0) {
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = r0 + 16 * bj + 4 * gq + rr;
                ksum_n[bj][rr] = load1<float>(ak_rd, row * ldq + 16 * w + lr);
                // fp32 tokens: the dV sum is read where it is added (both
                // prefetched, the fp32 kernel's registers spill).
                if constexpr (!kSplit)
                    vsum_n[bj][rr] = load1<float>(av_rd, row * ldv + 16 * w + lr);
                else
                    vsum_n[bj][rr] = 0.f;
            }
    };

    // Suffix state at the tile end: Z1^T[16 cb + 4 g + rr][16 w + lr], Y1[16 w + lr].
    const float* sr = suffix_records + (n * tiles + ti) * rec;
    f32x4 zt[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) zt[cb][rr] = sr[(16 * w + lr) * kBS + 16 * cb + 4 * gq + rr];
    float y1 = blk.alpha ? sr[kBS * kBS + 16 * w + lr] : 0.f;
    const bf16x8 tri0 = tril_frag(0, gq, lr), tri1 = tril_frag(16, gq, lr);
    const bf16x8 up0 = triu_frag(0, gq, lr), up1 = triu_frag(16, gq, lr);

    const int nslots = (3 * G::kBlk + kThreads - 1) / kThreads;
    auto slot_tensor = [&](int s) { return __builtin_amdgcn_readfirstlane((tid + s * kThreads) / G::kBlk); };
    StageBlock<TIn> st[2];
    auto stage_load = [&](int r0) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            if (s >= nslots) break;
            const int tensor = slot_tensor(s);
            if (tensor >= 3) continue;
            const int blk = (tid + s * kThreads) % G::kBlk;
            const int a = blk / (kBS / G::E), b = blk % (kBS / G::E);
            // One call per tensor: choosing the buffer and the row stride
            // with conditional expressions put the captured locals (and the
            // staging registers) in scratch memory, 3x slower.
            if (tensor == 0)
                st[s].load(kr, r0, a, b, ldq);
            else if (tensor == 1)
                st[s].load(vr, r0, a, b, ldv);
            else
                st[s].load(gr, r0, a, b, ldv);
        }
    };
    auto stage_store = [&]() {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            if (s >= nslots) break;
            const int tensor = slot_tensor(s);
            if (tensor >= 3) continue;
            const int blk = (tid + s * kThreads) % G::kBlk;
            const int a = blk / (kBS / G::E), b = blk % (kBS / G::E);
            st[s].template store_r<PR>(tensor == 0 ? Ks : tensor == 1 ? Vs : Gs, a, b);
        }
    };
    float qreg[2][4], dreg[2][4];
    auto load_qd = [&](int r0) {
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = r0 + 16 * bi + 4 * gq + rr;
                qreg[bi][rr] = load1<TIn>(qr, row * ldq + 16 * w + lr);
                dreg[bi][rr] = load1<float>(d32r, row * kBS + 16 * w + lr);
            }
    };

    const int subs = tile / kBC;
    const float* ap = apre + (n * tiles + ti) * int64_t(subs) * kBS + 16 * w + lr;
    const int last = ((rows - 1) / kBC) * kBC;
    // The running mass at a sub-chunk's start is prefetched with its tokens:
    // loaded where it is used, its wait would also wait for the prefetch of
    // the next sub-chunk issued just before it.
    float a0n;
    stage_load(last);
    load_qd(last);
    if constexpr (kSums) load_sums(last);
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            if constexpr (!kSums) ksum_n[bj][rr] = vsum_n[bj][rr] = 0.f;
    a0n = ap[(last / kBC) * kBS];
    for (int r0 = last; r0 >= 0; r0 -= kBC) {
        __syncthreads();
        stage_store();
        float qc[2][4], dc[2][4], ksum[2][4], vsum[2][4];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                qc[bi][rr] = qreg[bi][rr];
                dc[bi][rr] = dreg[bi][rr];
                ksum[bi][rr] = ksum_n[bi][rr];
                vsum[bi][rr] = vsum_n[bi][rr];
            }
        const float a0 = a0n;
        if (r0 > 0) {
            stage_load(r0 - kBC);
            load_qd(r0 - kBC);
            if constexpr (kSums) load_sums(r0 - kBC);
            a0n = ap[(r0 / kBC - 1) * kBS];
        }
        // Z1 (the suffix state after this sub-chunk) as a plane for dV: row s,
        // four consecutive c per lane.
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            uint2 hi, lo;
            split4<kSplit>(zt[cb][0], zt[cb][1], zt[cb][2], zt[cb][3], hi, lo);
            PR::put4(Zr, 16 * w + lr, 16 * cb + 4 * gq, hi, lo);
        }
        __syncthreads();

        // 1: Abar, r, W, alpha; W^T into its plane (row s, four consecutive i).
        bf16x8 kh, kl;
        PR::frag_tr(Ks, 0, 16 * w, gq, lr, kh, kl);
        f32x4 wv[2], al[2];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            f32x4 acc = {a0, a0, a0, a0};
            const bf16x8& tf = bi == 0 ? tri0 : tri1;
            if constexpr (kSplit) acc = mfma16(tf, kl, acc);
            acc = mfma16(tf, kh, acc);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                wv[bi][rr] = qc[bi][rr] * __builtin_amdgcn_rcpf(acc[rr] + kEps);
                al[bi][rr] = -wv[bi][rr] * dc[bi][rr];
            }
            uint2 hi, lo;
            split4<kSplit>(wv[bi][0], wv[bi][1], wv[bi][2], wv[bi][3], hi, lo);
            PM::put4(WT, 16 * w + lr, 16 * bi + 4 * gq, hi, lo);
        }
        __syncthreads();

        // 2: M blocks (i-block, j-block) on waves 0..2, P blocks on waves 1..3,
        //    blocks (0,0), (1,0), (1,1); written with rows j.
        {
            const int mb = w, pb = w - 1;  // block index 0..2
            f32x4 m = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
            if (mb < 3) {
                const int bi = mb >= 1 ? 1 : 0, bj = mb == 2 ? 1 : 0;
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    bf16x8 ah, alo, bh, bl;
                    PR::frag(Gs, 16 * bi + lr, kk, gq, ah, alo);
                    PR::frag(Vs, 16 * bj + lr, kk, gq, bh, bl);
                    m = mfma3<kSplit>(ah, alo, bh, bl, m);
                }
                if (bi == bj) {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        if (lr > 4 * gq + rr) m[rr] = 0.f;
                }
                uint2 hi, lo;
                split4<kSplit>(m[0], m[1], m[2], m[3], hi, lo);
                PM::put4(MT, 16 * bj + lr, 16 * bi + 4 * gq, hi, lo);
            }
            if (pb >= 0) {
                const int bi = pb >= 1 ? 1 : 0, bj = pb == 2 ? 1 : 0;
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    bf16x8 ah, alo, bh, bl;
                    PM::frag_tr(WT, 32 * kk, 16 * bi, gq, lr, ah, alo);
                    PR::frag(Ks, 16 * bj + lr, kk, gq, bh, bl);
                    pacc = mfma3<kSplit>(ah, alo, bh, bl, pacc);
                }
                if (bi == bj) {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        if (lr > 4 * gq + rr) pacc[rr] = 0.f;
                }
                uint2 hi, lo;
                split4<kSplit>(pacc[0], pacc[1], pacc[2], pacc[3], hi, lo);
                PM::put4(PTp, 16 * bj + lr, 16 * bi + 4 * gq, hi, lo);
            }
        }
        __syncthreads();

        bf16x8 wh, wl, ah2, al2;
        split8v<kSplit>(wv[0], wv[1], wh, wl);
        split8v<kSplit>(al[0], al[1], ah2, al2);
        // 3: dK[j][s] for s-block w.
        f32x4 dk[2];
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) dk[bj] = f32x4{y1, y1, y1, y1};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8 zh, zl;
            split8v<kSplit>(zt[2 * kk], zt[2 * kk + 1], zh, zl);
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
                bf16x8 vh, vl;
                PR::frag(Vs, 16 * bj + lr, kk, gq, vh, vl);
                dk[bj] = mfma3<kSplit>(vh, vl, zh, zl, dk[bj]);
            }
        }
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            bf16x8 mh, ml;
            PM::frag(MT, 16 * bj + lr, 0, gq, mh, ml);
            if (bj == 1) {
                // Tokens i < 16 of the second j-block are above the diagonal.
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    mh[e] = __bf16(0.0f);
                    if constexpr (kSplit) ml[e] = __bf16(0.0f);
                }
            }
            dk[bj] = mfma3<kSplit>(mh, ml, wh, wl, dk[bj]);
            const bf16x8& uf = bj == 0 ? up0 : up1;
            if constexpr (kSplit) dk[bj] = mfma16(uf, al2, dk[bj]);
            dk[bj] = mfma16(uf, ah2, dk[bj]);
        }
        // The stores are unconditional (a gradient not asked for has an empty
        // buffer view, which drops them): with one path through the loop the
        // compiler counts them, and the waits for the prefetched sub-chunk
        // at the loop's end leave them in flight.
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                put_grad(dkr, akr, fkr, blk.acc_k != nullptr, blk.k_first, blk.fin_k != nullptr, ldq,
                         r0 + 16 * bj + 4 * gq + rr, 16 * w + lr, dk[bj][rr], ksum[bj][rr]);
        // 4: dV[j][c] for c-block w.
        {
            f32x4 dv[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                bf16x8 zh, zl;
                PR::frag_tr(Zr, 32 * kk, 16 * w, gq, lr, zh, zl);
#pragma unroll
                for (int bj = 0; bj < 2; ++bj) {
                    bf16x8 kh2, kl2;
                    PR::frag(Ks, 16 * bj + lr, kk, gq, kh2, kl2);
                    dv[bj] = mfma3<kSplit>(kh2, kl2, zh, zl, dv[bj]);
                }
            }
            bf16x8 gh, gl;
            PR::frag_tr(Gs, 0, 16 * w, gq, lr, gh, gl);
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
                bf16x8 ph, pl;
                PM::frag(PTp, 16 * bj + lr, 0, gq, ph, pl);
                if (bj == 1) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ph[e] = __bf16(0.0f);
                        if constexpr (kSplit) pl[e] = __bf16(0.0f);
                    }
                }
                dv[bj] = mfma3<kSplit>(ph, pl, gh, gl, dv[bj]);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    put_grad(dvr, avr, fvr, blk.acc_v != nullptr, blk.v_first, blk.fin_v != nullptr, ldv,
                             r0 + 16 * bj + 4 * gq + rr, 16 * w + lr, dv[bj][rr],
                             kSplit ? load1<float>(av_rd, (r0 + 16 * bj + 4 * gq + rr) * ldv + 16 * w + lr)
                                    : vsum[bj][rr]);
            }
        }
        // 5: the suffix state before this sub-chunk.
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            bf16x8 gh, gl;
            PR::frag_tr(Gs, 0, 16 * cb, gq, lr, gh, gl);
            zt[cb] = mfma3<kSplit>(gh, gl, wh, wl, zt[cb]);
        }
        float ys = 0.f;
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) ys += al[bi][rr];
        ys = ys + __shfl_xor(ys, 16);
        ys = ys + __shfl_xor(ys, 32);
        y1 += ys;
    }
}

// ---------------------------------------------------------------------------
// B3 over a 128 x 128 block (bf16 tokens, d = 128): two 64-bucket groups
// (g2 = 0, 1: buckets 64 g2 .. of the block) and every value column in one
// backward walk, eight waves.  Wave w owns buckets 16 w .. 16 w + 15 of the
// block (dK, W, alpha, the carried Z1^T columns) and value columns 16 w ..
// 16 w + 15 (dV).  The steps are those of causal_bwd_dkv_mfma_kernel with
// the contractions over buckets and value columns four 32-wide steps long.
// dK of the block is complete (every value column is in the walk) and goes
// to the caller's dK; dV, a sum over the blocks of a problem, goes through
// its fp32 running sum unless the block is the only one.
constexpr int kWideS = 128, kWideD = 128, kWideWaves = 8, kWideThreads = 64 * kWideWaves;
// Sub-chunks of operands the block forward walk keeps in flight in
// registers.  Two measured slower at cfg5 (661-674 against 642-653 us per
// walk, two alternating runs on one box, 256 VGPRs): the walk is not waiting
// on its loads.
#ifndef RACE_BWD_WIDE_DQ_DEPTH
#define RACE_BWD_WIDE_DQ_DEPTH 1
#endif

struct WideGeo {
    using PR = Plane<false, 128>;  // rows = tokens (or buckets), k = buckets or value columns
    using PM = Plane<false, kBC>;  // k = tokens
    static constexpr int kRBytes = kBC * PR::kPitch;
    static constexpr int kWTBytes = kWideS * PM::kPitch;  // W^T [s][i]
    static constexpr int kMBytes = kBC * PM::kPitch;
    static constexpr int kZBytes = kWideS * PR::kPitch;   // Z1 [s][c]
    static constexpr int kLds = 3 * kRBytes + kWTBytes + 2 * kMBytes + kZBytes;
    using QT = OutTile<bf16_t, kWideS, kBC>;  // rows of 128 bf16
    using FT = OutTile<float, kWideS, kBC>;   // rows of 128 fp32
    static constexpr int kQTBytes = kBC * QT::kRowBytes;
    static constexpr int kFTBytes = kBC * FT::kRowBytes;
    static constexpr int kPlanesBytes = 3 * kRBytes;  // K, V, G of one sub-chunk
    static constexpr int kDqLds = 2 * kPlanesBytes + kMBytes + kFTBytes + kRBytes;  // B1: two plane slots, M, dQ tile, Q plane
    // B3 with its row tiles: Q, dQ hi and lo, dV's sum in; dK, dV out.
    static constexpr int kDkvLds = kLds + 3 * kRBytes + kQTBytes + 2 * kFTBytes;
    static_assert(kDkvLds <= 160 * 1024, "gfx950 gives a workgroup at most 160 KB of LDS");
    static constexpr int kBlk = (kBC / 4) * (128 / 8);    // staging blocks of one tensor
    static_assert(3 * kBlk <= kWideThreads && kBlk % 64 == 0, "one staging block per thread, a tensor per wave");
};

// B1 over 128 x 128 blocks (bf16 tokens, d = 128): the forward walk of
// causal_bwd_dq_mfma_kernel over 128 buckets and every value column at once,
// eight waves (wave w: buckets 16 w .. 16 w + 15 of the block).  For its
// block it writes dQ whole (bf16, the caller's dQ) and dQ's bf16 remainders
// [N T][128], the running mass at every sub-chunk start
// [N][tiles][subs][128], and the tile's suffix totals as four 64 x 64
// records, (bucket group g2, value half h) at bwd_records + (2 g2 + h) N tiles
// rec.  One launch walks the blocks of `pairs` consecutive 128-bucket groups
// (block b: buckets s0 + 128 b ..; its outputs at b times the *_ps strides):
// the workgroups of one tile and stream, which read the same V and dOut rows,
// are 8 apart in launch order, so they land on the same XCD and the second
// reads of those rows come from its L2.  With pp.whole a workgroup walks its
// stream's tiles one after another, its prefix state carried on from zero,
// so no forward records are needed (tile t's walk starts after a barrier
// that follows every LDS read of tile t - 1, so the slots may restart).
__global__ __launch_bounds__(kWideThreads, 1) void causal_bwd_dq_wide_kernel(
    const bf16_t* __restrict__ q_in, const bf16_t* __restrict__ k_in, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ g, bf16_t* __restrict__ dq_hi_in, bf16_t* __restrict__ dq_lo_in,
    float* __restrict__ apre_in, const float* __restrict__ fwd_records, float* __restrict__ bwd_records_in,
    int64_t N, int64_t T, int tile, int64_t tiles, int64_t rec, int ldq, int ld_hi, int s0_in, int64_t fwd_rec,
    DqWidePairs pp) {
    using G = WideGeo;
    using PR = G::PR;
    using PM = G::PM;
    using T32 = OutTile<float, kWideS, kBC>;
    extern __shared__ __align__(16) unsigned char lds[];
    // Two slots of the K, V, G planes (sub-chunks alternate), then M, the
    // dQ tile and the Q rows.
    unsigned char* Ms = lds + 2 * G::kPlanesBytes;
    unsigned char* D32s = Ms + G::kMBytes;
    unsigned char* Qt = D32s + kBC * kWideS * 4;  // Q of the sub-chunk as a plane (rows = tokens)
    using QT = G::QT;

    const int tid = threadIdx.x, l = tid & 63, gq = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s = 16 * w + lr;  // the lane's bucket in the block
    // An item is a tile of a stream, or with pp.whole a stream, walked tile
    // after tile from a zero prefix.
    const WideItem it = wide_item(blockIdx.x, pp.pairs, pp.whole ? N : N * tiles);
    if (it.item < 0) return;  // the last group's padding
    const int64_t n = pp.whole ? it.item : it.item / tiles;
    const int64_t ti0 = pp.whole ? 0 : it.item % tiles, ti1 = pp.whole ? tiles : ti0 + 1;
    const int b = it.block;
    const bf16_t* q = q_in + kWideS * b;
    const bf16_t* k = k_in + kWideS * b;
    bf16_t* dq_hi = dq_hi_in + b * pp.hi_ps;
    bf16_t* dq_lo = dq_lo_in ? dq_lo_in + b * pp.lo_ps : nullptr;
    float* apre = apre_in + b * pp.ap_ps;
    float* bwd_records = bwd_records_in + b * pp.rec_ps;
    const int s0 = s0_in + kWideS * b;
    // Prefix state at the walk's start, transposed: B0^T[16 cb + 4 g + rr][s],
    // from the forward record of its first tile (a whole stream starts at
    // zero).  It runs on through the tiles of a whole-stream walk.
    const float* fr = pp.whole ? nullptr : fwd_records + (n * tiles + ti0) * fwd_rec;
    f32x4 b0t[8];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) b0t[cb][rr] = fr ? fr[int64_t(s0 + s) * kWideD + 16 * cb + 4 * gq + rr] : 0.f;
    // The forward record holds B [S][128] then A [S]; S = ldq.
    float a0 = fr ? fr[int64_t(ldq) * kWideD + s0 + s] : 0.f;
    const bf16x8 tri0 = tril_frag(0, gq, lr), tri1 = tril_frag(16, gq, lr);

    for (int64_t ti = ti0; ti < ti1; ++ti) {
        const int64_t t_begin = ti * tile;
        const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
        const int64_t base = n * T + t_begin;
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + base * ldq, int64_t(rows) * ldq * 2);
        // dQ as bf16 (hi, the caller's dQ or workspace rows of ld_hi) and the
        // bf16 rounding of its remainder (lo, rows of 128): hi + lo is dQ to
        // about 2^-17, which the backward walk reads back.
        const __amdgpu_buffer_rsrc_t hir = make_rsrc(dq_hi + base * ld_hi, int64_t(rows) * ld_hi * 2);
        // No remainders when no backward walk reads them (dq_lo null: an empty
        // view drops the stores).
        const __amdgpu_buffer_rsrc_t lor =
            make_rsrc(dq_lo ? dq_lo + base * kWideS : nullptr, dq_lo ? int64_t(rows) * kWideS * 2 : 0);

        // The tile's suffix totals start at zero.
        f32x4 zt[8];
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) zt[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        float ypart = 0.f;

        // Staging as in causal_bwd_dkv_wide_kernel.
        const int tensor = __builtin_amdgcn_readfirstlane(tid / G::kBlk);
        const int sa = (tid % G::kBlk) / 16, sb = tid % 16;
        const int sld = tensor == 0 ? ldq : kWideD;
        const bf16_t* ssrc = tensor == 0 ? k + base * ldq : tensor == 1 ? v + base * kWideD : g + base * kWideD;
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(tensor < 3 ? ssrc : nullptr, tensor < 3 ? int64_t(rows) * sld * 2 : 0);
        const int splane = tensor * G::kRBytes;  // the staged tensor's plane inside a slot
        // Sub-chunks of operands in flight in registers ahead of the one in LDS.
        constexpr int kDepth = RACE_BWD_WIDE_DQ_DEPTH;
        StageBlock<bf16_t> st[kDepth];
        // Q's rows: chunk tid of the sub-chunk (row tid / 16, 8 buckets) in
        // from global memory, into a plane read transposed.
        static_assert(QT::kChunks * kBC == kWideThreads, "one Q chunk per thread");
        uint4 qx[kDepth];
        // Row chunk tid of the sub-chunk (row tid / 16, buckets 8 (tid % 16) ..
        // + 7) into a plane whose transposed reads give each lane its bucket's
        // values at the accumulator layout's rows.
        auto put_row_chunk = [&](unsigned char* plane, const uint4& x) {
            const int row = tid / QT::kChunks, k0 = 8 * (tid % QT::kChunks);
            PR::put4(plane, row, k0, uint2{x.x, x.y}, uint2{});
            PR::put4(plane, row, k0 + 4, uint2{x.z, x.w}, uint2{});
        };
        auto load_q = [&](uint4& x, int r0) {
            x = buf_load16<kPolicyDefault>(qr, ((r0 + tid / QT::kChunks) * ldq + 8 * (tid % QT::kChunks)) * 2);
        };

        const int subs = tile / kBC;
        float* ap = apre + (n * tiles + ti) * int64_t(subs) * kWideS;
        // The previous sub-chunk's dQ tile as whole rows: dQ as bf16 and the
        // bf16 remainders (16-byte chunk c of a tile row holds elements 4 c ..
        // 4 c + 3).
        constexpr int kChunksPerRow = T32::kChunks;
        auto flush = [&](int r0) {
            typename T32::template Chunks<kWideThreads> c32;
            T32::template read<kWideThreads>(D32s, c32);
#pragma unroll
            for (int i = 0; i < T32::template Chunks<kWideThreads>::kPer; ++i) {
                const int qi = tid + i * kWideThreads;
                const f32x4 x = __builtin_bit_cast(f32x4, c32.x[i]);
                const u32x2 hi = {pack2(x[0], x[1]), pack2(x[2], x[3])};
                const u32x2 lo = {pack2(x[0] - lo_half(hi[0]), x[1] - hi_half(hi[0])),
                                  pack2(x[2] - lo_half(hi[1]), x[3] - hi_half(hi[1]))};
                const int row = r0 + qi / kChunksPerRow, c4 = 4 * (qi % kChunksPerRow);
                __builtin_amdgcn_raw_buffer_store_b64(hi, hir, (row * ld_hi + c4) * 2, 0, kPolicyDefault);
                __builtin_amdgcn_raw_buffer_store_b64(lo, lor, (row * kWideS + c4) * 2, 0, kPolicyDefault);
            }
        };
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            st[d].load(srs, d * kBC, sa, sb, sld);
            load_q(qx[d], d * kBC);
        }
        // Sub-chunk r0 uses plane slot (r0 / kBC) & 1, so two barriers per
        // sub-chunk suffice: its staging and Q-row stores need none before them
        // (the slot was last read two sub-chunks back, with two barriers since;
        // the Q rows were last read before the previous sub-chunk's second
        // barrier), and the previous dQ tile is read after the first barrier and
        // rewritten only after the second.
        auto sub_chunk = [&](StageBlock<bf16_t>& stg, uint4& qv, int r0) {
            unsigned char* Ks = lds + ((r0 / kBC) & 1) * G::kPlanesBytes;
            unsigned char* Vs = Ks + G::kRBytes;
            unsigned char* Gs = Vs + G::kRBytes;
            if (tensor < 3) stg.store_r<PR>(Ks + splane, sa, sb);
            put_row_chunk(Qt, qv);
            stg.load(srs, r0 + kDepth * kBC, sa, sb, sld);  // past the tile: zeros, never used
            load_q(qv, r0 + kDepth * kBC);
            __syncthreads();
            // The previous sub-chunk's dQ tile, complete since this barrier.
            // Unconditional: at r0 = 0 the offsets are negative, outside the
            // buffer ranges, and the stores are dropped; a sub-chunk past a
            // ragged tile end reads zeros and stores nothing.
            flush(r0 - kBC);
            if (gq == 0 && r0 < rows) ap[(r0 / kBC) * kWideS + s] = a0;

            // 1: Abar[i][s] = A0[s] + sum_{j <= i} K[j][s], r and W.
            float qc[2][4];
            {
                bf16x8 qf, unused;
                PR::frag_tr(Qt, 0, 16 * w, gq, lr, qf, unused);
#pragma unroll
                for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) qc[bi][rr] = float(qf[4 * bi + rr]);
            }
            bf16x8 kh, kl;
            PR::frag_tr(Ks, 0, 16 * w, gq, lr, kh, kl);
            f32x4 rv[2], wv[2];
#pragma unroll
            for (int bi = 0; bi < 2; ++bi) {
                f32x4 acc = {a0, a0, a0, a0};
                acc = mfma16(bi == 0 ? tri0 : tri1, kh, acc);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    rv[bi][rr] = __builtin_amdgcn_rcpf(acc[rr] + kEps);
                    wv[bi][rr] = qc[bi][rr] * rv[bi][rr];
                }
                if (bi == 1) a0 = __shfl(acc[3], 48 + lr);  // inclusive mass at the last token
            }

            // 2: M^T blocks (j-block, i-block) = V G^T, j <= i: (0,0), (0,1), (1,1) on waves 0..2.
            if (w < 3) {
                const int mbj = w == 2 ? 1 : 0, mbi = w >= 1 ? 1 : 0;
                f32x4 mt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    bf16x8 ah, al, bh, bl;
                    PR::frag(Vs, 16 * mbj + lr, kk, gq, ah, al);
                    PR::frag(Gs, 16 * mbi + lr, kk, gq, bh, bl);
                    mt = mfma16(ah, bh, mt);
                }
                if (mbj == mbi) {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        if (4 * gq + rr > lr) mt[rr] = 0.f;
                }
                uint2 hi, lo;
                split4<false>(mt[0], mt[1], mt[2], mt[3], hi, lo);
                PM::put4(Ms, 16 * mbi + lr, 16 * mbj + 4 * gq, hi, lo);
            }
            __syncthreads();

            // 3: U = G B0^T + M K;  dQ = r U;  alpha = -W dQ.
            f32x4 u[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                bf16x8 bh, bl;
                split8v<false>(b0t[2 * kk], b0t[2 * kk + 1], bh, bl);
#pragma unroll
                for (int bi = 0; bi < 2; ++bi) {
                    bf16x8 gh, gl;
                    PR::frag(Gs, 16 * bi + lr, kk, gq, gh, gl);
                    u[bi] = mfma16(gh, bh, u[bi]);
                }
            }
#pragma unroll
            for (int bi = 0; bi < 2; ++bi) {
                bf16x8 mh, ml;
                PM::frag(Ms, 16 * bi + lr, 0, gq, mh, ml);
                if (bi == 0) {
                    // Tokens 16..31 of the first block's row are above the diagonal.
#pragma unroll
                    for (int e = 4; e < 8; ++e) mh[e] = __bf16(0.0f);
                }
                u[bi] = mfma16(mh, kh, u[bi]);
            }
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const float dqv = rv[bi][rr] * u[bi][rr];
                    T32::put1(D32s, 16 * bi + 4 * gq + rr, s, dqv);
                    ypart += -wv[bi][rr] * dqv;
                }

            // 4: Z^T += G^T W;  5: B0^T += V^T K.
            bf16x8 wh, wl;
            split8v<false>(wv[0], wv[1], wh, wl);
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                bf16x8 gh, gl, vh, vl;
                PR::frag_tr(Gs, 0, 16 * cb, gq, lr, gh, gl);
                zt[cb] = mfma16(gh, wh, zt[cb]);
                PR::frag_tr(Vs, 0, 16 * cb, gq, lr, vh, vl);
                b0t[cb] = mfma16(vh, kh, b0t[cb]);
            }
        };
        int r0 = 0;
        for (; r0 < rows; r0 += kDepth * kBC) {
#pragma unroll
            for (int d = 0; d < kDepth; ++d) sub_chunk(st[d], qx[d], r0 + d * kBC);
        }
        __syncthreads();
        if (r0 > 0) flush(r0 - kBC);

        // Suffix totals of this tile into the four 64 x 64 records: Z[s][c]
        // (record layout B[s][c]) and Y[s], the totals of alpha, in value half
        // 0's record (half 1's holds zero).
        float y = ypart + __shfl_xor(ypart, 16);
        y = y + __shfl_xor(y, 32);
        const int g2 = w >> 2, sl = 16 * (w & 3) + lr;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float* br = bwd_records + (int64_t(2 * g2 + h) * N * tiles + n * tiles + ti) * rec;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) br[sl * kBS + 16 * cb + 4 * gq + rr] = zt[4 * h + cb][rr];
            if (gq == 0) br[kBS * kBS + sl] = h == 0 ? y : 0.f;
        }
    }
}

__global__ __launch_bounds__(kWideThreads, 1) void causal_bwd_dkv_wide_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ g, bf16_t* __restrict__ dK, int64_t T, int tile, int64_t tiles, int64_t rec,
    BwdWide wb) {
    using G = WideGeo;
    using PR = G::PR;
    using PM = G::PM;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Ks = lds;
    unsigned char* Vs = Ks + G::kRBytes;
    unsigned char* Gs = Vs + G::kRBytes;
    unsigned char* WT = Gs + G::kRBytes;
    unsigned char* MT = WT + G::kWTBytes;
    unsigned char* PTp = MT + G::kMBytes;
    unsigned char* Zr = PTp + G::kMBytes;
    // Q and dQ (hi and lo) of the sub-chunk come in as whole rows into
    // planes read transposed, dV's running sum as whole rows into a row tile
    // read in the accumulator layout; dK and dV of the previous sub-chunk go
    // out through row tiles (written in the accumulator layout, stored as
    // whole rows).
    unsigned char* Qt = Zr + G::kZBytes;
    unsigned char* Dh = Qt + G::kRBytes;
    unsigned char* Dl = Dh + G::kRBytes;
    unsigned char* Vt = Dl + G::kRBytes;
    unsigned char* dKt = Vt + G::kFTBytes;
    unsigned char* dVt = dKt + G::kQTBytes;
    using QT = G::QT;
    using FT = G::FT;

    const int tid = threadIdx.x, l = tid & 63, gq = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g2 = w >> 2;               // this wave's 64-bucket group
    const int sl = 16 * (w & 3) + lr;    // the lane's bucket inside it
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min<int64_t>(T, t_begin + tile) - t_begin);
    const int64_t base = n * T + t_begin;
    const int ldq = wb.ldq;
    // The group's buffers, chosen without indexing the argument struct by a
    // run-time value (which copies it to scratch memory).
    const float* rec0 = g2 ? wb.rec[1][0] : wb.rec[0][0];
    const float* rec1 = g2 ? wb.rec[1][1] : wb.rec[0][1];
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + base * ldq, int64_t(rows) * ldq * 2);
    const __amdgpu_buffer_rsrc_t hir =
        make_rsrc(static_cast<const bf16_t*>(wb.dq_hi) + base * wb.ld_hi, int64_t(rows) * wb.ld_hi * 2);
    const __amdgpu_buffer_rsrc_t lor =
        make_rsrc(static_cast<const bf16_t*>(wb.dq_lo) + base * kWideS, int64_t(rows) * kWideS * 2);
    const __amdgpu_buffer_rsrc_t dkr = make_rsrc(dK ? dK + base * ldq : nullptr, dK ? int64_t(rows) * ldq * 2 : 0);
    // dV: the running sum (written; read unless this is the first addend)
    // and the caller's dV for the last addend.  A gradient not asked for has
    // empty views, which drop the stores.
    const __amdgpu_buffer_rsrc_t avr =
        make_rsrc(wb.acc_v ? wb.acc_v + base * kWideD : nullptr, wb.acc_v ? int64_t(rows) * kWideD * 4 : 0);
    const __amdgpu_buffer_rsrc_t av_rd = make_rsrc(wb.acc_v && !wb.v_first ? wb.acc_v + base * kWideD : nullptr,
                                                   wb.acc_v && !wb.v_first ? int64_t(rows) * kWideD * 4 : 0);
    const __amdgpu_buffer_rsrc_t fvr = make_rsrc(wb.fin_v ? static_cast<bf16_t*>(wb.fin_v) + base * kWideD : nullptr,
                                                 wb.fin_v ? int64_t(rows) * kWideD * 2 : 0);

    // Suffix state at the tile end: Z1^T[16 cb + 4 g + rr][16 w + lr] from the
    // records of (group g2, value half cb / 4); Y1 from value half 0's.
    f32x4 zt[8];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
        const float* sr = (cb < 4 ? rec0 : rec1) + (n * tiles + ti) * rec;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) zt[cb][rr] = sr[sl * kBS + 16 * (cb & 3) + 4 * gq + rr];
    }
    float y1 = rec0[(n * tiles + ti) * rec + kBS * kBS + sl];
    const bf16x8 tri0 = tril_frag(0, gq, lr), tri1 = tril_frag(16, gq, lr);
    const bf16x8 up0 = triu_frag(0, gq, lr), up1 = triu_frag(16, gq, lr);

    // Staging: threads 0..383 take one block of 4 tokens x 8 columns of K,
    // V or G (two waves per tensor); waves 6 and 7 stage nothing.
    // The wave's tensor is uniform, so its buffer, stride and plane are
    // chosen once; waves 6 and 7 get an empty view (loads return zero).
    const int tensor = __builtin_amdgcn_readfirstlane(tid / G::kBlk);
    const int sa = (tid % G::kBlk) / 16, sb = tid % 16;
    const int sld = tensor == 0 ? ldq : kWideD;
    const bf16_t* ssrc = tensor == 0 ? k + base * ldq : tensor == 1 ? v + base * kWideD : g + base * kWideD;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(tensor < 3 ? ssrc : nullptr, tensor < 3 ? int64_t(rows) * sld * 2 : 0);
    unsigned char* splane = tensor == 0 ? Ks : tensor == 1 ? Vs : Gs;
    StageBlock<bf16_t> st;
    // Row chunks of 16 bytes: Q's, dQ's hi and lo chunk tid (row tid / 16 of
    // the sub-chunk, 8 buckets), the dV sum's chunks tid and tid + 512 (rows
    // of 32 chunks).
    static_assert(QT::kChunks * kBC == kWideThreads && FT::kChunks * kBC == 2 * kWideThreads, "chunk split");
    uint4 qx, hx, lx, vx[2];
    // Row chunk tid (row tid / 16, buckets 8 (tid % 16) .. + 7) of Q and dQ's
    // two parts into planes whose transposed reads give each lane its
    // bucket's values at the accumulator layout's rows.
    auto put_row_chunk = [&](unsigned char* plane, const uint4& x) {
        const int row = tid / QT::kChunks, k0 = 8 * (tid % QT::kChunks);
        PR::put4(plane, row, k0, uint2{x.x, x.y}, uint2{});
        PR::put4(plane, row, k0 + 4, uint2{x.z, x.w}, uint2{});
    };
    auto load_rows = [&](int r0) {
        const int row = r0 + tid / QT::kChunks, c8 = 8 * (tid % QT::kChunks);
        qx = buf_load16<kPolicyDefault>(qr, (row * ldq + c8) * 2);
        hx = buf_load16<kPolicyDefault>(hir, (row * wb.ld_hi + c8) * 2);
        lx = buf_load16<kPolicyDefault>(lor, (row * kWideS + c8) * 2);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            vx[i] = buf_load16<kPolicyDefault>(av_rd, r0 * FT::kRowBytes + 16 * (tid + i * kWideThreads));
    };
    auto store_rows = [&]() {
        put_row_chunk(Qt, qx);
        put_row_chunk(Dh, hx);
        put_row_chunk(Dl, lx);
#pragma unroll
        for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(Vt + FT::chunk_at(tid + i * kWideThreads)) = vx[i];
    };
    // dK and dV rows of the sub-chunk at r0 (rows past the tile, and all of
    // them before the first sub-chunk, fall outside the views).
    auto flush = [&](int r0) {
        const uint4 kx = *reinterpret_cast<const uint4*>(dKt + QT::chunk_at(tid));
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, kx), dkr,
                                               ((r0 + tid / QT::kChunks) * ldq + 8 * (tid % QT::kChunks)) * 2, 0,
                                               kPolicyDefault);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kWideThreads;
            const uint4 x = *reinterpret_cast<const uint4*>(dVt + FT::chunk_at(c));
            if (wb.fin_v)
                __builtin_amdgcn_raw_buffer_store_b64(
                    u32x2{pack2(__uint_as_float(x.x), __uint_as_float(x.y)),
                          pack2(__uint_as_float(x.z), __uint_as_float(x.w))},
                    fvr, (r0 * kWideD + 4 * c) * 2, 0, kPolicyDefault);
            else
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), avr, (r0 * kWideD + 4 * c) * 4,
                                                       0, kPolicyDefault);
        }
    };

    const int subs = tile / kBC;
    const float* ap = wb.apre + (n * tiles + ti) * int64_t(subs) * kWideS + 16 * w + lr;
    const int last = ((rows - 1) / kBC) * kBC;
    st.load(srs, last, sa, sb, sld);
    load_rows(last);
    float a0n = ap[(last / kBC) * kWideS];
    for (int r0 = last; r0 >= 0; r0 -= kBC) {
        __syncthreads();
        flush(r0 + kBC);
        if (tensor < 3) st.store_r<PR>(splane, sa, sb);
        store_rows();
        const float a0 = a0n;
        if (r0 > 0) {
            st.load(srs, r0 - kBC, sa, sb, sld);
            load_rows(r0 - kBC);
            a0n = ap[(r0 / kBC - 1) * kWideS];
        }
        // Z1 as a plane for dV: row s, four consecutive c per lane.
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            uint2 hi, lo;
            split4<false>(zt[cb][0], zt[cb][1], zt[cb][2], zt[cb][3], hi, lo);
            PR::put4(Zr, 16 * w + lr, 16 * cb + 4 * gq, hi, lo);
        }
        __syncthreads();

        // 1: Abar, r, W, alpha; W^T into its plane (row s, four consecutive i).
        float qc[2][4], dc[2][4];
        {
            bf16x8 qf, hf, lf, unused;
            PR::frag_tr(Qt, 0, 16 * w, gq, lr, qf, unused);
            PR::frag_tr(Dh, 0, 16 * w, gq, lr, hf, unused);
            PR::frag_tr(Dl, 0, 16 * w, gq, lr, lf, unused);
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    qc[bi][rr] = float(qf[4 * bi + rr]);
                    dc[bi][rr] = float(hf[4 * bi + rr]) + float(lf[4 * bi + rr]);
                }
        }
        bf16x8 kh, kl;
        PR::frag_tr(Ks, 0, 16 * w, gq, lr, kh, kl);
        f32x4 wv[2], al[2];
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            f32x4 acc = {a0, a0, a0, a0};
            acc = mfma16(bi == 0 ? tri0 : tri1, kh, acc);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                wv[bi][rr] = qc[bi][rr] * __builtin_amdgcn_rcpf(acc[rr] + kEps);
                al[bi][rr] = -wv[bi][rr] * dc[bi][rr];
            }
            uint2 hi, lo;
            split4<false>(wv[bi][0], wv[bi][1], wv[bi][2], wv[bi][3], hi, lo);
            PM::put4(WT, 16 * w + lr, 16 * bi + 4 * gq, hi, lo);
        }
        __syncthreads();

        // 2: M = tril(G V^T) blocks on waves 0..2, P = tril(W K^T) blocks on
        //    waves 3..5; blocks (0,0), (1,0), (1,1), written with rows j.
        if (w < 6) {
            const int b = w < 3 ? w : w - 3;
            const int bi = b >= 1 ? 1 : 0, bj = b == 2 ? 1 : 0;
            // All four steps' fragments are read before the products, one
            // branch per wave (a branch per step made each product wait for
            // its own reads).
            bf16x8 ah[4], bh[4];
            if (w < 3) {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    bf16x8 alo, bl;
                    PR::frag(Gs, 16 * bi + lr, kk, gq, ah[kk], alo);
                    PR::frag(Vs, 16 * bj + lr, kk, gq, bh[kk], bl);
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    bf16x8 alo, bl;
                    PM::frag_tr(WT, 32 * kk, 16 * bi, gq, lr, ah[kk], alo);
                    PR::frag(Ks, 16 * bj + lr, kk, gq, bh[kk], bl);
                }
            }
            f32x4 m = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) m = mfma16(ah[kk], bh[kk], m);
            if (bi == bj) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (lr > 4 * gq + rr) m[rr] = 0.f;
            }
            uint2 hi, lo;
            split4<false>(m[0], m[1], m[2], m[3], hi, lo);
            PM::put4(w < 3 ? MT : PTp, 16 * bj + lr, 16 * bi + 4 * gq, hi, lo);
        }
        __syncthreads();

        bf16x8 wh, wl, ah2, al2;
        split8v<false>(wv[0], wv[1], wh, wl);
        split8v<false>(al[0], al[1], ah2, al2);
        // 3: dK for this wave's buckets: V Z1^T + M^T W + triu(1) alpha + Y1,
        //    formed transposed (each product with its operands swapped), so
        //    a lane holds buckets 16 w + 4 g .. + 3 of token 16 bj + lr: four
        //    consecutive values of a dK row.
        f32x4 dk[2];
        {
            f32x4 y4;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) y4[rr] = __shfl(y1, 4 * gq + rr);
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) dk[bj] = y4;
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            bf16x8 zh, zl;
            split8v<false>(zt[2 * kk], zt[2 * kk + 1], zh, zl);
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
                bf16x8 vh, vl;
                PR::frag(Vs, 16 * bj + lr, kk, gq, vh, vl);
                dk[bj] = mfma16(zh, vh, dk[bj]);
            }
        }
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            bf16x8 mh, ml;
            PM::frag(MT, 16 * bj + lr, 0, gq, mh, ml);
            if (bj == 1) {
                // Tokens i < 16 of the second j-block are above the diagonal.
#pragma unroll
                for (int e = 0; e < 4; ++e) mh[e] = __bf16(0.0f);
            }
            dk[bj] = mfma16(wh, mh, dk[bj]);
            dk[bj] = mfma16(ah2, bj == 0 ? up0 : up1, dk[bj]);
            QT::put(dKt, 16 * bj + lr, 16 * w + 4 * gq, dk[bj]);
        }
        // 4: dV for this wave's value columns: K Z1 + P^T G, transposed the
        //    same way (columns 16 w + 4 g .. + 3 of token 16 bj + lr), added
        //    to the running sum's four values of that row.
        {
            f32x4 dv[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                bf16x8 zh, zl;
                PR::frag_tr(Zr, 32 * kk, 16 * w, gq, lr, zh, zl);
#pragma unroll
                for (int bj = 0; bj < 2; ++bj) {
                    bf16x8 kh2, kl2;
                    PR::frag(Ks, 16 * bj + lr, kk, gq, kh2, kl2);
                    dv[bj] = mfma16(zh, kh2, dv[bj]);
                }
            }
            bf16x8 gh, gl;
            PR::frag_tr(Gs, 0, 16 * w, gq, lr, gh, gl);
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
                bf16x8 ph, pl;
                PM::frag(PTp, 16 * bj + lr, 0, gq, ph, pl);
                if (bj == 1) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) ph[e] = __bf16(0.0f);
                }
                dv[bj] = mfma16(gh, ph, dv[bj]);
                // The first addend's read view is empty: the sum is zero.
                const f32x4 sum = FT::get4(Vt, 16 * bj + lr, 16 * w + 4 * gq);
                FT::put(dVt, 16 * bj + lr, 16 * w + 4 * gq, dv[bj] + sum);
            }
        }
        // 5: the suffix state before this sub-chunk.
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            bf16x8 gh, gl;
            PR::frag_tr(Gs, 0, 16 * cb, gq, lr, gh, gl);
            zt[cb] = mfma16(gh, wh, zt[cb]);
        }
        float ys = 0.f;
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) ys += al[bi][rr];
        ys = ys + __shfl_xor(ys, 16);
        ys = ys + __shfl_xor(ys, 32);
        y1 += ys;
    }
    __syncthreads();
    flush(0);
}

}  // namespace

bool causal_bwd_mfma_supported(int S, int d) {
    return S % kBS == 0 && d % kBS == 0 && S >= kBS && d >= kBS && S <= 256 && d <= 128;
}

BwdBlock single_block(const Problem& p) {
    BwdBlock b;
    b.ldq = b.ldv = kBS;
    b.fwd_d = kBS;
    b.fwd_a = kBS * kBS;
    b.fwd_rec = p.rec;
    return b;
}

hipError_t launch_causal_bwd_dq_mfma(const void* q, const void* k, const void* v, const void* g,
                                     void* dQ, float* dq32, float* apre, const float* fwd_records,
                                     float* bwd_records, const Problem& p, const BwdBlock& blk,
                                     hipStream_t stream, int dv) {
    // p describes one 64 x 64 block (p.S = p.d = 64, p.rec its record); with
    // dv = 128 the walk takes both value groups of a d = 128 problem (bf16,
    // blocked) and writes one record array per group.
    if (p.S != kBS || p.d != kBS || p.tile % kBC != 0) return hipErrorInvalidValue;
    if (dv != kBS && !(dv == 2 * kBS && p.dtype == RACE_BF16 && blk.blocked)) return hipErrorInvalidValue;
    // fp32: dQ is written only as the fp32 copy (pass the caller's dQ as dq32).
    if (p.dtype != RACE_BF16 && dQ) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    if (p.dtype == RACE_BF16) {
        using G = BwdGeo<bf16_t>;
        if (dv == 2 * kBS) {
            causal_bwd_dq_mfma_kernel<bf16_t, true, 2 * kBS><<<grid, kThreads, G::kDqLdsV<2 * kBS>, stream>>>(
                static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), static_cast<bf16_t*>(dQ),
                dq32, apre, fwd_records, bwd_records, p.T, p.tile, p.tiles, p.rec, blk);
            return hipGetLastError();
        }
        const size_t lds = G::kDqLdsV<kBS>;
        auto kern = blk.blocked ? causal_bwd_dq_mfma_kernel<bf16_t, true, kBS>
                                : causal_bwd_dq_mfma_kernel<bf16_t, false, kBS>;
        kern<<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
            static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), static_cast<bf16_t*>(dQ),
            dq32, apre, fwd_records, bwd_records, p.T, p.tile, p.tiles, p.rec, blk);
    } else {
        using G = BwdGeo<float>;
        const size_t lds = G::kDqLdsV<kBS>;
        auto kern = blk.blocked ? causal_bwd_dq_mfma_kernel<float, true, kBS>
                                : causal_bwd_dq_mfma_kernel<float, false, kBS>;
        kern<<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
            static_cast<const float*>(g), static_cast<float*>(dQ), dq32, apre, fwd_records,
            bwd_records, p.T, p.tile, p.tiles, p.rec, blk);
    }
    return hipGetLastError();
}

hipError_t launch_causal_bwd_dkv_mfma(const void* q, const void* k, const void* v, const void* g,
                                      const float* dq32, const float* apre,
                                      const float* suffix_records, void* dK, void* dV,
                                      const Problem& p, const BwdBlock& blk, hipStream_t stream) {
    if (p.S != kBS || p.d != kBS || p.tile % kBC != 0) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
#define RACE_DKV(TIN)                                                                                \
    (blk.blocked ? causal_bwd_dkv_mfma_kernel<TIN, true> : causal_bwd_dkv_mfma_kernel<TIN, false>)   \
        <<<grid, kThreads, BwdGeo<TIN>::kDkvLds, stream>>>(                                          \
        static_cast<const TIN*>(q), static_cast<const TIN*>(k), static_cast<const TIN*>(v),         \
        static_cast<const TIN*>(g), dq32, apre, suffix_records, static_cast<TIN*>(dK),              \
        static_cast<TIN*>(dV), p.T, p.tile, p.tiles, p.rec, blk)
    if (p.dtype == RACE_BF16)
        RACE_DKV(bf16_t);
    else
        RACE_DKV(float);
#undef RACE_DKV
    return hipGetLastError();
}

hipError_t launch_causal_bwd_dq_wide(const void* q, const void* k, const void* v, const void* g, void* dq_hi,
                                     int ld_hi, void* dq_lo, float* apre, const float* fwd_records,
                                     float* bwd_records, const Problem& p, int s0, const DqWidePairs& pp,
                                     hipStream_t stream) {
    if (p.dtype != RACE_BF16 || p.d != kWideD || p.S % kWideS != 0 || s0 % kWideS != 0 || pp.pairs < 1 ||
        s0 + kWideS * pp.pairs > p.S || p.tile % kBC != 0 || !dq_hi || ld_hi < kWideS)
        return hipErrorInvalidValue;
    if (!pp.whole && !fwd_records) return hipErrorInvalidValue;
    const int64_t groups = ((pp.whole ? p.N : p.N * p.tiles) + kWideXcds - 1) / kWideXcds;
    // gfx950 takes at most 2^32 - 1 work-items along a grid dimension.
    if (groups * kWideXcds * pp.pairs * kWideThreads > int64_t(UINT32_MAX)) return hipErrorInvalidValue;
    const dim3 grid(unsigned(groups * kWideXcds * pp.pairs));
    causal_bwd_dq_wide_kernel<<<grid, kWideThreads, WideGeo::kDqLds, stream>>>(
        static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k), static_cast<const bf16_t*>(v),
        static_cast<const bf16_t*>(g), static_cast<bf16_t*>(dq_hi), static_cast<bf16_t*>(dq_lo), apre, fwd_records,
        bwd_records, p.N, p.T, p.tile, p.tiles, record_floats(kBS, kBS), p.S, ld_hi, s0, p.rec, pp);
    return hipGetLastError();
}

hipError_t launch_causal_bwd_dkv_wide(const void* q, const void* k, const void* v, const void* g, void* dK,
                                      const Problem& p, const BwdWide& wb, hipStream_t stream) {
    if (p.dtype != RACE_BF16 || p.d != kWideD || p.S % kWideS != 0 || p.tile % kBC != 0 || wb.ldq != p.S)
        return hipErrorInvalidValue;
    if (!wb.dq_hi || !wb.dq_lo || wb.ld_hi < kWideS || !wb.apre) return hipErrorInvalidValue;
    for (int g2 = 0; g2 < 2; ++g2)
        if (!wb.rec[g2][0] || !wb.rec[g2][1]) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    causal_bwd_dkv_wide_kernel<<<grid, kWideThreads, WideGeo::kDkvLds, stream>>>(
        static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k), static_cast<const bf16_t*>(v),
        static_cast<const bf16_t*>(g), static_cast<bf16_t*>(dK), p.T, p.tile, p.tiles, record_floats(kBS, kBS),
        wb);
    return hipGetLastError();
}

}  // namespace race
