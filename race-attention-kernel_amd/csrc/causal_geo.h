// causal_geo.h -- tile geometry and K/V staging shared by the per-bucket
// MFMA causal kernels (mfma_causal.hip: the op on bucket probabilities;
// hashed_causal.hip: the same op with the hashing inside).  Not part of the
// ABI.
#pragma once

#include "mfma_common.h"

namespace race {
namespace mfma {

// Geometry of one (S, D, C, dtype) specialization.  Every tile is stored with
// tokens as rows (W, K, V; P with queries as rows); products that contract
// over tokens read their fragments transposed (Plane::frag_tr).
// kPrecise (bf16 tokens): every product carries its fp32 operands as bf16
// hi + lo pairs, as the fp32 path does (W, P and the carried state; the lo
// parts of bf16 K and V are zero), so the result is fp32-accurate up to the
// output's own rounding.
template <typename TIn, int S, int D, int C, int NW = 4, bool kPrecise = false>
struct Geo {
    static constexpr int kT = 64 * NW;  // threads per workgroup (NW wave64s)
    static constexpr bool kSplit = std::is_same<TIn, float>::value || kPrecise;
    static constexpr int E = Elem<TIn>::kPerVec;
    using PS = Plane<kSplit, S>;  // token rows over buckets: W
    // The K tile (token rows over buckets, read transposed by the running mass
    // and the state update): bf16 rows of 256 buckets hold odd rows' chunk
    // halves swapped (Plane kHalfSwap), which leaves the transposed reads
    // without bank conflicts.
    static constexpr bool kKHalfSwap = !kSplit && S == 256;
    using PK = Plane<kSplit, S, kKHalfSwap>;
    using PC = Plane<kSplit, C>;  // query rows over keys: P
    using PD = Plane<kSplit, D>;  // token rows over value columns: V
    static constexpr int kWBytes = C * PS::kPitch;
    static constexpr int kKBytes = C * PK::kPitch;
    static constexpr int kPBytes = C * PC::kPitch;
    static constexpr int kVBytes = C * PD::kPitch;
    // The output tile [C][D] in TIn, rows of 16-byte chunks swizzled by row
    // (OutTile), staged so that global stores cover whole rows.
    static constexpr int kOBytes = C * D * int(sizeof(TIn));
    // bf16 Q is staged through LDS as well ([C][S], the same row swizzle), so
    // its global loads cover whole rows: read in the accumulator layout it
    // would be 32-byte pieces of 16 rows per instruction (10% slower at
    // cfg5).  fp32 Q (64-byte pieces) measured no faster staged.
    static constexpr bool kQStage = !kSplit;
    static constexpr int kQBytes = kQStage ? C * S * int(sizeof(TIn)) : 0;
    static constexpr int kOutputLds = kWBytes + kKBytes + kPBytes + kVBytes + kOBytes + kQBytes;
    static constexpr int kSumsLds = kKBytes + kVBytes + 16 * S * 4;
    // Register staging of K and V: blocks of 4 rows x E columns.
    static constexpr int kKBlk = (C / 4) * (S / E);
    static constexpr int kKPer = (kKBlk + kT - 1) / kT;
    static constexpr int kVBlk = (C / 4) * (D / E);
    static constexpr int kVPer = (kVBlk + kT - 1) / kT;
    static_assert(S % 64 == 0 && D % 64 == 0 && (C == 32 || C == 64), "unsupported tile");
    static_assert(S % (16 * NW) == 0 && D % (16 * NW) == 0, "every wave owns whole 16-blocks");
};

// Raw K and V registers of one sub-chunk.
template <typename TIn, int S, int D, int C, int P, int NW = 4, bool kPrecise = false>
struct KVStage {
    using G = Geo<TIn, S, D, C, NW, kPrecise>;
    uint4 k[G::kKPer][4];
    uint4 v[G::kVPer][4];

    // Rows r0 .. r0 + C - 1 of the tile buffers (row r0 is the sub-chunk's
    // first token relative to the tile; rows past the tile read as zero).
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr, int r0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < G::kKPer; ++p) {
            const int blk = tid + p * G::kT;
            const int a = blk / (S / G::E), b = blk % (S / G::E);
            if (G::kKBlk % G::kT == 0 || blk < G::kKBlk) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    k[p][rr] = buf_load16<P>(kr, ((r0 + 4 * a + rr) * S + b * G::E) * int(sizeof(TIn)));
            }
        }
#pragma unroll
        for (int p = 0; p < G::kVPer; ++p) {
            const int blk = tid + p * G::kT;
            const int a = blk / (D / G::E), b = blk % (D / G::E);
            if (G::kVBlk % G::kT == 0 || blk < G::kVBlk) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    v[p][rr] = buf_load16<P>(vr, ((r0 + 4 * a + rr) * D + b * G::E) * int(sizeof(TIn)));
            }
        }
    }

    // The K rows [C][S] and V rows [C][D] as plane tiles (each element split
    // once), and the column sums of K into asum when given.
    __device__ __forceinline__ void store(unsigned char* Ks, unsigned char* Vs, float* asum) const {
        constexpr bool kSplit = G::kSplit;
        constexpr int E = G::E;
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < G::kKPer; ++p) {
            const int blk = tid + p * G::kT;
            if (blk >= G::kKBlk) continue;
            const int a = blk / (S / E), b = blk % (S / E);
#pragma unroll
            for (int h = 0; h < E / 4; ++h) {
                float x[4][4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                    for (int c = 0; c < 4; ++c) x[rr][c] = Elem<TIn>::get(k[p][rr], 4 * h + c);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    uint2 hi, lo;
                    if constexpr (kSplit) {
                        split4<true>(x[rr][0], x[rr][1], x[rr][2], x[rr][3], hi, lo);
                    } else {  // bf16 rows go in as they are
                        hi = make_uint2(h ? k[p][rr].z : k[p][rr].x, h ? k[p][rr].w : k[p][rr].y);
                        lo = hi;
                    }
                    G::PK::put4(Ks, 4 * a + rr, b * E + 4 * h, hi, lo);
                }
                if (asum) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        asum[p * E + 4 * h + c] += ((x[0][c] + x[1][c]) + x[2][c]) + x[3][c];
                }
            }
        }
#pragma unroll
        for (int p = 0; p < G::kVPer; ++p) {
            const int blk = tid + p * G::kT;
            if (blk >= G::kVBlk) continue;
            const int a = blk / (D / E), b = blk % (D / E);
#pragma unroll
            for (int h = 0; h < E / 4; ++h)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    uint2 hi, lo;
                    if constexpr (kSplit) {
                        split4<true>(Elem<TIn>::get(v[p][rr], 4 * h), Elem<TIn>::get(v[p][rr], 4 * h + 1),
                                     Elem<TIn>::get(v[p][rr], 4 * h + 2), Elem<TIn>::get(v[p][rr], 4 * h + 3),
                                     hi, lo);
                    } else {
                        hi = make_uint2(h ? v[p][rr].z : v[p][rr].x, h ? v[p][rr].w : v[p][rr].y);
                        lo = hi;
                    }
                    G::PD::put4(Vs, 4 * a + rr, b * E + 4 * h, hi, lo);
                }
        }
    }
};

}  // namespace mfma
}  // namespace race
