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
//   1. tile_sums_mfma_kernel   per (tile, stream): B_tile = K^T V, A_tile = 1^T K
//   2. tile_scan_kernel        exclusive scan of the tile records (VALU file)
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
// product without a trip through LDS.  Every LDS operand tile is stored in
// "slots" of 4 consecutive elements of one row -- 16 bytes (4 bf16 hi, then
// 4 bf16 lo) with hi/lo, 8 bytes without -- so one fragment is two slot reads.
#include <type_traits>

#include "race_internal.h"

namespace race {
namespace {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// acc += A B with optional hi/lo operands: lo*hi and hi*lo first, then hi*hi.
template <bool kSplit>
__device__ __forceinline__ f32x4 mfma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                       const bf16x8& bl, f32x4 acc) {
    if constexpr (kSplit) {
        acc = mfma16(al, bh, acc);
        acc = mfma16(ah, bl, acc);
    }
    return mfma16(ah, bh, acc);
}

__device__ __forceinline__ bf16x8 cat(const bf16x4& a, const bf16x4& b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Four consecutive elements of one row of an LDS operand tile.
template <bool kSplit>
struct alignas(kSplit ? 16 : 8) Slot {
    bf16x4 hi;
    bf16x4 lo;
};
template <>
struct alignas(8) Slot<false> {
    bf16x4 hi;
};

template <bool kSplit>
__device__ __forceinline__ Slot<kSplit> make_slot(const f32x4& x) {
    Slot<kSplit> s;
    s.hi = __builtin_convertvector(x, bf16x4);  // round to nearest even
    if constexpr (kSplit) s.lo = __builtin_convertvector(x - __builtin_convertvector(s.hi, f32x4), bf16x4);
    return s;
}

// Fragment of row `row` of a slot tile for contraction step kk (permuted k).
template <bool kSplit>
__device__ __forceinline__ void read_frag(const unsigned char* tile, int pitch, int row, int kk,
                                          int g, bf16x8& hi, bf16x8& lo) {
    constexpr int kSlot = sizeof(Slot<kSplit>);
    const unsigned char* p = tile + row * pitch + (8 * kk + g) * kSlot;
    const Slot<kSplit> s0 = *reinterpret_cast<const Slot<kSplit>*>(p);
    const Slot<kSplit> s1 = *reinterpret_cast<const Slot<kSplit>*>(p + 4 * kSlot);
    hi = cat(s0.hi, s1.hi);
    if constexpr (kSplit) lo = cat(s0.lo, s1.lo);
}

// ---------------------------------------------------------------------------
// Global <-> register traffic.  Token rows of one stream are contiguous, so a
// sub-chunk of C tokens is one contiguous block of C*W elements.

template <typename TIn>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int kPerVec = 4;  // elements per 16-byte vector
    __device__ static float get(const uint4& v, int i) {
        return __uint_as_float(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
    }
};
template <>
struct Elem<bf16_t> {
    static constexpr int kPerVec = 8;
    __device__ static float get(const uint4& v, int i) {
        const uint32_t w = (i >> 1) == 0 ? v.x : (i >> 1) == 1 ? v.y : (i >> 1) == 2 ? v.z : v.w;
        return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
    }
};

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Geometry of one (S, D, C, dtype) specialization.
template <typename TIn, int S, int D, int C>
struct Geo {
    static constexpr bool kSplit = std::is_same<TIn, float>::value;
    static constexpr int kSlot = sizeof(Slot<kSplit>);
    static constexpr int E = Elem<TIn>::kPerVec;
    // Row pitches in bytes: the slots of a row plus one 16-byte pad.
    static constexpr int kPitchS = (S / 4) * kSlot + 16;
    static constexpr int kPitchC = (C / 4) * kSlot + 16;
    static constexpr int kQBytes = C * kPitchS;  // Q, then W in place
    static constexpr int kKBytes = C * (kPitchS > kPitchC ? kPitchS : kPitchC);  // K, then P
    static constexpr int kKTBytes = S * kPitchC;
    static constexpr int kVTBytes = D * kPitchC;
    static constexpr int kOutputLds = kQBytes + kKBytes + kKTBytes + kVTBytes;
    static constexpr int kSumsLds = kKTBytes + kVTBytes + 16 * S * 4;
    // Register staging of one sub-chunk.
    static constexpr int kQVec = C * S / E;          // 16-byte vectors of Q
    static constexpr int kQPer = (kQVec + kThreads - 1) / kThreads;
    static constexpr int kKBlk = (C / 4) * (S / E);  // 4-row x E-column blocks of K
    static constexpr int kKPer = (kKBlk + kThreads - 1) / kThreads;
    static constexpr int kVBlk = (C / 4) * (D / E);
    static constexpr int kVPer = (kVBlk + kThreads - 1) / kThreads;
    static_assert(S % 64 == 0 && D % 64 == 0 && C % 32 == 0 && C <= 64, "unsupported tile");
    static_assert(S >= C, "P overlays the K tile");
};

// Raw registers of one sub-chunk (rows >= cnt read as zero).
template <typename TIn, int S, int D, int C>
struct Stage {
    using G = Geo<TIn, S, D, C>;
    uint4 q[G::kQPer];
    uint4 k[G::kKPer][4];
    uint4 v[G::kVPer][4];

    __device__ __forceinline__ void load(const TIn* qn, const TIn* kn, const TIn* vn, int64_t t0,
                                         int cnt, bool want_q) {
        const int tid = threadIdx.x;
        const uint4 zero = make_uint4(0, 0, 0, 0);
        if (want_q) {
#pragma unroll
            for (int p = 0; p < G::kQPer; ++p) {
                const int idx = tid + p * kThreads;
                const int row = idx / (S / G::E);
                q[p] = (idx < G::kQVec && row < cnt) ? load16(qn + t0 * S + int64_t(idx) * G::E) : zero;
            }
        }
#pragma unroll
        for (int p = 0; p < G::kKPer; ++p) {
            const int blk = tid + p * kThreads;
            const int a = blk / (S / G::E), b = blk % (S / G::E);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = 4 * a + rr;
                k[p][rr] = (blk < G::kKBlk && row < cnt)
                               ? load16(kn + (t0 + row) * S + b * G::E)
                               : zero;
            }
        }
#pragma unroll
        for (int p = 0; p < G::kVPer; ++p) {
            const int blk = tid + p * kThreads;
            const int a = blk / (D / G::E), b = blk % (D / G::E);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = 4 * a + rr;
                v[p][rr] = (blk < G::kVBlk && row < cnt)
                               ? load16(vn + (t0 + row) * D + b * G::E)
                               : zero;
            }
        }
    }

    // K^T [S][C] and V^T [D][C] slot tiles; K [C][S] too when Ks is given;
    // column sums of K into asum when given.
    __device__ __forceinline__ void store_kv(unsigned char* Ks, unsigned char* KTs,
                                             unsigned char* VTs, float* asum) const {
        constexpr bool kSplit = G::kSplit;
        constexpr int E = G::E;
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < G::kKPer; ++p) {
            const int blk = tid + p * kThreads;
            if (blk >= G::kKBlk) continue;
            const int a = blk / (S / E), b = blk % (S / E);
            float x[4][E];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int c = 0; c < E; ++c) x[rr][c] = Elem<TIn>::get(k[p][rr], c);
            if (Ks) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                    for (int h = 0; h < E / 4; ++h) {
                        const f32x4 f = {x[rr][4 * h], x[rr][4 * h + 1], x[rr][4 * h + 2], x[rr][4 * h + 3]};
                        *reinterpret_cast<Slot<kSplit>*>(Ks + (4 * a + rr) * G::kPitchS +
                                                         (b * E / 4 + h) * G::kSlot) = make_slot<kSplit>(f);
                    }
            }
#pragma unroll
            for (int c = 0; c < E; ++c) {
                const f32x4 f = {x[0][c], x[1][c], x[2][c], x[3][c]};
                *reinterpret_cast<Slot<kSplit>*>(KTs + (b * E + c) * G::kPitchC + a * G::kSlot) =
                    make_slot<kSplit>(f);
                if (asum) asum[p * E + c] += ((x[0][c] + x[1][c]) + x[2][c]) + x[3][c];
            }
        }
#pragma unroll
        for (int p = 0; p < G::kVPer; ++p) {
            const int blk = tid + p * kThreads;
            if (blk >= G::kVBlk) continue;
            const int a = blk / (D / E), b = blk % (D / E);
#pragma unroll
            for (int c = 0; c < E; ++c) {
                const f32x4 f = {Elem<TIn>::get(v[p][0], c), Elem<TIn>::get(v[p][1], c),
                                 Elem<TIn>::get(v[p][2], c), Elem<TIn>::get(v[p][3], c)};
                *reinterpret_cast<Slot<kSplit>*>(VTs + (b * E + c) * G::kPitchC + a * G::kSlot) =
                    make_slot<kSplit>(f);
            }
        }
    }

    // Raw Q into the Q tile: fp32 values (16-byte slots) or bf16 (8-byte slots).
    __device__ __forceinline__ void store_q(unsigned char* Qs) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < G::kQPer; ++p) {
            const int idx = tid + p * kThreads;
            if (idx >= G::kQVec) continue;
            const int row = idx / (S / G::E), col = (idx % (S / G::E)) * G::E;
            *reinterpret_cast<uint4*>(Qs + row * G::kPitchS + (col / 4) * G::kSlot) = q[p];
        }
    }
};

// Four consecutive Q values of row i (fp32 or bf16 slot) as floats.
template <bool kSplit>
__device__ __forceinline__ f32x4 read_q4(const unsigned char* p) {
    if constexpr (kSplit) {
        return *reinterpret_cast<const f32x4*>(p);
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        return f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u)};
    }
}

__device__ __forceinline__ void store4(float* p, const f32x4& x) { *reinterpret_cast<f32x4*>(p) = x; }
__device__ __forceinline__ void store4(bf16_t* p, const f32x4& x) {
    const bf16x4 b = __builtin_convertvector(x, bf16x4);
    *reinterpret_cast<bf16x4*>(p) = b;
}

// ---------------------------------------------------------------------------
// K1: per (tile, stream) totals B_tile = K^T V and A_tile = colsum(K) into the
// tile record (B [S][D] then A [S]).  Wave w owns the V columns of c-blocks
// w, w + 4, ...; its accumulators hold B[16 sb + 4 g + r][16 cb + lr].
template <typename TIn, int S, int D, int C, int kMinBlocks>
__global__ __launch_bounds__(kThreads, kMinBlocks) void tile_sums_mfma_kernel(
    const TIn* __restrict__ k, const TIn* __restrict__ v, float* __restrict__ records, int64_t T,
    int tile, int64_t tiles, int64_t rec) {
    using G = Geo<TIn, S, D, C>;
    constexpr bool kSplit = G::kSplit;
    constexpr int NSB = S / 16, NKC = C / 32, CBW = D / 64;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* KTs = lds;
    unsigned char* VTs = KTs + G::kKTBytes;
    float* Apart = reinterpret_cast<float*>(VTs + G::kVTBytes);  // [16][S]

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, lr = l & 15;
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const TIn* kn = k + n * T * S;
    const TIn* vn = v + n * T * D;

    f32x4 acc[NSB][CBW];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) acc[sb][cbw] = f32x4{0.f, 0.f, 0.f, 0.f};
    float asum[G::kKPer * G::E];
#pragma unroll
    for (int i = 0; i < G::kKPer * G::E; ++i) asum[i] = 0.f;

    Stage<TIn, S, D, C> st;
    st.load(nullptr, kn, vn, t_begin, int(min<int64_t>(C, t_end - t_begin)), false);
    for (int64_t t0 = t_begin; t0 < t_end; t0 += C) {
        __syncthreads();
        st.store_kv(nullptr, KTs, VTs, asum);
        const int64_t t1 = t0 + C;
        if (t1 < t_end) st.load(nullptr, kn, vn, t1, int(min<int64_t>(C, t_end - t1)), false);
        __syncthreads();
        bf16x8 vh[CBW][NKC], vl[CBW][NKC];
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk)
                read_frag<kSplit>(VTs, G::kPitchC, 16 * (w + 4 * cbw) + lr, kk, g, vh[cbw][kk], vl[cbw][kk]);
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) {
                bf16x8 kh, kl;
                read_frag<kSplit>(KTs, G::kPitchC, 16 * sb + lr, kk, g, kh, kl);
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
//   2. W [C][S] = Q / (Abar + eps), in place over Q
//   3. P^T blocks (j-block <= i-block) = K W^T, masked j > i; written as
//      P [C][C] over the dead K tile (upper blocks as zeros)
//   4. O^T [D][C] = B0^T W^T + V^T P^T         wave w: c-blocks w, w+4, ..
//   5. B0 += K^T V                             same c-blocks, all s-blocks
template <typename TIn, int S, int D, int C, int kMinBlocks>
__global__ __launch_bounds__(kThreads, kMinBlocks) void causal_output_mfma_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    TIn* __restrict__ out, const float* __restrict__ records, int64_t T, int tile, int64_t tiles,
    int64_t rec) {
    using G = Geo<TIn, S, D, C>;
    constexpr bool kSplit = G::kSplit;
    constexpr int NSB = S / 16, NBI = C / 16, NKS = S / 32, NKC = C / 32;
    constexpr int SBW = S / 64, CBW = D / 64;
    constexpr int NPB = NBI * NBI;                  // P blocks, lower triangle first
    constexpr int PBW = (NPB + 3) / 4;              // P blocks per wave
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Qs = lds;
    unsigned char* Ks = Qs + G::kQBytes;
    unsigned char* Ps = Ks;
    unsigned char* KTs = Ks + G::kKBytes;
    unsigned char* VTs = KTs + G::kKTBytes;

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, lr = l & 15;
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const TIn* qn = q + n * T * S;
    const TIn* kn = k + n * T * S;
    const TIn* vn = v + n * T * D;
    TIn* on = out + n * T * D;

    // Carried state from the tile's exclusive prefix record.
    const float* rec_p = records + (n * tiles + ti) * rec;
    f32x4 b0[NSB][CBW];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                b0[sb][cbw][rr] = rec_p[(16 * sb + 4 * g + rr) * D + 16 * (w + 4 * cbw) + lr];
    float a0[SBW][4];
#pragma unroll
    for (int sbw = 0; sbw < SBW; ++sbw)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) a0[sbw][rr] = rec_p[S * D + 16 * (w + 4 * sbw) + 4 * g + rr];

    // Lower-triangular ones as a B operand: L^T[j][i] = (j <= i) for j in the
    // permuted k set of step kk and i = 16 bi + lr.
    auto tril_frag = [&](int kk, int bi) {
        bf16x8 f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int j = 32 * kk + 4 * g + (e & 3) + 16 * (e >> 2);
            f[e] = (j <= 16 * bi + lr) ? __bf16(1.0f) : __bf16(0.0f);
        }
        return f;
    };

    Stage<TIn, S, D, C> st;
    st.load(qn, kn, vn, t_begin, int(min<int64_t>(C, t_end - t_begin)), true);
    for (int64_t t0 = t_begin; t0 < t_end; t0 += C) {
        const int cnt = int(min<int64_t>(C, t_end - t0));
        __syncthreads();
        st.store_q(Qs);
        st.store_kv(Ks, KTs, VTs, nullptr);
        const int64_t t1 = t0 + C;
        if (t1 < t_end) st.load(qn, kn, vn, t1, int(min<int64_t>(C, t_end - t1)), true);
        __syncthreads();

        // 1 + 2: running mass and W.
#pragma unroll
        for (int sbw = 0; sbw < SBW; ++sbw) {
            const int sb = w + 4 * sbw;
            bf16x8 kh[NKC], kl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) read_frag<kSplit>(KTs, G::kPitchC, 16 * sb + lr, kk, g, kh[kk], kl[kk]);
            f32x4 last;
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
                f32x4 acc = {a0[sbw][0], a0[sbw][1], a0[sbw][2], a0[sbw][3]};
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    if (32 * kk > 16 * bi + 15) continue;
                    const bf16x8 lf = tril_frag(kk, bi);
                    if constexpr (kSplit) acc = mfma16(kl[kk], lf, acc);
                    acc = mfma16(kh[kk], lf, acc);
                }
                unsigned char* qp = Qs + (16 * bi + lr) * G::kPitchS + (4 * sb + g) * G::kSlot;
                const f32x4 qv = read_q4<kSplit>(qp);
                f32x4 wv;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) wv[rr] = qv[rr] * __builtin_amdgcn_rcpf(acc[rr] + kEps);
                *reinterpret_cast<Slot<kSplit>*>(qp) = make_slot<kSplit>(wv);
                last = acc;
            }
            // Inclusive mass at the chunk's last row (zero rows past cnt add nothing).
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) a0[sbw][rr] = __shfl(last[rr], 16 * g + 15);
        }
        __syncthreads();

        // 3: P^T blocks.
        f32x4 pacc[PBW];
#pragma unroll
        for (int pb = 0; pb < PBW; ++pb) {
            const int idx = w + 4 * pb;
            pacc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (idx >= NPB) continue;
            int bi = 0, bj = 0;
            if (idx < NBI * (NBI + 1) / 2) {
                int rem = idx;
                while (rem > bi) { rem -= bi + 1; ++bi; }
                bj = rem;
            } else {
                continue;  // upper blocks stay zero
            }
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                bf16x8 ah, al, bh, bl;
                read_frag<kSplit>(Ks, G::kPitchS, 16 * bj + lr, kk, g, ah, al);
                read_frag<kSplit>(Qs, G::kPitchS, 16 * bi + lr, kk, g, bh, bl);
                pacc[pb] = mfma3<kSplit>(ah, al, bh, bl, pacc[pb]);
            }
            if (bj == bi) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (4 * g + rr > lr) pacc[pb][rr] = 0.f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int pb = 0; pb < PBW; ++pb) {
            const int idx = w + 4 * pb;
            if (idx >= NPB) continue;
            int bi = 0, bj = 0;
            if (idx < NBI * (NBI + 1) / 2) {
                int rem = idx;
                while (rem > bi) { rem -= bi + 1; ++bi; }
                bj = rem;
            } else {
                int rem = idx - NBI * (NBI + 1) / 2;  // upper blocks (bj > bi), row by row
                bi = 0;
                while (rem >= NBI - 1 - bi) { rem -= NBI - 1 - bi; ++bi; }
                bj = bi + 1 + rem;
            }
            *reinterpret_cast<Slot<kSplit>*>(Ps + (16 * bi + lr) * G::kPitchC + (4 * bj + g) * G::kSlot) =
                make_slot<kSplit>(pacc[pb]);
        }
        __syncthreads();

        // 4 + 5: output and state update for this wave's c-blocks.
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) {
            const int cb = w + 4 * cbw;
            bf16x8 vh[NKC], vl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) read_frag<kSplit>(VTs, G::kPitchC, 16 * cb + lr, kk, g, vh[kk], vl[kk]);
            f32x4 o[NBI];
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) o[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                const f32x4 x0 = b0[2 * kk][cbw], x1 = b0[2 * kk + 1][cbw];
                const Slot<kSplit> s0 = make_slot<kSplit>(x0), s1 = make_slot<kSplit>(x1);
                bf16x8 bh = cat(s0.hi, s1.hi), bl;
                if constexpr (kSplit) bl = cat(s0.lo, s1.lo);
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi) {
                    bf16x8 wh, wl;
                    read_frag<kSplit>(Qs, G::kPitchS, 16 * bi + lr, kk, g, wh, wl);
                    o[bi] = mfma3<kSplit>(bh, bl, wh, wl, o[bi]);
                }
            }
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    if (32 * kk > 16 * bi + 15) continue;
                    bf16x8 ph, pl;
                    read_frag<kSplit>(Ps, G::kPitchC, 16 * bi + lr, kk, g, ph, pl);
                    o[bi] = mfma3<kSplit>(vh[kk], vl[kk], ph, pl, o[bi]);
                }
                const int i = 16 * bi + lr;
                if (i < cnt) store4(on + (t0 + i) * D + 16 * cb + 4 * g, o[bi]);
            }
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    bf16x8 kh, kl;
                    read_frag<kSplit>(KTs, G::kPitchC, 16 * sb + lr, kk, g, kh, kl);
                    b0[sb][cbw] = mfma3<kSplit>(kh, kl, vh[kk], vl[kk], b0[sb][cbw]);
                }
        }
    }
}

template <typename TIn, int S, int D, int C, int kMinBlocks>
hipError_t launch_mfma_family(const void* q, const void* k, const void* v, void* out, float* records,
                              float* state, const Problem& p, hipStream_t stream, Marks* marks) {
    using G = Geo<TIn, S, D, C>;
    if (p.tile % C != 0) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    tile_sums_mfma_kernel<TIn, S, D, C, kMinBlocks><<<grid, kThreads, G::kSumsLds, stream>>>(
        static_cast<const TIn*>(k), static_cast<const TIn*>(v), records, p.T, p.tile, p.tiles, p.rec);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    if ((err = launch_tile_scan(records, state, p, stream)) != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    causal_output_mfma_kernel<TIn, S, D, C, kMinBlocks><<<grid, kThreads, G::kOutputLds, stream>>>(
        static_cast<const TIn*>(q), static_cast<const TIn*>(k), static_cast<const TIn*>(v),
        static_cast<TIn*>(out), records, p.T, p.tile, p.tiles, p.rec);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (marks) return marks->mark(stream);
    return hipSuccess;
}

template <typename TIn>
hipError_t dispatch_mfma(const void* q, const void* k, const void* v, void* out, float* records,
                         float* state, const Problem& p, hipStream_t stream, Marks* marks) {
    if (p.S == 64 && p.d == 64)
        return launch_mfma_family<TIn, 64, 64, 64, 2>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 64 && p.d == 128)
        return launch_mfma_family<TIn, 64, 128, 64, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 128 && p.d == 64)
        return launch_mfma_family<TIn, 128, 64, 64, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 128 && p.d == 128)
        return launch_mfma_family<TIn, 128, 128, 64, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 256 && p.d == 64)
        return launch_mfma_family<TIn, 256, 64, 32, 1>(q, k, v, out, records, state, p, stream, marks);
    if (p.S == 256 && p.d == 128)
        return launch_mfma_family<TIn, 256, 128, 32, 1>(q, k, v, out, records, state, p, stream, marks);
    return hipErrorInvalidValue;
}

}  // namespace

bool mfma_causal_supported(int S, int d) {
    return (S == 64 || S == 128 || S == 256) && (d == 64 || d == 128);
}

hipError_t launch_causal_mfma(const void* q, const void* k, const void* v, void* out,
                              float* records, float* state, const Problem& p, hipStream_t stream,
                              Marks* marks) {
    if (!mfma_causal_supported(p.S, p.d)) return hipErrorInvalidValue;
    if (p.dtype == RACE_BF16)
        return dispatch_mfma<bf16_t>(q, k, v, out, records, state, p, stream, marks);
    return dispatch_mfma<float>(q, k, v, out, records, state, p, stream, marks);
}

}  // namespace race
