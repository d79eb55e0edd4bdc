// hash_stage.h -- the hashing of BatchedACE (src/race_baseline.py:41-44) as a
// stage inside the per-bucket MFMA causal kernels (hashed_causal.hip).  Not
// part of the ABI.
//
// For a token row x (D values), table l < L and plane k < K (R = 2^K
// corners):
//     p_k      = <x, planes[l K + k]>                     (planes [L K][D] fp32)
//     z_k      = 2 tanh(p_k) / sqrt(D)
//     probs[l][r] = softmax_r(sum_k s_{r,k} tanh(p_k) / sqrt(D))
//                 = prod_k sigma(s_{r,k} z_k),  s_{r,k} = +1 iff bit K-1-k of r
// (the corner softmax factorises into independent sigmoids; corner order of
// itertools.product([-1, 1], repeat=K), src/race_baseline.py:30-32).
//
// Steps, per sub-chunk of C tokens:
//   1. projection on the fp32 matrix cores: U^T [planes][tokens] = planes
//      X^T, 16 tokens per wave job.  The token rows go from HBM straight into
//      B-operand registers, the planes (cached) into A-operand registers;
//      fp32 products are exact and accumulate in fp32, as a plain fp32 dot
//      product would, with no operand splitting.
//   2. the plane values z as copysign(sigma(-|z|), z) into U [C][LPP + 1]
//      floats in LDS: tanh |p| = (1 - e1) / (1 + e1) with e1 = exp(-2 |p|) and
//      sigma(-|z|) = e / (1 + e) with e = exp(-|z|), every exponential <= 1.
//   3. corners in quads (4 consecutive r share the planes above the last two):
//      prod over the upper planes times the four products of the last two.
#pragma once

#include "mfma_common.h"

namespace race {
namespace mfma {

// sigma pair (sigma(z), sigma(-z)) of a plane from its stored value
// s = copysign(sigma(-|z|), z); the sign bit (also of -0) picks the order.
__device__ __forceinline__ float2 hs_sigma_pair(float s) {
    const float b = fabsf(s), a = 1.0f - b;
    return (__float_as_uint(s) >> 31) ? make_float2(b, a) : make_float2(a, b);
}

// Projection of one 16-token block of rows against the planes: U^T
// [planes][tokens] = planes X^T, lane (g, lr) receiving D[4 g + r][lr] =
// plane 16 pb + 4 g + r of row lr, as every MFMA here hands it out.  The
// contraction index runs in a fixed bijection in which the four lane groups
// of one 16-byte load instruction hold one contiguous 64-byte run of each
// row (a row is 16 lanes' worth of whole cache lines over the instructions,
// rather than 16-byte pieces 64 bytes apart):
//   fp32 rows: v_mfma_f32_16x16x4_f32; load i of lane group g holds elements
//     16 i + 4 g .. + 3, element j of it is the contraction index of step
//     4 i + j; against fp32 planes, products exact in the fp32 accumulation.
//   bf16 rows: v_mfma_f32_16x16x32_bf16; step kk takes elements 32 kk + 8 g
//     .. + 7 (one 16-byte load) against the planes as three bf16 terms
//     hi + mid + lo (their sum is the fp32 plane to 2^-24); the rows are
//     exact in bf16, so the three products give fp32 accuracy at a quarter of
//     the fp32 MFMA cost.
//   TIn   row element type (float or bf16_t)
//   D     row length (the contraction), a multiple of 32
//   NPB   16-plane blocks (L K <= 16 NPB; planes past L K are zero)
template <typename TIn, int D, int NPB>
struct Projector {
    static constexpr int kSeg = D / 4;                             // values per lane
    static constexpr int kVecs = kSeg * int(sizeof(TIn)) / 16;     // 16-byte loads per lane
    static constexpr bool kF32 = std::is_same<TIn, float>::value;
    static constexpr int kPerVec = 16 / int(sizeof(TIn));          // elements per load
    uint4 x[kVecs];

    // Rows r0 .. r0 + 15 of a row buffer (rows past its range read as zero):
    // load i of lane group g is elements 4 kPerVec i + kPerVec g .. + kPerVec - 1.
    template <int P>
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t xr, int r0, int g, int lr) {
#pragma unroll
        for (int i = 0; i < kVecs; ++i)
            x[i] = buf_load16<P>(xr, ((r0 + lr) * D + 4 * kPerVec * i + kPerVec * g) * int(sizeof(TIn)));
    }

    template <typename PW>
    __device__ __forceinline__ void project(const PW& wp, int g, int lr, f32x4 (&acc)[NPB]) const {
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb) {
            const int row = 16 * pb + lr;
            if constexpr (kF32) {
                // Four accumulators break the dependent chain.
                f32x4 a[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f},
                              {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int s4 = 0; s4 < kSeg; s4 += 4) {
                    const f32x4 w = wp.template get4<D>(row, 16 * (s4 / 4) + 4 * g);
                    const f32x4 xv = __builtin_bit_cast(f32x4, x[s4 / 4]);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        a[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[j], xv[j], a[j], 0, 0, 0);
                }
                acc[pb] = (a[0] + a[1]) + (a[2] + a[3]);
            } else {
                f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < kSeg / 8; ++kk) {
                    const bf16x8 xb = __builtin_bit_cast(bf16x8, x[kk]);
                    const int c = 32 * kk + 8 * g;
                    f32x4& a = (kk & 1) ? a1 : a0;
                    // Smallest terms first.
                    a = mfma16(wp.template get8<D>(2, row, c), xb, a);
                    a = mfma16(wp.template get8<D>(1, row, c), xb, a);
                    a = mfma16(wp.template get8<D>(0, row, c), xb, a);
                }
                acc[pb] = a0 + a1;
            }
        }
    }
};

// Where the planes are staged for the projection: fp32 LDS rows (PlanesLds)
// or the cached planes buffer itself (PlanesGlobal, for kernels whose LDS is
// full) hand the fp32 projection the four values of plane row `row` at
// columns c .. c + 3; PlanesB3 hands the bf16 projection its three terms.
// fp32 rows: padded to D + 4 floats, or (kSwz) D floats with 16-byte chunk
// c / 4 of row `row` at chunk (c / 4) ^ (row % 16).  Either way the 16 rows a
// lane group reads at one column spread over every bank; the padded layout
// reads at immediate offsets from one address, the swizzled one saves the
// padding (256 bytes per 16 rows at D = 64) for an address per chunk.
template <int D, bool kSwz>
__device__ __forceinline__ int plane_at(int row, int c) {
    static_assert(!kSwz || D % 64 == 0, "at least 16 chunks per row for the swizzle");
    return kSwz ? row * D + 4 * ((c >> 2) ^ (row & 15)) : row * (D + 4) + c;
}
template <bool kSwz>
struct PlanesLdsT {
    const float* w;
    template <int D>
    __device__ __forceinline__ f32x4 get4(int row, int c) const {
        return *reinterpret_cast<const f32x4*>(w + plane_at<D, kSwz>(row, c));
    }
};
using PlanesLds = PlanesLdsT<false>;
// The planes as three bf16 terms (hi, mid, lo) in LDS, [3][16 NPB][D + 8]
// (the padding spreads a 16-lane column of rows over the banks): the A
// operand of the bf16 projection.
struct PlanesB3 {
    const unsigned char* w;
    int rows;  // 16 NPB
    template <int D>
    __device__ __forceinline__ bf16x8 get8(int term, int row, int c) const {
        return *reinterpret_cast<const bf16x8*>(w + ((term * rows + row) * (D + 8) + c) * 2);
    }
};
struct PlanesGlobal {
    __amdgpu_buffer_rsrc_t r;  // over [LK][D] fp32; rows past LK read as zero
    template <int D>
    __device__ __forceinline__ f32x4 get4(int row, int c) const {
        return __builtin_bit_cast(f32x4, buf_load16<kPolicyDefault>(r, (row * D + c) * 4));
    }
};

// The planes [LK][D] fp32 into LDS rows as PlanesLdsT<kSwz> reads them, rows
// LK .. 16 NPB - 1 zero.
// Cooperative over the NT threads of the workgroup; the caller synchronizes.
template <int D, int NPB, int NT, bool kSwz = false>
__device__ __forceinline__ void stage_planes(float* Wl, const float* __restrict__ planes, int LK) {
    for (int e = threadIdx.x; e < 16 * NPB * (D / 4); e += NT) {
        const int row = e / (D / 4), c4 = 4 * (e % (D / 4));
        f32x4 w = {0.f, 0.f, 0.f, 0.f};
        if (row < LK) w = *reinterpret_cast<const f32x4*>(planes + row * D + c4);
        *reinterpret_cast<f32x4*>(Wl + plane_at<D, kSwz>(row, c4)) = w;
    }
}

// The planes [LK][D] fp32 as bf16 terms into PlanesB3's layout, rows LK ..
// 16 NPB - 1 zero.  Cooperative; the caller synchronizes.
template <int D, int NPB, int NT>
__device__ __forceinline__ void stage_planes_b3(unsigned char* Wb, const float* __restrict__ planes, int LK) {
    constexpr int kRows = 16 * NPB;
    for (int e = threadIdx.x; e < kRows * (D / 4); e += NT) {
        const int row = e / (D / 4), c4 = 4 * (e % (D / 4));
        f32x4 w = {0.f, 0.f, 0.f, 0.f};
        if (row < LK) w = *reinterpret_cast<const f32x4*>(planes + row * D + c4);
        uint2 t[3];
        f32x4 r = w;
#pragma unroll
        for (int term = 0; term < 3; ++term) {
            t[term] = make_uint2(pack2(r[0], r[1]), pack2(r[2], r[3]));
            r = r - f32x4{lo_half(t[term].x), hi_half(t[term].x), lo_half(t[term].y), hi_half(t[term].y)};
        }
#pragma unroll
        for (int term = 0; term < 3; ++term)
            *reinterpret_cast<uint2*>(Wb + ((term * kRows + row) * (D + 8) + c4) * 2) = t[term];
    }
}

// LDS of the staged planes for rows of TIn.
template <typename TIn, int D, int NPB, bool kSwz = false>
constexpr int planes_lds_bytes() {
    return std::is_same<TIn, float>::value ? 16 * NPB * (kSwz ? D : D + 4) * 4 : 3 * 16 * NPB * (D + 8) * 2;
}

// z = scale2 tanh(p) of the projections in acc (scale2 = 2 / sqrt(D)),
// stored as copysign(sigma(-|z|), z) at U[token][plane] for token t and the
// lane's planes 16 pb + 4 g + r.
template <int NPB>
__device__ __forceinline__ void hs_write_sigmas(float* U, int pitch, int t, const f32x4 (&acc)[NPB],
                                                float scale2, int g) {
    constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
    for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float x = acc[pb][rr];
            const float e1 = __builtin_amdgcn_exp2f(-2.0f * kLog2e * fabsf(x));
            const float th = (1.0f - e1) * __builtin_amdgcn_rcpf(1.0f + e1);
            const float z = scale2 * copysignf(th, x);
            const float e = __builtin_amdgcn_exp2f(-kLog2e * fabsf(z));
            const float b = e * __builtin_amdgcn_rcpf(1.0f + e);
            U[t * pitch + 16 * pb + 4 * g + rr] = copysignf(b, z);
        }
}

// The corners of one table from its KP stored plane values (KP >= 2; plane 0
// the most significant bit of r), decoded once: quad m (corners 4 m .. 4 m +
// 3) is the product over the upper KP - 2 planes, chosen by the bits of m,
// times the four products of the last two planes.
template <int KP>
struct CornerTable {
    float2 sp[KP];
    f32x4 low;
    __device__ __forceinline__ void decode(const float* u) {
#pragma unroll
        for (int p = 0; p < KP; ++p) sp[p] = hs_sigma_pair(u[p]);
        const float2 s1 = sp[KP - 2], s2 = sp[KP - 1];
        low = f32x4{s1.y * s2.y, s1.y * s2.x, s1.x * s2.y, s1.x * s2.x};
    }
    __device__ __forceinline__ f32x4 quad(int m) const {
        float base = 1.f;
#pragma unroll
        for (int p = 0; p < KP - 2; ++p) base *= ((m >> (KP - 3 - p)) & 1) ? sp[p].x : sp[p].y;
        return base * low;
    }
};

}  // namespace mfma
}  // namespace race
