// alg1.hip -- causal RACE attention with the hashing inside and one global
// normalization per query (paper Algorithm 1 made causal) on gfx950 matrix
// cores.  This is the function of the reference's causal v2 forward
// (src/causal_v2/kernels/race_causal_fwd.h:6-10; ground truth
// src/causal_v2/reference.py:100-128):
//
//   Phi(x) in R^S, S = L R, R = 2^P, table-major (s = l R + r):
//       u_p        = tanh(<W[l][p], x>)                       (W [L][P][D] fp32)
//       Phi_l(x)[r] = softmax_r(beta sum_p u_p c_{r,p})
//                  = prod_p (c_{r,p} = +1 ? sigma(2 beta u_p) : sigma(-2 beta u_p))
//       (c_{r,p} = +1 iff bit P-1-p of r is set; the softmax factorises into
//       the Bernoulli product, src/noncausal/reference.py:103-125)
//   B_t = sum_{j<=t} Phi(k_j) (x) v_j,   A_t = sum_{j<=t} Phi(k_j)
//   out_t = (Phi(q_t) . B_t) / (Phi(q_t) . A_t), 0 where the denominator is 0.
//
// Launches (the three-launch decomposition of race_causal_fwd.h:23-27):
//   1. alg1_sums_kernel    per (tile, stream): hashes the tile's keys and
//                          writes B_tile = Phi_K^T V and A_tile = colsum Phi_K
//                          into the tile record (B [S][D] then A [S])
//   2. tile_scan_kernel    exclusive scan of the records (valu_kernels.hip)
//   3. alg1_output_kernel  per (tile, stream): walks 64-token sub-chunks from
//                          the tile's exclusive prefix, with, per sub-chunk,
//                            Abar = A0 + Phi_K^T tril(1)      (running mass)
//                            den_i = Phi_Q,i . Abar_i          (= Phi_Q,i . A_i)
//                            G   = tril(Phi_Q Phi_K^T)
//                            out = (Phi_Q B0 + G V) / den
//                            A0 += colsum Phi_K,  B0 += Phi_K^T V.
// Hashing runs on the MFMA too: U^T = W X^T (q, k, v arrive as bf16, exact
// operands; W as three bf16 terms in the fp32 variant, two in the bf16 one),
// then tanh and the two sigmoids of every plane, then the corner products
// (plane 0 the most significant bit).
//
// Every LDS tile is stored with tokens as rows (q, k, v rows, Phi_Q, Phi_K).
// The products that contract over tokens (Phi_K^T V, Phi_K^T tril(1), V^T G^T)
// take their operand fragments with gfx950's transposing LDS read
// (ds_read_b64_tr_b16, Plane::frag_tr), so no tile is ever written twice.
//
// Two rounding variants, chosen by the template flag kPhiSplit (the
// reference's v2a / v2b split, race_causal_fwd.h:33-41):
//   kPhiSplit = true   Phi_Q and Phi_K enter every product as bf16 hi/lo
//                      pairs (three products), so the result is fp32-accurate
//                      up to a ~2^-17 relative error per product;
//   kPhiSplit = false  Phi_Q and Phi_K are rounded to bf16 once (one product);
//                      the masked Gram matrix G and the carried state B0 stay
//                      hi/lo, the rounding points of the reference's v2b.
// The carried state and G are hi/lo in both.
//
// Padding: S is padded to SP in {32, 64, 128} buckets and the L*P planes to
// LPP in {16, 32}; padded buckets have Phi = 0 and padded planes W = 0.  Rows
// past the sequence read as zero through the buffer resources, and their
// Phi_K is set to 0 (phi(0) = 1/R, not 0, so zero keys alone would add mass).
#include <cmath>

#include "mfma_common.h"

namespace race {
namespace {

using namespace mfma;

constexpr int kA1Chunk = 64;  // tokens per sub-chunk (C)

// acc += A B where A and/or B are bf16 hi/lo pairs (small terms first).
template <bool kSA, bool kSB>
__device__ __forceinline__ f32x4 mfma_mix(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                          const bf16x8& bl, f32x4 acc) {
    if constexpr (kSA) acc = mfma16(al, bh, acc);
    if constexpr (kSB) acc = mfma16(ah, bl, acc);
    return mfma16(ah, bh, acc);
}

// One float as bf16 hi (and lo) bit patterns.
template <bool kSplit>
__device__ __forceinline__ void split1(float x, uint16_t& hi, uint16_t& lo) {
    const uint32_t h = pack2(x, 0.f);
    hi = uint16_t(h & 0xffffu);
    lo = 0;
    if constexpr (kSplit) lo = uint16_t(pack2(x - lo_half(h), 0.f) & 0xffffu);
}

__device__ __forceinline__ uint32_t word4(const uint4& u, int i) {
    return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w;
}

// Four consecutive elements k0 .. k0 + 3 (k0 % 4 == 0) of a plane row as
// floats (hi + lo).
template <typename PL, bool kSplit>
__device__ __forceinline__ f32x4 get4(const unsigned char* t, int row, int k0) {
    const int pos = fpos(k0);
    const unsigned char* p = t + row * PL::kPitch + 16 * ((pos >> 3) ^ PL::sw(row)) + 8 * ((pos >> 2) & 1);
    const uint2 h = *reinterpret_cast<const uint2*>(p);
    f32x4 r = {lo_half(h.x), hi_half(h.x), lo_half(h.y), hi_half(h.y)};
    if constexpr (kSplit) {
        const uint2 l = *reinterpret_cast<const uint2*>(p + PL::kLoOff);
        r += f32x4{lo_half(l.x), hi_half(l.x), lo_half(l.y), hi_half(l.y)};
    }
    return r;
}

// The sigmoid pair (sigma(z), sigma(-z)) of a plane from its stored value
// s = copysign(sigma(-|z|), z): sigma(|z|) = 1 - sigma(-|z|) >= 1/2 is formed
// without cancellation, and the sign bit (also of -0) picks the order.
__device__ __forceinline__ float2 sigma_pair(float s) {
    const float b = fabsf(s), a = 1.0f - b;
    return (__float_as_uint(s) >> 31) ? make_float2(b, a) : make_float2(a, b);
}

template <bool kPhiSplit, int SP, int D, int LPP>
struct A1Geo {
    static constexpr int C = kA1Chunk;
    static constexpr int kD = D;
    using PX = Plane<false, D>;       // token rows over features: the q, k, v rows (bf16)
    using PW = Plane<true, D>;        // plane rows over features: W as hi/lo
    using PW3 = Plane<false, D>;      // plane rows over features: third bf16 term of W
    using PS = Plane<kPhiSplit, SP>;  // token rows over buckets: Phi_Q, Phi_K
    using PG = Plane<true, C>;        // query rows over keys: G
    static constexpr int kUPitch = LPP + 1;  // floats per token: one per plane
    static constexpr int kUBytes = C * kUPitch * 4;
    static constexpr int kXBytes = C * PX::kPitch;
    static constexpr int kPhiBytes = C * PS::kPitch;
    static constexpr int kGBytes = C * PG::kPitch;
    static constexpr int kDenBytes = 4 * C * 4;
    static constexpr int mx(int a, int b) { return a > b ? a : b; }
    // Output pass: region A holds the q and k rows, then Phi_Q and Phi_K;
    // then G; region U the plane values of q and k, then the partial
    // denominators; the V rows; W.
    static constexpr int kRegionOut = mx(2 * kXBytes, 2 * kPhiBytes);
    static constexpr int kRegionU = mx(2 * kUBytes, kDenBytes);
    // W = hi + mid + lo in the fp32 variant where the output pass still fits
    // 160 KB of LDS (the projection is then exact in fp32 arithmetic), hi + mid
    // otherwise and in the bf16 variant.
    static constexpr int kOutBase = kRegionOut + kGBytes + kRegionU + kXBytes + LPP * PW::kPitch;
    static constexpr bool kW3 = kPhiSplit && kOutBase + LPP * PW3::kPitch <= 160 * 1024;
    static constexpr int kWBytes = LPP * PW::kPitch + (kW3 ? LPP * PW3::kPitch : 0);
    static constexpr int kOutputLds = kOutBase + kWBytes - LPP * PW::kPitch;
    // Tile sums: the k rows, then Phi_K; U; the V rows; W.
    static constexpr int kRegionSums = mx(kXBytes, kPhiBytes);
    static constexpr int kSumsLds = kRegionSums + kUBytes + kXBytes + kWBytes;
    static constexpr int kOutBlocks = kOutputLds <= 80 * 1024 ? 2 : 1;
    // (S = D = 128 holds a 128 x 128 accumulator tile: one workgroup per CU.)
    static constexpr int kSumsBlocks = kSumsLds <= 80 * 1024 && SP * D < 128 * 128 ? 2 : 1;
    static constexpr int NSB = SP / 16, NBI = C / 16, NKS = SP / 32, NKC = C / 32, NKD = D / 32;
    static constexpr int CBW = D / 64;         // c-blocks per wave
    static constexpr int SBW = (NSB + 3) / 4;  // s-blocks per wave
    static constexpr int NPB = LPP / 16;       // plane blocks
    static_assert(C * D % (8 * kThreads) == 0, "row staging");
    static_assert(kOutputLds <= 160 * 1024, "output pass LDS");
};

// Raw registers of one sub-chunk: the token rows of NX bf16 tensors, as
// 16-byte vectors (8 features); vector e of a thread is row e / (D / 8).
template <int D, int NX>
struct A1Stage {
    static constexpr int kPer = kA1Chunk * D / 8 / kThreads;
    uint4 x[NX][kPer];

    __device__ __forceinline__ void load(const __amdgpu_buffer_rsrc_t (&xr)[NX], int r0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int e = tid + p * kThreads, t = e / (D / 8), b = e % (D / 8);
#pragma unroll
            for (int i = 0; i < NX; ++i)
                x[i][p] = buf_load16<kOutKVPolicy>(xr[i], ((r0 + t) * D + 8 * b) * 2);
        }
    }

    // Rows into token-row planes.
    template <typename PX>
    __device__ __forceinline__ void store(unsigned char* const (&X)[NX]) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int e = tid + p * kThreads, t = e / (D / 8), b = e % (D / 8);
#pragma unroll
            for (int i = 0; i < NX; ++i) {
                PX::put4(X[i], t, 8 * b, make_uint2(x[i][p].x, x[i][p].y), make_uint2(0, 0));
                PX::put4(X[i], t, 8 * b + 4, make_uint2(x[i][p].z, x[i][p].w), make_uint2(0, 0));
            }
        }
    }
};

// The planes W [L][P][D] as bf16 plane rows j = l P + p (rows past L*P
// zero): hi and mid in the hi/lo plane Ws, and with G::kW3 the third term
// lo = bf16(W - hi - mid) in the plane after it.
template <typename G, bool kPhiSplit>
__device__ __forceinline__ void load_planes(unsigned char* Ws, const float* __restrict__ W, int LP) {
    constexpr int kD = G::kD;
    unsigned char* W3 = Ws + 16 * G::NPB * G::PW::kPitch;
    for (int e = threadIdx.x; e < 16 * G::NPB * kD / 4; e += kThreads) {
        const int j = e / (kD / 4), c0 = 4 * (e % (kD / 4));
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (j < LP) x = *reinterpret_cast<const f32x4*>(W + j * kD + c0);
        uint2 hi, mid;
        split4<true>(x[0], x[1], x[2], x[3], hi, mid);
        G::PW::put4(Ws, j, c0, hi, mid);
        if constexpr (G::kW3) {
            const f32x4 r = {(x[0] - lo_half(hi.x)) - lo_half(mid.x), (x[1] - hi_half(hi.x)) - hi_half(mid.x),
                             (x[2] - lo_half(hi.y)) - lo_half(mid.y), (x[3] - hi_half(hi.y)) - hi_half(mid.y)};
            const uint2 lo = make_uint2(pack2(r[0], r[1]), pack2(r[2], r[3]));
            G::PW3::put4(W3, j, c0, lo, lo);
        }
    }
}

// U^T blocks of one x plane: wave w takes token block w; lane (g, lr) gets
// plane 16 pb + 4 g + r of token 16 w + lr.  The x rows are exact bf16, so
// each term of W contributes one exact product.
template <typename G, bool kPhiSplit>
__device__ __forceinline__ void project(const unsigned char* X, const unsigned char* Ws, int w, int g,
                                        int lr, f32x4 (&acc)[G::NPB]) {
    const unsigned char* W3 = Ws + 16 * G::NPB * G::PW::kPitch;
#pragma unroll
    for (int pb = 0; pb < G::NPB; ++pb) acc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < G::NKD; ++kk) {
        bf16x8 xh, xl;
        G::PX::frag(X, 16 * w + lr, kk, g, xh, xl);
#pragma unroll
        for (int pb = 0; pb < G::NPB; ++pb) {
            bf16x8 wh, wm;
            G::PW::frag(Ws, 16 * pb + lr, kk, g, wh, wm);
            if constexpr (G::kW3) {
                bf16x8 wl, unused;
                G::PW3::frag(W3, 16 * pb + lr, kk, g, wl, unused);
                acc[pb] = mfma16(wl, xh, acc[pb]);
            }
            acc[pb] = mfma_mix<true, false>(wh, wm, xh, xh, acc[pb]);
        }
    }
}

// z = 2 beta tanh(u) of the projections in `acc`, stored as
// copysign(sigma(-|z|), z) in U [C][kUPitch] (one float per token and plane).
// tanh |u| = (1 - e1) / (1 + e1) with e1 = exp(-2|u|), sigma(-|z|) = e / (1 + e)
// with e = exp(-|z|): every exponential is <= 1, so nothing overflows at any
// beta, and both are accurate to a few fp32 ulps in absolute terms.
template <typename G>
__device__ __forceinline__ void write_sigmas(float* U, const f32x4 (&acc)[G::NPB], float beta2, int w,
                                             int g, int lr) {
    constexpr float kLog2e = 1.4426950408889634f;
    const int t = 16 * w + lr;
#pragma unroll
    for (int pb = 0; pb < G::NPB; ++pb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float x = acc[pb][rr];
            const float e1 = __builtin_amdgcn_exp2f(-2.0f * kLog2e * fabsf(x));
            const float th = (1.0f - e1) * __builtin_amdgcn_rcpf(1.0f + e1);
            const float z = beta2 * copysignf(th, x);
            const float e = __builtin_amdgcn_exp2f(-kLog2e * fabsf(z));
            const float b = e * __builtin_amdgcn_rcpf(1.0f + e);
            U[t * G::kUPitch + 16 * pb + 4 * g + rr] = copysignf(b, z);
        }
}

// Phi of the sub-chunk's C tokens from U into a token-row plane; tokens >=
// valid get 0.  Item (t, l) = (tid % 64, tid / 64), one per thread: the P
// sigmoid pairs of token t, table l are decoded once; the corners go out in
// quads, the planes above the last two selecting by the bits of the quad
// index (plane 0 the most significant bit of r) and the last two giving the
// quad's four corners.  The item's U offset and its quads' LDS offsets are
// fixed for the whole tile and computed once.
template <typename PS, bool kSplit, int kUP>
struct RowBuilder {
    int t, uoff, P, R;
    bool active;
    int poff[8];  // byte offsets of corners 4 m .. 4 m + 3 of row t

    __device__ __forceinline__ void init(int L, int P_) {
        const int e = threadIdx.x, l = e / kA1Chunk;
        t = e % kA1Chunk;
        P = P_;
        R = 1 << P_;
        active = e < kA1Chunk * L;
        uoff = t * kUP + l * P_;
#pragma unroll
        for (int m = 0; m < 8; ++m) poff[m] = 4 * m < R ? PS::off4(t, (l << P_) + 4 * m) : 0;
    }

    __device__ __forceinline__ void build(const float* U, unsigned char* Ph, int valid) const {
        if (!active) return;
        const float* ur = U + uoff;
        const float live = t < valid ? 1.f : 0.f;
        if (P >= 2) {
            float2 hp[3];
#pragma unroll
            for (int p = 0; p < 3; ++p) hp[p] = p < P - 2 ? sigma_pair(ur[p]) : make_float2(1.f, 1.f);
            const float2 s1 = sigma_pair(ur[P - 2]), s2 = sigma_pair(ur[P - 1]);
            const float q0 = s1.y * s2.y, q1 = s1.y * s2.x, q2 = s1.x * s2.y, q3 = s1.x * s2.x;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                if (4 * m >= R) continue;
                float base = live;
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    if (p < P - 2) base *= ((m >> (P - 3 - p)) & 1) ? hp[p].x : hp[p].y;
                uint2 hi, lo;
                split4<kSplit>(base * q0, base * q1, base * q2, base * q3, hi, lo);
                *reinterpret_cast<uint2*>(Ph + poff[m]) = hi;
                if constexpr (kSplit) *reinterpret_cast<uint2*>(Ph + poff[m] + PS::kLoOff) = lo;
            }
        } else {
            const float2 sp = sigma_pair(ur[0]);
            const float x[2] = {live * sp.y, live * sp.x};
            const int l = threadIdx.x / kA1Chunk;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                uint16_t hi, lo;
                split1<kSplit>(x[r], hi, lo);
                PS::put1(Ph, t, 2 * l + r, hi, lo);
            }
        }
    }
};

// Zero buckets S .. SP - 1 of every row of a token-row Phi plane.
template <typename PL, int SP>
__device__ __forceinline__ void zero_pad_rows(unsigned char* Ph, int S) {
    const int pad = SP - S;
    for (int e = threadIdx.x; e < kA1Chunk * pad; e += kThreads) {
        const int t = e / pad, s = S + e % pad;
        PL::put1(Ph, t, s, 0, 0);
    }
}

// ---------------------------------------------------------------------------
// K1: per (tile, stream) B_tile = Phi_K^T V and A_tile = colsum Phi_K.  Wave w
// owns the V columns of c-blocks w, w + 4 (all s-blocks) and the A entries of
// s-blocks w, w + 4.
template <bool kPhiSplit, int SP, int D, int LPP>
__global__ __launch_bounds__(kThreads, (A1Geo<kPhiSplit, SP, D, LPP>::kSumsBlocks)) void alg1_sums_kernel(
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const float* __restrict__ W,
    const float* __restrict__ beta_p, float* __restrict__ records, int64_t T, int tile, int64_t tiles,
    int64_t rec, int L, int P) {
    using G = A1Geo<kPhiSplit, SP, D, LPP>;
    using PS = typename G::PS;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Xk = lds;
    unsigned char* PhK = lds;  // once the k rows are projected
    float* U = reinterpret_cast<float*>(lds + G::kRegionSums);
    unsigned char* Vs = lds + G::kRegionSums + G::kUBytes;
    unsigned char* Ws = Vs + G::kXBytes;

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min(T, t_begin + tile) - t_begin);
    const int S = L << P;
    const float beta2 = 2.0f * beta_p[0];
    const __amdgpu_buffer_rsrc_t xr[2] = {make_rsrc(k + (n * T + t_begin) * D, int64_t(rows) * D * 2),
                                          make_rsrc(v + (n * T + t_begin) * D, int64_t(rows) * D * 2)};

    load_planes<G, kPhiSplit>(Ws, W, L * P);

    f32x4 bacc[G::NSB][G::CBW], aacc[G::SBW];
#pragma unroll
    for (int sb = 0; sb < G::NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < G::CBW; ++cbw) bacc[sb][cbw] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < G::SBW; ++j) aacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = __bf16(1.0f);
    unsigned char* const Xs[2] = {Xk, Vs};

    RowBuilder<PS, kPhiSplit, G::kUPitch> rb;
    rb.init(L, P);

    A1Stage<D, 2> st;
    st.load(xr, 0);
    for (int r0 = 0; r0 < rows; r0 += kA1Chunk) {
        __syncthreads();
        st.template store<typename G::PX>(Xs);
        st.load(xr, r0 + kA1Chunk);  // past the tile: zeros, never used
        __syncthreads();
        f32x4 uk[G::NPB];
        project<G, kPhiSplit>(Xk, Ws, w, g, lr, uk);
        write_sigmas<G>(U, uk, beta2, w, g, lr);
        __syncthreads();  // the k rows are dead: Phi_K takes their space
        rb.build(U, PhK, rows - r0);
        if (SP > S) zero_pad_rows<PS, SP>(PhK, S);
        __syncthreads();
        // Phi_K^T and V fragments straight from the token-row planes.
#pragma unroll
        for (int cbw = 0; cbw < G::CBW; ++cbw) {
            bf16x8 vh[G::NKC];
#pragma unroll
            for (int kk = 0; kk < G::NKC; ++kk) {
                bf16x8 dummy;
                G::PX::frag_tr(Vs, 32 * kk, 16 * (w + 4 * cbw), g, lr, vh[kk], dummy);
            }
#pragma unroll
            for (int sb = 0; sb < G::NSB; ++sb)
#pragma unroll
                for (int kk = 0; kk < G::NKC; ++kk) {
                    bf16x8 kh, kl;
                    PS::frag_tr(PhK, 32 * kk, 16 * sb, g, lr, kh, kl);
                    bacc[sb][cbw] = mfma_mix<kPhiSplit, false>(kh, kl, vh[kk], vh[kk], bacc[sb][cbw]);
                }
        }
#pragma unroll
        for (int j = 0; j < G::SBW; ++j) {
            const int sb = w + 4 * j;
            if (sb >= G::NSB) continue;
#pragma unroll
            for (int kk = 0; kk < G::NKC; ++kk) {
                bf16x8 kh, kl;
                PS::frag_tr(PhK, 32 * kk, 16 * sb, g, lr, kh, kl);
                aacc[j] = mfma_mix<kPhiSplit, false>(kh, kl, ones, ones, aacc[j]);
            }
        }
    }

    float* r = records + (n * tiles + ti) * rec;
#pragma unroll
    for (int sb = 0; sb < G::NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < G::CBW; ++cbw)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int s = 16 * sb + 4 * g + rr;
                if (s < S) r[s * D + 16 * (w + 4 * cbw) + lr] = bacc[sb][cbw][rr];
            }
#pragma unroll
    for (int j = 0; j < G::SBW; ++j) {
        const int sb = w + 4 * j;
        if (sb >= G::NSB || lr != 0) continue;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int s = 16 * sb + 4 * g + rr;
            if (s < S) r[S * D + s] = aacc[j][rr];
        }
    }
}

// ---------------------------------------------------------------------------
// K3: the output pass, one workgroup per (tile, stream).  Per sub-chunk (the
// numbers are the barriers): stage the q, k, v rows (1) -> project q, k and
// store their plane values (2) -> Phi_Q, Phi_K (3) -> running mass,
// denominators, G blocks (4) -> output and state update.
template <bool kPhiSplit, int SP, int D, int LPP>
__global__ __launch_bounds__(kThreads, (A1Geo<kPhiSplit, SP, D, LPP>::kOutBlocks)) void alg1_output_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const float* __restrict__ W, const float* __restrict__ beta_p, bf16_t* __restrict__ out,
    const float* __restrict__ records, int64_t T, int tile, int64_t tiles, int64_t rec, int L, int P) {
    using G = A1Geo<kPhiSplit, SP, D, LPP>;
    using PS = typename G::PS;
    using PG = typename G::PG;
    constexpr int NSB = G::NSB, NBI = G::NBI, NKS = G::NKS, NKC = G::NKC, CBW = G::CBW, SBW = G::SBW;
    constexpr int NLB = NBI * (NBI + 1) / 2;  // lower-triangular G blocks
    constexpr int PBW = (NLB + 3) / 4;        // G blocks per wave
    constexpr int C = kA1Chunk;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Xq = lds;
    unsigned char* Xk = lds + G::kXBytes;
    unsigned char* PhQ = lds;  // once the q and k rows are projected
    unsigned char* PhK = lds + G::kPhiBytes;
    unsigned char* Gs = lds + G::kRegionOut;
    float* Uq = reinterpret_cast<float*>(Gs + G::kGBytes);
    float* Uk = Uq + C * G::kUPitch;
    float* denp = Uq;  // [4][C], once the builder has read U
    unsigned char* Vs = Gs + G::kGBytes + G::kRegionU;
    unsigned char* Ws = Vs + G::kXBytes;

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n = blockIdx.y, ti = blockIdx.x;
    const int64_t t_begin = ti * tile;
    const int rows = int(min(T, t_begin + tile) - t_begin);
    const int S = L << P;
    const float beta2 = 2.0f * beta_p[0];
    const int64_t bytes = int64_t(rows) * D * 2;
    const __amdgpu_buffer_rsrc_t xr[3] = {make_rsrc(q + (n * T + t_begin) * D, bytes),
                                          make_rsrc(k + (n * T + t_begin) * D, bytes),
                                          make_rsrc(v + (n * T + t_begin) * D, bytes)};
    const __amdgpu_buffer_rsrc_t or_ = make_rsrc(out + (n * T + t_begin) * D, bytes);

    load_planes<G, kPhiSplit>(Ws, W, L * P);

    // Carried state from the tile's exclusive prefix record (zero past S).
    const float* rp = records + (n * tiles + ti) * rec;
    f32x4 b0[NSB][CBW];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int s = 16 * sb + 4 * g + rr;
                b0[sb][cbw][rr] = s < S ? rp[s * D + 16 * (w + 4 * cbw) + lr] : 0.f;
            }
    float a0[SBW][4];
#pragma unroll
    for (int j = 0; j < SBW; ++j)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int s = 16 * (w + 4 * j) + 4 * g + rr;
            a0[j][rr] = s < S ? rp[S * D + s] : 0.f;
        }

    const bf16x8 tri0 = tril_frag(0, g, lr), tri1 = tril_frag(16, g, lr);
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = __bf16(1.0f);
    unsigned char* const Xs[3] = {Xq, Xk, Vs};

    RowBuilder<PS, kPhiSplit, G::kUPitch> rb;
    rb.init(L, P);
    // The lower-triangular G blocks of this wave, round robin: block index
    // w + 4 pb is (bi, bj) with bj <= bi.
    int pbi[PBW], pbj[PBW];
#pragma unroll
    for (int pb = 0; pb < PBW; ++pb) {
        int bi = 0, rem = w + 4 * pb;
        while (rem > bi) {
            rem -= bi + 1;
            ++bi;
        }
        pbi[pb] = bi;
        pbj[pb] = rem;
    }

    A1Stage<D, 3> st;
    st.load(xr, 0);
    for (int r0 = 0; r0 < rows; r0 += C) {
        __syncthreads();
        st.template store<typename G::PX>(Xs);
        st.load(xr, r0 + C);  // past the tile: zeros, never used
        __syncthreads();  // (1)
        f32x4 uq[G::NPB], uk[G::NPB];
        project<G, kPhiSplit>(Xq, Ws, w, g, lr, uq);
        project<G, kPhiSplit>(Xk, Ws, w, g, lr, uk);
        write_sigmas<G>(Uq, uq, beta2, w, g, lr);
        write_sigmas<G>(Uk, uk, beta2, w, g, lr);
        __syncthreads();  // (2) the x planes are dead: Phi_Q and Phi_K take their space
        rb.build(Uq, PhQ, C);
        rb.build(Uk, PhK, rows - r0);
        if (SP > S) {
            zero_pad_rows<PS, SP>(PhQ, S);
            zero_pad_rows<PS, SP>(PhK, S);
        }
        __syncthreads();  // (3) U is dead: the partial denominators take its space

        // Running mass Abar^T [s][i] = A0 + Phi_K^T tril(1) for this wave's
        // s-blocks, and the partial denominators sum_s Phi_Q[i][s] Abar[s][i].
        float dsum[NBI];
#pragma unroll
        for (int bi = 0; bi < NBI; ++bi) dsum[bi] = 0.f;
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const int sb = w + 4 * j;
            if (sb >= NSB) continue;
            bf16x8 kh[NKC], kl[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) PS::frag_tr(PhK, 32 * kk, 16 * sb, g, lr, kh[kk], kl[kk]);
            f32x4 last;
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
                f32x4 acc = {a0[j][0], a0[j][1], a0[j][2], a0[j][3]};
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    const int off = 16 * bi - 32 * kk;
                    if (off < 0) continue;
                    const bf16x8& lf = off == 0 ? tri0 : off == 16 ? tri1 : ones;
                    if constexpr (kPhiSplit) acc = mfma16(kl[kk], lf, acc);
                    acc = mfma16(kh[kk], lf, acc);
                }
                const f32x4 fq = get4<PS, kPhiSplit>(PhQ, 16 * bi + lr, 16 * sb + 4 * g);
                dsum[bi] += ((fq[0] * acc[0] + fq[1] * acc[1]) + fq[2] * acc[2]) + fq[3] * acc[3];
                last = acc;
            }
            // Inclusive mass at the chunk's last row (rows past the tile add nothing).
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) a0[j][rr] = __shfl(last[rr], 16 * g + 15);
        }
#pragma unroll
        for (int bi = 0; bi < NBI; ++bi) {
            float x = dsum[bi];
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            if (g == 0) denp[w * C + 16 * bi + lr] = x;
        }

        // G^T blocks of the lower triangle, round robin over the waves:
        // lane (g, lr) of block (bi, bj) holds G[16 bi + lr][16 bj + 4 g + r].
        f32x4 pacc[PBW];
#pragma unroll
        for (int pb = 0; pb < PBW; ++pb) {
            const int bi = pbi[pb], rem = pbj[pb];
            pacc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (w + 4 * pb >= NLB) continue;
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                bf16x8 ah, al, bh, bl_;
                PS::frag(PhK, 16 * rem + lr, kk, g, ah, al);
                PS::frag(PhQ, 16 * bi + lr, kk, g, bh, bl_);
                pacc[pb] = mfma3<kPhiSplit>(ah, al, bh, bl_, pacc[pb]);
            }
            if (rem == bi) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (4 * g + rr > lr) pacc[pb][rr] = 0.f;
            }
        }
#pragma unroll
        for (int pb = 0; pb < PBW; ++pb) {
            if (w + 4 * pb >= NLB) continue;
            uint2 hi, lo;
            split4<true>(pacc[pb][0], pacc[pb][1], pacc[pb][2], pacc[pb][3], hi, lo);
            PG::put4(Gs, 16 * pbi[pb] + lr, 16 * pbj[pb] + 4 * g, hi, lo);
        }
        __syncthreads();  // (4)

        // Reciprocal denominators of this lane's query rows (fixed wave order).
        float rden[NBI];
#pragma unroll
        for (int bi = 0; bi < NBI; ++bi) {
            const int i = 16 * bi + lr;
            const float den = ((denp[i] + denp[C + i]) + denp[2 * C + i]) + denp[3 * C + i];
            rden[bi] = den == 0.f ? 0.f : __builtin_amdgcn_rcpf(den);  // 1 ulp; the output is bf16
        }

        // Output and state update for this wave's c-blocks.
#pragma unroll
        for (int cbw = 0; cbw < CBW; ++cbw) {
            const int cb = w + 4 * cbw;
            bf16x8 vh[NKC];
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk) {
                bf16x8 dummy;
                G::PX::frag_tr(Vs, 32 * kk, 16 * cb, g, lr, vh[kk], dummy);
            }
            f32x4 o[NBI];
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) o[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                const f32x4 x0 = b0[2 * kk][cbw], x1 = b0[2 * kk + 1][cbw];
                uint2 h0, l0, h1, l1;
                split4<true>(x0[0], x0[1], x0[2], x0[3], h0, l0);
                split4<true>(x1[0], x1[1], x1[2], x1[3], h1, l1);
                const bf16x8 bh = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                const bf16x8 bl_ = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi) {
                    bf16x8 wh, wl;
                    PS::frag(PhQ, 16 * bi + lr, kk, g, wh, wl);
                    o[bi] = mfma_mix<true, kPhiSplit>(bh, bl_, wh, wl, o[bi]);
                }
            }
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    if (32 * kk > 16 * bi) continue;
                    bf16x8 gh, gl;
                    PG::frag(Gs, 16 * bi + lr, kk, g, gh, gl);
                    if (32 * kk == 16 * bi) {
                        // The upper half of this step is the block above the
                        // diagonal: zero, and never written to the G plane.
#pragma unroll
                        for (int e = 4; e < 8; ++e) {
                            gh[e] = __bf16(0.0f);
                            gl[e] = __bf16(0.0f);
                        }
                    }
                    o[bi] = mfma_mix<false, true>(vh[kk], vh[kk], gh, gl, o[bi]);
                }
                store4<bf16_t, kAlg1StorePolicy>(or_, ((r0 + 16 * bi + lr) * D + 16 * cb + 4 * g) * 2,
                                                o[bi] * rden[bi]);
            }
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    bf16x8 kh, kl;
                    PS::frag_tr(PhK, 32 * kk, 16 * sb, g, lr, kh, kl);
                    b0[sb][cbw] = mfma_mix<kPhiSplit, false>(kh, kl, vh[kk], vh[kk], b0[sb][cbw]);
                }
        }
    }
}

template <bool kPhiSplit, int SP, int D, int LPP>
hipError_t launch_alg1_family(const Alg1Args& a, const Problem& p, hipStream_t stream, Marks* marks) {
    using G = A1Geo<kPhiSplit, SP, D, LPP>;
    if (p.tile % kA1Chunk != 0) return hipErrorInvalidValue;
    if (int64_t(p.tile) * D * 2 >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    alg1_sums_kernel<kPhiSplit, SP, D, LPP><<<grid, kThreads, G::kSumsLds, stream>>>(
        static_cast<const bf16_t*>(a.k), static_cast<const bf16_t*>(a.v), a.W, a.beta, a.records, p.T,
        p.tile, p.tiles, p.rec, a.L, a.P);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    if ((err = launch_tile_scan(a.records, a.state, p, stream)) != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    alg1_output_kernel<kPhiSplit, SP, D, LPP><<<grid, kThreads, G::kOutputLds, stream>>>(
        static_cast<const bf16_t*>(a.q), static_cast<const bf16_t*>(a.k), static_cast<const bf16_t*>(a.v),
        a.W, a.beta, static_cast<bf16_t*>(a.out), a.records, p.T, p.tile, p.tiles, p.rec, a.L, a.P);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return marks ? marks->mark(stream) : hipSuccess;
}

int alg1_sp(int S) { return S <= 32 ? 32 : S <= 64 ? 64 : 128; }
int alg1_lpp(int LP) { return LP <= 16 ? 16 : 32; }

template <bool kPhiSplit, int SP, int D>
hipError_t dispatch_lpp(const Alg1Args& a, const Problem& p, hipStream_t s, Marks* m) {
    if (alg1_lpp(a.L * a.P) == 16) return launch_alg1_family<kPhiSplit, SP, D, 16>(a, p, s, m);
    return launch_alg1_family<kPhiSplit, SP, D, 32>(a, p, s, m);
}

template <bool kPhiSplit, int D>
hipError_t dispatch_sp(const Alg1Args& a, const Problem& p, hipStream_t s, Marks* m) {
    switch (alg1_sp(p.S)) {
        case 32: return dispatch_lpp<kPhiSplit, 32, D>(a, p, s, m);
        case 64: return dispatch_lpp<kPhiSplit, 64, D>(a, p, s, m);
        default: return dispatch_lpp<kPhiSplit, 128, D>(a, p, s, m);
    }
}

template <bool kPhiSplit, int SP, int D, int LPP>
int lds_of() {
    return A1Geo<kPhiSplit, SP, D, LPP>::kOutputLds;
}

}  // namespace

bool alg1_shape_ok(int D, int P, int L) {
    return (D == 64 || D == 128) && P >= 1 && P <= 5 && L >= 1 && L <= 4;
}

size_t alg1_output_lds_bytes(int D, int P, int L, int variant) {
    if (!alg1_shape_ok(D, P, L)) return 0;
    const bool split = variant == 0;
    const int sp = alg1_sp(L << P), lpp = alg1_lpp(L * P);
#define RACE_A1_LDS(SPLIT, SPV, DV, LPPV) \
    if (split == SPLIT && sp == SPV && D == DV && lpp == LPPV) return size_t(lds_of<SPLIT, SPV, DV, LPPV>());
#define RACE_A1_LDS_D(SPLIT, SPV, DV) RACE_A1_LDS(SPLIT, SPV, DV, 16) RACE_A1_LDS(SPLIT, SPV, DV, 32)
#define RACE_A1_LDS_SP(SPLIT, DV) \
    RACE_A1_LDS_D(SPLIT, 32, DV) RACE_A1_LDS_D(SPLIT, 64, DV) RACE_A1_LDS_D(SPLIT, 128, DV)
    RACE_A1_LDS_SP(true, 64)
    RACE_A1_LDS_SP(true, 128)
    RACE_A1_LDS_SP(false, 64)
    RACE_A1_LDS_SP(false, 128)
#undef RACE_A1_LDS_SP
#undef RACE_A1_LDS_D
#undef RACE_A1_LDS
    return 0;
}

int alg1_blocks_per_cu(int D, int P, int L, int variant) {
    return alg1_output_lds_bytes(D, P, L, variant) <= 80 * 1024 ? 2 : 1;
}

hipError_t launch_alg1(const Alg1Args& a, const Problem& p, int variant, hipStream_t stream,
                       Marks* marks) {
    if (!alg1_shape_ok(p.d, a.P, a.L) || p.S != (a.L << a.P)) return hipErrorInvalidValue;
    if (variant == 0) {
        return p.d == 64 ? dispatch_sp<true, 64>(a, p, stream, marks)
                         : dispatch_sp<true, 128>(a, p, stream, marks);
    }
    return p.d == 64 ? dispatch_sp<false, 64>(a, p, stream, marks)
                     : dispatch_sp<false, 128>(a, p, stream, marks);
}

}  // namespace race
