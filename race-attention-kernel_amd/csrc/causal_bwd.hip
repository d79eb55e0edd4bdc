// causal_bwd.hip -- backward of the causal per-bucket function, fp32 vector-
// ALU kernels for every shape whose per-bucket state fits one workgroup's LDS.
//
// The reference has no kernel for this; its design outline for the other
// (globally normalized) function is docs/causal_v2_design.md:689-742: prefix
// states walked forward, suffix states walked backward, a [V | 1] column for
// the denominator.  For the per-bucket function of src/race_baseline.py:45-51
// (per stream; A_i, B_i inclusive prefix sums of k and k (x) v;
// r_i = 1 / (A_i + eps); W_i = q_i r_i elementwise over buckets; g = dOut):
//     dq_i[s]    = r_i[s] <B_i[s][:], g_i>
//     alpha_i[s] = -W_i[s] dq_i[s]                          (dLoss / dA_i)
//     Z_j = sum_{i>=j} W_i (x) g_i,   Y_j = sum_{i>=j} alpha_i   (suffix sums)
//     dk_j[s] = <Z_j[s][:], v_j> + Y_j[s],   dv_j[c] = sum_s k_j[s] Z_j[s][c].
// In a sub-chunk of C tokens with prefix state (A0, B0) before it and suffix
// state (Z1, Y1) after it (i, j local):
//     Abar = A0 + tril(1) K,  r = 1 / (Abar + eps),  W = Q r,
//     M = tril(G V^T),  P = tril(W K^T)                (diagonal included)
//     dQ = r (G B0^T + M K),  alpha = -W dQ
//     dK = V Z1^T + 1 Y1^T + M^T W + triu(1) alpha   (reverse running sum)
//     dV = K Z1 + P^T G
//     Z1 += W^T G, Y1 += 1^T alpha;  B0 += K^T V, A0 += 1^T K.
//
// Launch sequence (race_api.hip):
//   1. forward tile totals and their exclusive scan (the forward's K1, K2):
//      the prefix state at every tile start
//   2. causal_bwd_dq_kernel: per tile, walk the sub-chunks forward: dQ, an
//      fp32 copy of dQ and the running mass at every sub-chunk start into the
//      workspace, and the tile's suffix totals (Z, Y) into a record
//   3. tile_scan_kernel in reverse tile order: suffix state at every tile end
//   4. causal_bwd_dkv_kernel: per tile, walk the sub-chunks backward: dK, dV
// Every sum has a fixed order, so the gradients are bitwise reproducible for
// a given tile length.
//
// Column groups.  Every term above is linear in the value columns: a group
// of columns c0 .. c0 + dg - 1 of V and g (the forward prefix B0 restricted to
// them, its own Z) yields dV of its columns exactly, and a partial dQ (hence a
// partial alpha and Y) and a partial dK whose sum over the groups is the
// whole.  Where the state of all d columns does not fit one workgroup's LDS,
// race_api.hip runs the walks once per group, in group order, adding each
// group's dQ and dK to an fp32 running sum (BwdCols); dq32 then holds the
// current group's partial dQ, which is what its backward walk needs.
#include "race_internal.h"

namespace race {
namespace {

template <typename TIn>
__device__ __forceinline__ float ldf(const TIn* __restrict__ p, int64_t i) {
    return to_f32(p[i]);
}

// Buckets per stream the walks take (the library's limit): the forward walk
// keeps Y in kBwdMaxS / kThreads registers per thread.
constexpr int kBwdMaxS = 256;
static_assert(kBwdMaxS % kThreads == 0, "whole register rows of Y");

int64_t dq_lds_floats(int S, int d, int C) {
    return int64_t(S) * d + S + 3 * int64_t(C) * S + 2 * int64_t(C) * d + int64_t(C) * C;
}
int64_t dkv_lds_floats(int S, int d, int C) {
    return int64_t(S) * d + S + 3 * int64_t(C) * S + 2 * int64_t(C) * d + 2 * int64_t(C) * C;
}

// ---------------------------------------------------------------------------
// Forward walk of one (tile, stream).  Thread e of the workgroup owns the
// suffix-total elements Z[e + kThreads m] (registers) and, for e < S, Y[e].
template <typename TIn, int MZ>
__global__ __launch_bounds__(kThreads) void causal_bwd_dq_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    const TIn* __restrict__ g, TIn* __restrict__ dQ, float* __restrict__ dq32,
    float* __restrict__ apre, const float* __restrict__ fwd_records,
    float* __restrict__ bwd_records, int64_t T, int S, int d, int C, int tile, int64_t tiles,
    int64_t rec, BwdCols cols) {
    extern __shared__ float smem[];
    const int Sd = S * d;
    float* B0 = smem;          // [S][d]
    float* A0 = B0 + Sd;       // [S]
    float* Wq = A0 + S;        // [C][S]: q, then W = q r
    float* Rs = Wq + C * S;    // [C][S]: r, then alpha
    float* Ks = Rs + C * S;    // [C][S]
    float* Vs = Ks + C * S;    // [C][d]
    float* Gs = Vs + C * d;    // [C][d]
    float* M = Gs + C * d;     // [C][C]: tril(G V^T)
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y, ti = blockIdx.x;

    // B0: the group's columns of the forward prefix record (rows of
    // cols.fwd_d values), then A0.
    const float* fr = fwd_records + (n * tiles + ti) * cols.fwd_rec;
    for (int e = tid; e < Sd; e += kThreads) {
        const int s = e / d, c = e - s * d;
        B0[e] = fr[int64_t(s) * cols.fwd_d + cols.c0 + c];
    }
    for (int s = tid; s < S; s += kThreads) A0[s] = fr[int64_t(S) * cols.fwd_d + s];
    float z[MZ];
#pragma unroll
    for (int m = 0; m < MZ; ++m) z[m] = 0.f;
    float y[kBwdMaxS / kThreads];  // Y[tid + kThreads m]
#pragma unroll
    for (int m = 0; m < kBwdMaxS / kThreads; ++m) y[m] = 0.f;

    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    float* ap = apre + (n * tiles + ti) * int64_t(tile / C) * S;
    for (int64_t t0 = t_begin; t0 < t_end; t0 += C) {
        const int cnt = int(min<int64_t>(C, t_end - t0));
        const int sub = int((t0 - t_begin) / C);
        const int64_t rs = (n * T + t0) * S, rd = (n * T + t0) * cols.ld;
        __syncthreads();
        for (int e = tid; e < cnt * S; e += kThreads) {
            Wq[e] = ldf(q, rs + e);
            Ks[e] = ldf(k, rs + e);
        }
        for (int e = tid; e < cnt * d; e += kThreads) {
            const int i = e / d, c = e - i * d;
            Vs[e] = ldf(v, rd + int64_t(i) * cols.ld + c);
            Gs[e] = ldf(g, rd + int64_t(i) * cols.ld + c);
        }
        __syncthreads();
        // Running mass (saved per sub-chunk for the backward walk), r and W.
        for (int s = tid; s < S; s += kThreads) {
            float run = A0[s];
            ap[sub * S + s] = run;
            for (int i = 0; i < cnt; ++i) {
                run += Ks[i * S + s];
                const float r = 1.f / (run + kEps);
                Rs[i * S + s] = r;
                Wq[i * S + s] *= r;
            }
            A0[s] = run;
        }
        for (int e = tid; e < cnt * cnt; e += kThreads) {
            const int i = e / cnt, j = e - i * cnt;
            float acc = 0.f;
            if (j <= i)
                for (int c = 0; c < d; ++c) acc = fmaf(Gs[i * d + c], Vs[j * d + c], acc);
            M[i * C + j] = acc;
        }
        __syncthreads();
        // dQ = r (G B0^T + M K); alpha = -W dQ over r in place.
        for (int e = tid; e < cnt * S; e += kThreads) {
            const int i = e / S, s = e - i * S;
            float u = 0.f;
            for (int c = 0; c < d; ++c) u = fmaf(Gs[i * d + c], B0[s * d + c], u);
            for (int j = 0; j <= i; ++j) u = fmaf(M[i * C + j], Ks[j * S + s], u);
            const float dqv = Rs[e] * u;
            dq32[rs + e] = dqv;
            float tot = dqv;  // dQ over the groups so far
            if (cols.acc_q_in) tot = cols.acc_q_in[rs + e] + dqv;
            if (cols.acc_q_out) cols.acc_q_out[rs + e] = tot;
            if (dQ) store_val(dQ + rs + e, tot);
            Rs[e] = -Wq[e] * dqv;
        }
        __syncthreads();
        // Z += W^T G and B0 += K^T V (thread-owned elements), Y += 1^T alpha.
#pragma unroll
        for (int m = 0; m < MZ; ++m) {
            const int e = tid + m * kThreads;
            if (e < Sd) {
                const int s = e / d, c = e - s * d;
                float za = z[m], ba = 0.f;
                for (int i = 0; i < cnt; ++i) {
                    za = fmaf(Wq[i * S + s], Gs[i * d + c], za);
                    ba = fmaf(Ks[i * S + s], Vs[i * d + c], ba);
                }
                z[m] = za;
                B0[e] += ba;
            }
        }
#pragma unroll
        for (int m = 0; m < kBwdMaxS / kThreads; ++m) {
            const int sy = tid + m * kThreads;
            if (sy < S)
                for (int i = 0; i < cnt; ++i) y[m] += Rs[i * S + sy];
        }
    }
    float* br = bwd_records + (n * tiles + ti) * rec;
#pragma unroll
    for (int m = 0; m < MZ; ++m) {
        const int e = tid + m * kThreads;
        if (e < Sd) br[e] = z[m];
    }
#pragma unroll
    for (int m = 0; m < kBwdMaxS / kThreads; ++m)
        if (tid + m * kThreads < S) br[Sd + tid + m * kThreads] = y[m];
}

// ---------------------------------------------------------------------------
// Backward walk of one (tile, stream) from the suffix state at the tile end.
template <typename TIn>
__global__ __launch_bounds__(kThreads) void causal_bwd_dkv_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    const TIn* __restrict__ g, const float* __restrict__ dq32, const float* __restrict__ apre,
    const float* __restrict__ suffix_records, TIn* __restrict__ dK, TIn* __restrict__ dV, int64_t T,
    int S, int d, int C, int tile, int64_t tiles, int64_t rec, BwdCols cols) {
    extern __shared__ float smem[];
    const int Sd = S * d;
    float* Z1 = smem;          // [S][d]
    float* Y1 = Z1 + Sd;       // [S]
    float* Ws = Y1 + S;        // [C][S]: q, then W
    float* Ks = Ws + C * S;    // [C][S]
    float* Al = Ks + C * S;    // [C][S]: dQ, then alpha, then its reverse running sum
    float* Vs = Al + C * S;    // [C][d]
    float* Gs = Vs + C * d;    // [C][d]
    float* M = Gs + C * d;     // [C][C]: tril(G V^T)
    float* P = M + C * C;      // [C][C]: tril(W K^T)
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y, ti = blockIdx.x;

    const float* sr = suffix_records + (n * tiles + ti) * rec;
    for (int e = tid; e < Sd + S; e += kThreads) Z1[e] = sr[e];  // Z1, then Y1

    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const int nsub = int((t_end - t_begin + C - 1) / C);
    const float* ap = apre + (n * tiles + ti) * int64_t(tile / C) * S;
    for (int sub = nsub - 1; sub >= 0; --sub) {
        const int64_t t0 = t_begin + int64_t(sub) * C;
        const int cnt = int(min<int64_t>(C, t_end - t0));
        const int64_t rs = (n * T + t0) * S, rd = (n * T + t0) * cols.ld;
        __syncthreads();
        for (int e = tid; e < cnt * S; e += kThreads) {
            Ws[e] = ldf(q, rs + e);
            Ks[e] = ldf(k, rs + e);
            Al[e] = dq32[rs + e];
        }
        for (int e = tid; e < cnt * d; e += kThreads) {
            const int i = e / d, c = e - i * d;
            Vs[e] = ldf(v, rd + int64_t(i) * cols.ld + c);
            Gs[e] = ldf(g, rd + int64_t(i) * cols.ld + c);
        }
        __syncthreads();
        // W exactly as the forward walk computed it, and alpha = -W dQ.
        for (int s = tid; s < S; s += kThreads) {
            float run = ap[sub * S + s];
            for (int i = 0; i < cnt; ++i) {
                run += Ks[i * S + s];
                const float r = 1.f / (run + kEps);
                const float w = Ws[i * S + s] * r;
                Ws[i * S + s] = w;
                Al[i * S + s] = -w * Al[i * S + s];
            }
        }
        for (int e = tid; e < cnt * cnt; e += kThreads) {
            const int i = e / cnt, j = e - i * cnt;
            float acc = 0.f;
            if (j <= i)
                for (int c = 0; c < d; ++c) acc = fmaf(Gs[i * d + c], Vs[j * d + c], acc);
            M[i * C + j] = acc;
        }
        __syncthreads();
        for (int e = tid; e < cnt * cnt; e += kThreads) {
            const int i = e / cnt, j = e - i * cnt;
            float acc = 0.f;
            if (j <= i)
                for (int s = 0; s < S; ++s) acc = fmaf(Ws[i * S + s], Ks[j * S + s], acc);
            P[i * C + j] = acc;
        }
        // Reverse running sum of alpha over the sub-chunk's tokens.
        for (int s = tid; s < S; s += kThreads) {
            float acc = 0.f;
            for (int i = cnt - 1; i >= 0; --i) {
                acc += Al[i * S + s];
                Al[i * S + s] = acc;
            }
        }
        __syncthreads();
        // dK = V Z1^T + Y1 + M^T W + reverse running alpha.
        const bool want_dk = dK || cols.acc_k_out;
        for (int e = tid; want_dk && e < cnt * S; e += kThreads) {
            const int j = e / S, s = e - j * S;
            float acc = 0.f;
            for (int c = 0; c < d; ++c) acc = fmaf(Vs[j * d + c], Z1[s * d + c], acc);
            for (int i = j; i < cnt; ++i) acc = fmaf(M[i * C + j], Ws[i * S + s], acc);
            float tot = acc + (Y1[s] + Al[e]);  // dK over the groups so far
            if (cols.acc_k_in) tot = cols.acc_k_in[rs + e] + tot;
            if (cols.acc_k_out) cols.acc_k_out[rs + e] = tot;
            if (dK) store_val(dK + rs + e, tot);
        }
        // dV = K Z1 + P^T G.
        for (int e = tid; dV && e < cnt * d; e += kThreads) {
            const int j = e / d, c = e - j * d;
            float acc = 0.f;
            for (int s = 0; s < S; ++s) acc = fmaf(Ks[j * S + s], Z1[s * d + c], acc);
            for (int i = j; i < cnt; ++i) acc = fmaf(P[i * C + j], Gs[i * d + c], acc);
            store_val(dV + rd + int64_t(j) * cols.ld + c, acc);
        }
        __syncthreads();
        // Suffix state before this sub-chunk.
        for (int e = tid; e < Sd; e += kThreads) {
            const int s = e / d, c = e - s * d;
            float acc = 0.f;
            for (int i = 0; i < cnt; ++i) acc = fmaf(Ws[i * S + s], Gs[i * d + c], acc);
            Z1[e] += acc;
        }
        for (int s = tid; s < S; s += kThreads) Y1[s] += Al[s];
    }
}

int z_regs(int S, int d) {
    const int need = (S * d + kThreads - 1) / kThreads;
    int m = 1;
    while (m < need) m *= 2;
    return m;
}

}  // namespace

int causal_bwd_chunk(int S, int d, int lds_limit_bytes) {
    if (S > kBwdMaxS) return 0;
    for (int C : {32, 16}) {
        const int64_t need =
            (dq_lds_floats(S, d, C) > dkv_lds_floats(S, d, C) ? dq_lds_floats(S, d, C)
                                                              : dkv_lds_floats(S, d, C)) *
            int64_t(sizeof(float));
        if (need <= lds_limit_bytes && z_regs(S, d) <= 128) return C;
    }
    return 0;
}

hipError_t launch_causal_bwd_dq(const void* q, const void* k, const void* v, const void* g,
                                void* dQ, float* dq32, float* apre, const float* fwd_records,
                                float* bwd_records, const Problem& p, int C, const BwdCols& cols,
                                hipStream_t stream) {
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    const size_t lds = size_t(dq_lds_floats(p.S, p.d, C)) * sizeof(float);
#define RACE_DQ(TIN, MZ)                                                                          \
    causal_bwd_dq_kernel<TIN, MZ><<<grid, kThreads, lds, stream>>>(                               \
        static_cast<const TIN*>(q), static_cast<const TIN*>(k), static_cast<const TIN*>(v),       \
        static_cast<const TIN*>(g), static_cast<TIN*>(dQ), dq32, apre, fwd_records, bwd_records, \
        p.T, p.S, p.d, C, p.tile, p.tiles, p.rec, cols)
#define RACE_DQ_MZ(TIN)                         \
    switch (z_regs(p.S, p.d)) {                 \
        case 1: RACE_DQ(TIN, 1); break;         \
        case 2: RACE_DQ(TIN, 2); break;         \
        case 4: RACE_DQ(TIN, 4); break;         \
        case 8: RACE_DQ(TIN, 8); break;         \
        case 16: RACE_DQ(TIN, 16); break;       \
        case 32: RACE_DQ(TIN, 32); break;       \
        case 64: RACE_DQ(TIN, 64); break;       \
        case 128: RACE_DQ(TIN, 128); break;     \
        default: return hipErrorInvalidValue;   \
    }
    if (p.dtype == RACE_BF16) {
        RACE_DQ_MZ(bf16_t)
    } else {
        RACE_DQ_MZ(float)
    }
#undef RACE_DQ_MZ
#undef RACE_DQ
    return hipGetLastError();
}

hipError_t launch_causal_bwd_dkv(const void* q, const void* k, const void* v, const void* g,
                                 const float* dq32, const float* apre,
                                 const float* suffix_records, void* dK, void* dV, const Problem& p,
                                 int C, const BwdCols& cols, hipStream_t stream) {
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    const size_t lds = size_t(dkv_lds_floats(p.S, p.d, C)) * sizeof(float);
    if (p.dtype == RACE_BF16) {
        causal_bwd_dkv_kernel<bf16_t><<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
            static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), dq32, apre,
            suffix_records, static_cast<bf16_t*>(dK), static_cast<bf16_t*>(dV), p.T, p.S, p.d, C,
            p.tile, p.tiles, p.rec, cols);
    } else {
        causal_bwd_dkv_kernel<float><<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(q), static_cast<const float*>(k),
            static_cast<const float*>(v), static_cast<const float*>(g), dq32, apre,
            suffix_records, static_cast<float*>(dK), static_cast<float*>(dV), p.T, p.S, p.d, C,
            p.tile, p.tiles, p.rec, cols);
    }
    return hipGetLastError();
}

}  // namespace race
