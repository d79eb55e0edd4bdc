// decode.hip -- the causal op continued from a carried state, token by token:
// the decode step of incremental generation.
//
// The reference hands the per-bucket sums over all tokens off as final_state
// (src/causal_v2/kernels/race_causal_fwd.h:20-21, :113-116) and its chunked
// forward carries A_state, B_state into the next chunk
// (src/race_chunked.py:54-63); it has no kernel that consumes the state.  This
// one does, for a few tokens per call (decode, short appends):
//
//     A += k_t,  B += k_t (x) v_t,  out_t = sum_s q_t[s] B[s][:] / (A[s] + eps)
//
// for t = 0 .. T-1 in order, starting from init (B [S][d] then A [S] per
// stream) and leaving the advanced state in `state` (when not null).
//
// One workgroup per stream holds that stream's whole state in registers: wave
// w owns the RPT bucket rows [w RPT, (w+1) RPT), lane c owns the value columns
// c and c + 64.  Each wave reads and writes only its own rows of the state, so
// `state` may be `init` (an in-place decode step).  Tokens are staged in
// groups of kDecodeGroup: their q, k rows (zero-padded to 4 RPT buckets) and v
// rows go to LDS, every wave advances its rows through the group keeping a
// per-token partial sum over its buckets, and the four partials meet in LDS
// and are added in wave order, so the result is bitwise reproducible.
// Memory per call: the state is read and written once (8 (S d + S) bytes per
// stream) plus the tokens; the step is bound by that traffic or, for a few
// streams, by the serial token chain.
#include "race_internal.h"

namespace race {
namespace {

constexpr int kDecodeGroup = 16;

template <int RPT, int CPT>
struct DecodeGeo {
    static constexpr int kSP = 4 * RPT;   // LDS pitch of the q, k rows (buckets, zero-padded)
    static constexpr int kDP = 64 * CPT;  // LDS pitch of the v rows and partials (columns)
    static constexpr int kLdsFloats = kDecodeGroup * (2 * kSP + kDP + 4 * kDP);
};

template <typename TIn, int RPT, int CPT>
__global__ __launch_bounds__(kThreads) void decode_kernel(const TIn* __restrict__ q,
                                                          const TIn* __restrict__ k,
                                                          const TIn* __restrict__ v,
                                                          TIn* __restrict__ out, const float* init,
                                                          float* state, int64_t T, int S, int d) {
    using G = DecodeGeo<RPT, CPT>;
    extern __shared__ float lds[];
    float* qs = lds;                                 // [group][kSP]
    float* ks = qs + kDecodeGroup * G::kSP;          // [group][kSP]
    float* vs = ks + kDecodeGroup * G::kSP;          // [group][kDP]
    float* ps = vs + kDecodeGroup * G::kDP;          // [4][group][kDP]
    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63;
    const int64_t n = blockIdx.x;
    const int64_t used = int64_t(S) * d + S;
    const int s0 = w * RPT;

    float B[RPT][CPT], A[RPT];
    {
        const float* st = init + n * used;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int s = s0 + i;
            A[i] = s < S ? st[int64_t(S) * d + s] : 0.f;
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const int c = lane + 64 * j;
                B[i][j] = (s < S && c < d) ? st[int64_t(s) * d + c] : 0.f;
            }
        }
    }

    for (int64_t t0 = 0; t0 < T; t0 += kDecodeGroup) {
        const int g = int(T - t0 < kDecodeGroup ? T - t0 : kDecodeGroup);
        const int64_t row0 = n * T + t0;
        // Stage the group's rows; buckets >= S and columns >= d read as zero,
        // which leaves A, B and the partial sums unchanged.
        for (int idx = tid; idx < kDecodeGroup * G::kSP; idx += kThreads) {
            const int tt = idx / G::kSP, s = idx % G::kSP;
            const bool ok = tt < g && s < S;
            qs[idx] = ok ? to_f32(q[(row0 + tt) * S + s]) : 0.f;
            ks[idx] = ok ? to_f32(k[(row0 + tt) * S + s]) : 0.f;
        }
        for (int idx = tid; idx < kDecodeGroup * G::kDP; idx += kThreads) {
            const int tt = idx / G::kDP, c = idx % G::kDP;
            vs[idx] = (tt < g && c < d) ? to_f32(v[(row0 + tt) * d + c]) : 0.f;
        }
        __syncthreads();
        for (int tt = 0; tt < g; ++tt) {
            float vv[CPT], part[CPT];
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                vv[j] = vs[tt * G::kDP + lane + 64 * j];
                part[j] = 0.f;
            }
            const float4* k4 = reinterpret_cast<const float4*>(ks + tt * G::kSP + s0);
            const float4* q4 = reinterpret_cast<const float4*>(qs + tt * G::kSP + s0);
#pragma unroll
            for (int i4 = 0; i4 < RPT / 4; ++i4) {
                const float4 kk = k4[i4], qq = q4[i4];
                const float kv[4] = {kk.x, kk.y, kk.z, kk.w};
                const float qv[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * i4 + e;
                    A[i] += kv[e];
                    const float r = qv[e] * __builtin_amdgcn_rcpf(A[i] + kEps);
#pragma unroll
                    for (int j = 0; j < CPT; ++j) {
                        B[i][j] = fmaf(kv[e], vv[j], B[i][j]);
                        part[j] = fmaf(r, B[i][j], part[j]);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < CPT; ++j) ps[(w * kDecodeGroup + tt) * G::kDP + lane + 64 * j] = part[j];
        }
        __syncthreads();
        for (int idx = tid; idx < g * G::kDP; idx += kThreads) {
            const int tt = idx / G::kDP, c = idx % G::kDP;
            if (c >= d) continue;
            float o = ps[(0 * kDecodeGroup + tt) * G::kDP + c];
            o += ps[(1 * kDecodeGroup + tt) * G::kDP + c];
            o += ps[(2 * kDecodeGroup + tt) * G::kDP + c];
            o += ps[(3 * kDecodeGroup + tt) * G::kDP + c];
            store_val(out + (row0 + tt) * d + c, o);
        }
        // The next group's staging overwrites qs, ks, vs only after every
        // wave has passed the barrier above, so the partials' reads above and
        // the next group's partial writes are ordered by the next barrier.
    }

    if (!state) return;
    float* st = state + n * used;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int s = s0 + i;
        if (s >= S) break;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = lane + 64 * j;
            if (c < d) st[int64_t(s) * d + c] = B[i][j];
        }
        if (lane == (i & 63)) st[int64_t(S) * d + s] = A[i];
    }
}

template <typename TIn, int RPT, int CPT>
hipError_t launch_decode_t(const void* q, const void* k, const void* v, void* out,
                           const float* init, float* state, const Problem& p, hipStream_t stream) {
    const size_t lds = size_t(DecodeGeo<RPT, CPT>::kLdsFloats) * sizeof(float);
    decode_kernel<TIn, RPT, CPT><<<dim3(unsigned(p.N)), kThreads, lds, stream>>>(
        static_cast<const TIn*>(q), static_cast<const TIn*>(k), static_cast<const TIn*>(v),
        static_cast<TIn*>(out), init, state, p.T, p.S, p.d);
    return hipGetLastError();
}

template <typename TIn, int CPT>
hipError_t launch_decode_rows(const void* q, const void* k, const void* v, void* out,
                              const float* init, float* state, const Problem& p,
                              hipStream_t stream) {
    if (p.S <= 16) return launch_decode_t<TIn, 4, CPT>(q, k, v, out, init, state, p, stream);
    if (p.S <= 32) return launch_decode_t<TIn, 8, CPT>(q, k, v, out, init, state, p, stream);
    if (p.S <= 64) return launch_decode_t<TIn, 16, CPT>(q, k, v, out, init, state, p, stream);
    if (p.S <= 128) return launch_decode_t<TIn, 32, CPT>(q, k, v, out, init, state, p, stream);
    return launch_decode_t<TIn, 64, CPT>(q, k, v, out, init, state, p, stream);
}

template <typename TIn>
hipError_t launch_decode_typed(const void* q, const void* k, const void* v, void* out,
                               const float* init, float* state, const Problem& p,
                               hipStream_t stream) {
    if (p.d <= 64) return launch_decode_rows<TIn, 1>(q, k, v, out, init, state, p, stream);
    return launch_decode_rows<TIn, 2>(q, k, v, out, init, state, p, stream);
}

}  // namespace

hipError_t launch_decode(const void* q, const void* k, const void* v, void* out,
                         const float* init, float* state, const Problem& p, hipStream_t stream) {
    // Every lane index and row count below assumes these limits.
    if (p.S < 1 || p.S > 256 || p.d < 1 || p.d > 128 || p.N < 1 || p.N > INT32_MAX || p.T < 0)
        return hipErrorInvalidValue;
    if (!init) return hipErrorInvalidValue;
    if (p.dtype == RACE_BF16) return launch_decode_typed<bf16_t>(q, k, v, out, init, state, p, stream);
    return launch_decode_typed<float>(q, k, v, out, init, state, p, stream);
}

}  // namespace race
