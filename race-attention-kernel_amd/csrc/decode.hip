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
// One workgroup per stream holds that stream's whole state in registers:
// NW = ceil(S / RPT) waves (at most 16), wave w owning the RPT bucket rows
// [w RPT, (w+1) RPT) and lane c the value columns c and c + 64.  Each wave
// reads and writes only its own rows of the state, so `state` may be `init`
// (an in-place decode step).  Tokens are staged in groups of kDecodeGroup:
// their q, k rows (zero-padded to 16 RPT buckets) and v rows go to LDS, every
// wave advances its rows through the group keeping a per-token partial sum
// over its buckets, and the NW partials meet in LDS and are added in wave
// order, so the result is bitwise reproducible.  Sixteen waves per stream keep
// enough state loads in flight to stream a stream's 132 KB state (S = 256,
// d = 128) at a useful rate from one compute unit.
// Memory per call: the state is read and written once (8 (S d + S) bytes per
// stream) plus the tokens; the step is bound by that traffic or, for a few
// streams, by the serial token chain (S d fused multiply-adds per token on
// one compute unit).
#include "race_internal.h"

namespace race {
namespace {

constexpr int kDecodeGroup = 8;
constexpr int kDecodeMaxWaves = 16;

template <int RPT, int CPT>
struct DecodeGeo {
    static constexpr int kSP = kDecodeMaxWaves * RPT;  // LDS pitch of the q, k rows (buckets)
    static constexpr int kDP = 64 * CPT;               // LDS pitch of the v rows and partials
    static constexpr int kLdsFloats = kDecodeGroup * (2 * kSP + kDP + kDecodeMaxWaves * kDP);
};

// Rows per wave for S buckets: the fewest (a multiple of 4, for 16-byte LDS
// reads) that cover S with at most kDecodeMaxWaves waves.
inline int decode_rows_per_wave(int S) { return S <= 64 ? 4 : (S <= 128 ? 8 : 16); }

template <typename TIn, int RPT, int CPT>
__global__ __launch_bounds__(64 * kDecodeMaxWaves) void decode_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    TIn* __restrict__ out, const float* init, float* state, int64_t T, int S, int d) {
    using G = DecodeGeo<RPT, CPT>;
    extern __shared__ float lds[];
    float* qs = lds;                                 // [group][kSP]
    float* ks = qs + kDecodeGroup * G::kSP;          // [group][kSP]
    float* vs = ks + kDecodeGroup * G::kSP;          // [group][kDP]
    float* ps = vs + kDecodeGroup * G::kDP;          // [waves][group][kDP]
    const int tid = threadIdx.x, nthreads = blockDim.x;
    const int nw = nthreads >> 6;
    const int w = tid >> 6, lane = tid & 63;
    const int64_t n = blockIdx.x;
    const int64_t used = int64_t(S) * d + S;
    const int s0 = w * RPT;

    // The wave's state rows.  Addresses are clamped into the stream's state so
    // that every load is unconditional (a select on a loaded value compiles
    // to a branch and a wait per load); rows >= S are then cleared with a
    // wave-uniform mask.  Lanes with columns >= d hold a copy of column d - 1
    // that never reaches an output or the stored state.  Lane i < RPT loads
    // A[s0 + i] and the wave shares it.
    float B[RPT][CPT], A[RPT];
    {
        const float* st = init + n * used;
        const int sa = s0 + lane < S ? s0 + lane : S - 1;
        const float a_lane = st[int64_t(S) * d + sa];
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int s = s0 + i < S ? s0 + i : S - 1;
            const unsigned keep = s0 + i < S ? ~0u : 0u;
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const int c = lane + 64 * j < d ? lane + 64 * j : d - 1;
                B[i][j] = __uint_as_float(__float_as_uint(st[int64_t(s) * d + c]) & keep);
            }
        }
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const unsigned a = unsigned(__builtin_amdgcn_readlane(__float_as_int(a_lane), i));
            A[i] = __uint_as_float(a & (s0 + i < S ? ~0u : 0u));
        }
    }

    for (int64_t t0 = 0; t0 < T; t0 += kDecodeGroup) {
        const int g = int(T - t0 < kDecodeGroup ? T - t0 : kDecodeGroup);
        const int64_t row0 = n * T + t0;
        // Stage the group's rows; buckets >= S and columns >= d read as zero,
        // which leaves A, B and the partial sums unchanged.
        for (int idx = tid; idx < kDecodeGroup * G::kSP; idx += nthreads) {
            const int tt = idx / G::kSP, s = idx % G::kSP;
            const bool ok = tt < g && s < S;
            qs[idx] = ok ? to_f32(q[(row0 + tt) * S + s]) : 0.f;
            ks[idx] = ok ? to_f32(k[(row0 + tt) * S + s]) : 0.f;
        }
        for (int idx = tid; idx < kDecodeGroup * G::kDP; idx += nthreads) {
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
        for (int idx = tid; idx < g * G::kDP; idx += nthreads) {
            const int tt = idx / G::kDP, c = idx % G::kDP;
            if (c >= d) continue;
            float o = ps[tt * G::kDP + c];
            for (int ww = 1; ww < nw; ++ww) o += ps[(ww * kDecodeGroup + tt) * G::kDP + c];
            store_val(out + (row0 + tt) * d + c, o);
        }
        // The next group stages into qs, ks, vs after every wave has passed
        // the barrier above (the last reads of this group's rows) and writes
        // its partials after the next barrier (after this group's sums).
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
    }
    // Lane i stores A[s0 + i]: one coalesced store per wave.
    float a_mine = A[0];
#pragma unroll
    for (int i = 1; i < RPT; ++i) a_mine = lane == i ? A[i] : a_mine;
    if (lane < RPT && s0 + lane < S) st[int64_t(S) * d + s0 + lane] = a_mine;
}

template <typename TIn, int RPT, int CPT>
hipError_t launch_decode_t(const void* q, const void* k, const void* v, void* out,
                           const float* init, float* state, const Problem& p, hipStream_t stream) {
    const int waves = (p.S + RPT - 1) / RPT;
    if (waves > kDecodeMaxWaves) return hipErrorInvalidValue;
    const size_t lds = size_t(DecodeGeo<RPT, CPT>::kLdsFloats) * sizeof(float);
    decode_kernel<TIn, RPT, CPT><<<dim3(unsigned(p.N)), dim3(64 * waves), lds, stream>>>(
        static_cast<const TIn*>(q), static_cast<const TIn*>(k), static_cast<const TIn*>(v),
        static_cast<TIn*>(out), init, state, p.T, p.S, p.d);
    return hipGetLastError();
}

template <typename TIn, int CPT>
hipError_t launch_decode_rows(const void* q, const void* k, const void* v, void* out,
                              const float* init, float* state, const Problem& p,
                              hipStream_t stream) {
    switch (decode_rows_per_wave(p.S)) {
        case 4: return launch_decode_t<TIn, 4, CPT>(q, k, v, out, init, state, p, stream);
        case 8: return launch_decode_t<TIn, 8, CPT>(q, k, v, out, init, state, p, stream);
        default: return launch_decode_t<TIn, 16, CPT>(q, k, v, out, init, state, p, stream);
    }
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
