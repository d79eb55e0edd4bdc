// hashing.hip -- the bucket-probability front end of BatchedACE on gfx950.
//
// src/race_baseline.py:41-44: for every token row x (d_k values) and hash
// table l, with the shared planes planes_T [d_k][L*K] and the 2^K corners
// s_r in {-1, +1}^K (itertools.product([-1, 1], repeat=K): corner r has
// s_{r,k} = +1 iff bit K-1-k of r is set),
//     u_k      = tanh(<x, planes_T[:, l K + k]>) / sqrt(d_k)
//     logit_r  = sum_k u_k s_{r,k}
//     probs[l] = softmax_r(logit)
// The corner softmax factorises: exp(sum_k s_k u_k) / prod_k (e^u_k + e^-u_k)
// = prod_k sigma(2 s_k u_k), so a table costs K exponentials, not 2^K.
// One workgroup owns 256 token rows, one per thread:
//   1. the rows are staged in LDS 32 columns at a time (coalesced 16-byte
//      loads, the next chunk prefetched into registers), and each thread
//      accumulates its row's L*K projections against LDS broadcasts of the
//      planes;
//   2. the sigmoids sigma(2 u_k) are written to LDS, one row per thread;
//   3. the L x 2^K probabilities of the 256 rows are written out in memory
//      order, four per thread per step (16-byte stores for fp32).
#include <algorithm>
#include <cmath>

#include "race_internal.h"

namespace race {
namespace {

constexpr int kHashRows = kThreads;
constexpr int kChunk = 32;              // x columns staged per step
constexpr int kXPitch = kChunk + 4;     // odd count of 16-byte words: b128 reads conflict-free
constexpr int kGroups = kChunk / 4;     // 4-column groups per staged row

template <typename TIn>
struct Quad;
template <>
struct Quad<float> {
    float4 v;
    __device__ void load(const float* p) { v = *reinterpret_cast<const float4*>(p); }
    __device__ float4 f32() const { return v; }
};
template <>
struct Quad<bf16_t> {
    uint2 v;
    __device__ void load(const bf16_t* p) { v = *reinterpret_cast<const uint2*>(p); }
    __device__ float4 f32() const {
        return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                           __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
    }
};

__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void store4(bf16_t* p, float a, float b, float c, float d) {
    *reinterpret_cast<uint2*>(p) = make_uint2(uint32_t(f32_to_bf16(a)) | (uint32_t(f32_to_bf16(b)) << 16),
                                              uint32_t(f32_to_bf16(c)) | (uint32_t(f32_to_bf16(d)) << 16));
}

// The 4-column groups of one staged chunk owned by this thread: group
// g = tid + 256 i is row g / 8, columns c0 + 4 (g % 8) .. + 3.  Vec: d_k is a
// multiple of 4, so a group is one aligned vector load.  The loads are
// unconditional (rows past the tile and columns past d_k read a valid
// element) and keep the raw input; the conversion, with those positions
// zeroed, happens when the chunk is staged.  (Converting or zeroing right
// after each load made the compiler wait for every bf16 load in turn.)
template <typename TIn, bool Vec>
struct RawChunk {
    Quad<TIn> q[kGroups];
    TIn e[Vec ? 1 : kGroups][4];

    __device__ __forceinline__ void load(const TIn* __restrict__ x, int64_t row0, int cnt, int dk,
                                         int c0, int tid) {
#pragma unroll
        for (int i = 0; i < kGroups; ++i) {
            const int g = tid + kThreads * i;
            const int row = min(g / kGroups, cnt - 1), col = c0 + 4 * (g % kGroups);
            if constexpr (Vec) {
                q[i].load(x + (row0 + row) * dk + (col < dk ? col : 0));
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) e[i][t] = x[(row0 + row) * dk + (col + t < dk ? col + t : 0)];
            }
        }
    }
    // Group i as floats, zero past the tile's rows and past d_k.
    __device__ __forceinline__ float4 get(int i, int cnt, int dk, int c0, int tid) const {
        const int g = tid + kThreads * i, row = g / kGroups, col = c0 + 4 * (g % kGroups);
        if constexpr (Vec) {
            return row < cnt && col < dk ? q[i].f32() : make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            float v[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = row < cnt && col + t < dk ? to_f32(e[i][t]) : 0.f;
            return make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

template <typename TIn, int LKT, bool Vec>
__global__ __launch_bounds__(kThreads) void hash_probs_kernel(const TIn* __restrict__ x,
                                                              const float* __restrict__ planes_T,
                                                              TIn* __restrict__ probs, int64_t rows,
                                                              int dk, int L, int K) {
    extern __shared__ float smem[];
    const int LK = L * K, R = 1 << K, LR = L * R, dk4 = (dk + 3) & ~3;
    float* pl = smem;                  // [dk4][LKT], zero past d_k rows and L*K columns
    float* xs = pl + dk4 * LKT;        // [256][kXPitch] staged x, then [256][LK + 1] sigmoids
    const int tid = threadIdx.x;
    const int64_t row0 = int64_t(blockIdx.x) * kHashRows;
    const int cnt = int(min<int64_t>(kHashRows, rows - row0));

    // Planes staged with their loads in groups of 8 (clamped addresses, the
    // padding zeroed at the store), not one memory round trip per element.
    for (int e0 = 0; e0 < dk4 * LKT; e0 += 8 * kThreads) {
        float v[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int e = e0 + tid + m * kThreads;
            const int c = min(e / LKT, dk - 1), j = min(e % LKT, LK - 1);
            v[m] = planes_T[c * LK + j];
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int e = e0 + tid + m * kThreads;
            const int c = e / LKT, j = e % LKT;
            if (e < dk4 * LKT) pl[e] = (j < LK && c < dk) ? v[m] : 0.f;
        }
    }

    float acc[LKT];
#pragma unroll
    for (int j = 0; j < LKT; ++j) acc[j] = 0.f;
    RawChunk<TIn, Vec> xr;
    xr.load(x, row0, cnt, dk, 0, tid);
    for (int c0 = 0; c0 < dk; c0 += kChunk) {
        __syncthreads();  // the previous chunk has been read
#pragma unroll
        for (int i = 0; i < kGroups; ++i) {
            const int g = tid + kThreads * i;
            *reinterpret_cast<float4*>(xs + (g / kGroups) * kXPitch + 4 * (g % kGroups)) =
                xr.get(i, cnt, dk, c0, tid);
        }
        __syncthreads();
        if (c0 + kChunk < dk) xr.load(x, row0, cnt, dk, c0 + kChunk, tid);
        const int width = min(kChunk, dk4 - c0);
        const float* xrow = xs + tid * kXPitch;
        for (int cc = 0; cc < width; cc += 4) {
            const float4 xv = *reinterpret_cast<const float4*>(xrow + cc);
            const float xc[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float* prow = pl + (c0 + cc + u) * LKT;
#pragma unroll
                for (int j = 0; j < LKT; j += 4) {
                    const float4 pv = *reinterpret_cast<const float4*>(prow + j);
                    acc[j] = fmaf(xc[u], pv.x, acc[j]);
                    acc[j + 1] = fmaf(xc[u], pv.y, acc[j + 1]);
                    acc[j + 2] = fmaf(xc[u], pv.z, acc[j + 2]);
                    acc[j + 3] = fmaf(xc[u], pv.w, acc[j + 3]);
                }
            }
        }
    }

    // sigma(2 u) with u = tanh(projection) / sqrt(d_k); |u| <= 1, no overflow.
    const float two_over_scale = 2.0f / sqrtf(float(dk));
    __syncthreads();  // the staged x is dead: its space takes the sigmoids
    float* sg = xs + tid * (LK + 1);
#pragma unroll
    for (int j = 0; j < LKT; ++j)
        if (j < LK) sg[j] = 1.0f / (1.0f + expf(-two_over_scale * tanhf(acc[j])));
    __syncthreads();

    // probs[row][l][r] = prod_k (bit K-1-k of r ? sigma_k : 1 - sigma_k).
    if (K >= 2) {  // L * R is a multiple of 4: four corners of one table per step
        const int quads = LR / 4, total = cnt * quads;
        for (int g = tid; g < total; g += kThreads) {
            const int row = g / quads, c = 4 * (g - row * quads);
            const int l = c >> K, r0 = c & (R - 1);
            const float* s = xs + row * (LK + 1) + l * K;
            float p[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k < K) {
                    const float sk = s[k], sn = 1.0f - sk;
#pragma unroll
                    for (int t = 0; t < 4; ++t) p[t] *= (((r0 + t) >> (K - 1 - k)) & 1) ? sk : sn;
                }
            }
            store4(probs + (row0 + row) * LR + c, p[0], p[1], p[2], p[3]);
        }
    } else {  // K = 1: two corners per table
        const int total = cnt * LR;
        for (int e = tid; e < total; e += kThreads) {
            const int row = e / LR, c = e - row * LR;
            const float sk = xs[row * (LK + 1) + (c >> 1)];
            store_val(probs + (row0 + row) * LR + c, (c & 1) ? sk : 1.0f - sk);
        }
    }
}

// Gradient of the hashing w.r.t. the rows, one row per thread.  The
// projections and sigmoids are recomputed as the forward computes them; then
// per table, with g_r = dprobs_r probs_r and sigma_k = sigma(2 u_k),
//     du_k = 2 (sum_{r: bit K-1-k of r set} g_r - sigma_k sum_r g_r)
// (d probs_r / d u_k = 2 probs_r ([s_{r,k} = +1] - sigma_k)), and
//     dx = sum_k du_k (1 - tanh^2(p_k)) / sqrt(d_k) planes_T[:, k].
template <typename TIn, int LKT>
__global__ __launch_bounds__(kThreads) void hash_probs_bwd_kernel(
    const TIn* __restrict__ x, const float* __restrict__ planes_T, const TIn* __restrict__ dprobs,
    TIn* __restrict__ dx, int64_t rows, int dk, int L, int K) {
    extern __shared__ float pl[];  // [dk][LKT], zero past L*K columns
    const int LK = L * K, R = 1 << K, LR = L * R;
    for (int e = threadIdx.x; e < dk * LKT; e += kThreads) {
        const int c = e / LKT, j = e % LKT;
        pl[e] = j < LK ? planes_T[c * LK + j] : 0.f;
    }
    __syncthreads();
    const int64_t row = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (row >= rows) return;
    const TIn* xr = x + row * dk;
    float acc[LKT];
#pragma unroll
    for (int j = 0; j < LKT; ++j) acc[j] = 0.f;
    for (int c = 0; c < dk; ++c) {
        const float xc = to_f32(xr[c]);
#pragma unroll
        for (int j = 0; j < LKT; ++j) acc[j] = fmaf(xc, pl[c * LKT + j], acc[j]);
    }
    const float inv_scale = 1.0f / sqrtf(float(dk));
    float th[LKT], sg[LKT];
#pragma unroll
    for (int j = 0; j < LKT; ++j) {
        th[j] = tanhf(acc[j]);
        sg[j] = 1.0f / (1.0f + expf(-2.0f * inv_scale * th[j]));
    }
    const TIn* gr = dprobs + row * LR;
    float dpj[LKT];
#pragma unroll
    for (int j = 0; j < LKT; ++j) dpj[j] = 0.f;
    for (int l = 0; l < L; ++l) {
        float tot = 0.f, pos[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int r = 0; r < R; ++r) {
            // prod_k (bit K-1-k of r ? sigma_k : 1 - sigma_k) for table l.
            float prob = 1.f;
#pragma unroll
            for (int j = 0; j < LKT; ++j) {
                const int k = j - l * K;
                if (k >= 0 && k < K) prob *= ((r >> (K - 1 - k)) & 1) ? sg[j] : 1.0f - sg[j];
            }
            const float gv = to_f32(gr[l * R + r]) * prob;
            tot += gv;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (k < K && ((r >> (K - 1 - k)) & 1)) pos[k] += gv;
        }
#pragma unroll
        for (int j = 0; j < LKT; ++j) {
            const int k = j - l * K;
            if (k >= 0 && k < K) {
                float pk = 0.f;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk)
                    if (kk == k) pk = pos[kk];
                const float du = 2.0f * (pk - sg[j] * tot);
                dpj[j] = du * (1.0f - th[j] * th[j]) * inv_scale;
            }
        }
    }
    TIn* dxr = dx + row * dk;
    for (int c = 0; c < dk; ++c) {
        float v = 0.f;
#pragma unroll
        for (int j = 0; j < LKT; ++j) v = fmaf(dpj[j], pl[c * LKT + j], v);
        store_val(dxr + c, v);
    }
}

int lk_tier(int LK) { return LK <= 16 ? 16 : LK <= 32 ? 32 : 64; }

}  // namespace

bool hash_shape_ok(int64_t rows, int dk, int L, int K) {
    return rows >= 0 && dk >= 1 && dk <= 128 && L >= 1 && K >= 1 && K <= 8 && L * K <= 64 &&
           L * (1 << K) <= 256;
}

size_t hash_lds_bytes(int dk, int L, int K) {
    const int dk4 = (dk + 3) & ~3;
    return size_t(dk4 * lk_tier(L * K) + kHashRows * std::max(kXPitch, L * K + 1)) * sizeof(float);
}

hipError_t launch_hash_probs(const void* x, const float* planes_T, void* probs, int64_t rows,
                            int dk, int L, int K, int dtype, hipStream_t stream) {
    const dim3 grid(unsigned((rows + kHashRows - 1) / kHashRows));
    const size_t lds = hash_lds_bytes(dk, L, K);
    const bool vec = dk % 4 == 0;
#define RACE_HASH(TIN, LKT, VEC)                                                             \
    hash_probs_kernel<TIN, LKT, VEC><<<grid, kThreads, lds, stream>>>(                       \
        static_cast<const TIN*>(x), planes_T, static_cast<TIN*>(probs), rows, dk, L, K)
#define RACE_HASH_LK(TIN, VEC)                         \
    switch (lk_tier(L * K)) {                          \
        case 16: RACE_HASH(TIN, 16, VEC); break;       \
        case 32: RACE_HASH(TIN, 32, VEC); break;       \
        default: RACE_HASH(TIN, 64, VEC); break;       \
    }
    if (dtype == RACE_BF16) {
        if (vec) {
            RACE_HASH_LK(bf16_t, true)
        } else {
            RACE_HASH_LK(bf16_t, false)
        }
    } else {
        if (vec) {
            RACE_HASH_LK(float, true)
        } else {
            RACE_HASH_LK(float, false)
        }
    }
#undef RACE_HASH_LK
#undef RACE_HASH
    return hipGetLastError();
}

hipError_t launch_hash_probs_bwd(const void* x, const float* planes_T, const void* dprobs, void* dx,
                                int64_t rows, int dk, int L, int K, int dtype, hipStream_t stream) {
    const dim3 grid(unsigned((rows + kThreads - 1) / kThreads));
    const int tier = lk_tier(L * K);
    const size_t lds = size_t(dk) * tier * sizeof(float);
#define RACE_HASH_BWD(TIN, LKT)                                                               \
    hash_probs_bwd_kernel<TIN, LKT><<<grid, kThreads, lds, stream>>>(                         \
        static_cast<const TIN*>(x), planes_T, static_cast<const TIN*>(dprobs), static_cast<TIN*>(dx), \
        rows, dk, L, K)
    if (dtype == RACE_BF16) {
        if (tier == 16) RACE_HASH_BWD(bf16_t, 16);
        else if (tier == 32) RACE_HASH_BWD(bf16_t, 32);
        else RACE_HASH_BWD(bf16_t, 64);
    } else {
        if (tier == 16) RACE_HASH_BWD(float, 16);
        else if (tier == 32) RACE_HASH_BWD(float, 32);
        else RACE_HASH_BWD(float, 64);
    }
#undef RACE_HASH_BWD
    return hipGetLastError();
}

}  // namespace race
