// hashing.hip -- the bucket-probability front end of BatchedACE on gfx950.
//
// src/race_baseline.py:41-44: for every token row x (d_k values) and hash
// table l, with the shared planes planes_T [d_k][L*K] and the 2^K corners
// s_r in {-1, +1}^K (itertools.product([-1, 1], repeat=K): corner r has
// s_{r,k} = +1 iff bit K-1-k of r is set),
//     u_k      = tanh(<x, planes_T[:, l K + k]>) / sqrt(d_k)
//     logit_r  = sum_k u_k s_{r,k}
//     probs[l] = softmax_r(logit)
// One workgroup owns 64 token rows: the rows and the planes are staged in
// LDS (rows padded by one float so the per-table dot products are
// conflict-free), each thread computes one (row, table) pair, and the 64 x
// L x R probabilities are written back through LDS with coalesced stores.
#include <cmath>

#include "race_internal.h"

namespace race {
namespace {

constexpr int kHashRows = 64;

template <typename TIn>
__global__ __launch_bounds__(kThreads) void hash_probs_kernel(const TIn* __restrict__ x,
                                                              const float* __restrict__ planes_T,
                                                              TIn* __restrict__ probs, int64_t rows,
                                                              int dk, int L, int K) {
    extern __shared__ float smem[];
    const int LK = L * K, R = 1 << K, LR = L * R;
    const int xp = dk + 1;  // padded row pitch
    float* xs = smem;                  // [kHashRows][dk + 1]
    float* pl = xs + kHashRows * xp;   // [dk][L*K]
    float* os = pl + dk * LK;          // [kHashRows][L*R]
    const int tid = threadIdx.x;
    const int64_t row0 = int64_t(blockIdx.x) * kHashRows;
    const int cnt = int(min<int64_t>(kHashRows, rows - row0));

    for (int e = tid; e < dk * LK; e += kThreads) pl[e] = planes_T[e];
    for (int e = tid; e < cnt * dk; e += kThreads) {
        const int i = e / dk, c = e - i * dk;
        xs[i * xp + c] = to_f32(x[row0 * dk + e]);
    }
    __syncthreads();
    const float inv_scale = 1.0f / sqrtf(float(dk));
    for (int e = tid; e < cnt * L; e += kThreads) {
        const int i = e / L, l = e - i * L;
        float u[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (k >= K) break;
            float acc = 0.f;
            for (int c = 0; c < dk; ++c) acc = fmaf(xs[i * xp + c], pl[c * LK + l * K + k], acc);
            u[k] = tanhf(acc) * inv_scale;
        }
        // logit_r = sum_k u_k s_{r,k}; softmax over the corners.
        float mx = -INFINITY;
        for (int r = 0; r < R; ++r) {
            float lg = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k >= K) break;
                lg += ((r >> (K - 1 - k)) & 1) ? u[k] : -u[k];
            }
            os[i * LR + l * R + r] = lg;
            mx = fmaxf(mx, lg);
        }
        float sum = 0.f;
        for (int r = 0; r < R; ++r) {
            const float ex = expf(os[i * LR + l * R + r] - mx);
            os[i * LR + l * R + r] = ex;
            sum += ex;
        }
        const float inv = 1.0f / sum;
        for (int r = 0; r < R; ++r) os[i * LR + l * R + r] *= inv;
    }
    __syncthreads();
    for (int e = tid; e < cnt * LR; e += kThreads) store_val(probs + row0 * LR + e, os[e]);
}

}  // namespace

bool hash_shape_ok(int64_t rows, int dk, int L, int K) {
    return rows >= 0 && dk >= 1 && dk <= 128 && L >= 1 && K >= 1 && K <= 8 && L * K <= 64 &&
           L * (1 << K) <= 256;
}

size_t hash_lds_bytes(int dk, int L, int K) {
    return size_t(kHashRows * (dk + 1) + dk * L * K + kHashRows * L * (1 << K)) * sizeof(float);
}

hipError_t launch_hash_probs(const void* x, const float* planes_T, void* probs, int64_t rows,
                            int dk, int L, int K, int dtype, hipStream_t stream) {
    const dim3 grid(unsigned((rows + kHashRows - 1) / kHashRows));
    const size_t lds = hash_lds_bytes(dk, L, K);
    if (dtype == RACE_BF16) {
        hash_probs_kernel<bf16_t><<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(x), planes_T, static_cast<bf16_t*>(probs), rows, dk, L, K);
    } else {
        hash_probs_kernel<float><<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(x), planes_T, static_cast<float*>(probs), rows, dk, L, K);
    }
    return hipGetLastError();
}

}  // namespace race
