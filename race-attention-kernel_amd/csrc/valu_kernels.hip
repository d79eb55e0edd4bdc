// valu_kernels.hip -- fp32 vector-ALU kernels of the RACE attention op, for
// every supported shape (1 <= S <= 256, 1 <= d <= 128).
//
// These are the reference-shaped kernels: the causal forward is the
// three-launch decomposition of the reference's v2a
// (src/causal_v2/kernels/race_causal_fwd.h:23-27) -- per-tile totals, an
// exclusive scan over tiles, an output pass walking sub-chunks -- computing
// the per-bucket function of src/race_baseline.py:45-51 from the chunk
// identity (docs/causal_v2_design.md:70-77):
//     Abar_i = A0 + sum_{j<=i} k_j,  W_i = q_i / (Abar_i + eps),
//     O_i    = W_i . B0 + sum_{j<=i} (W_i . k_j) v_j.
// The non-causal forward and backward are bucket reductions over T
// (tile partials, fixed-order reduce) followed by token-parallel maps.
//
// Work split: V/out columns are cut into slices of 64 (grid.z) so the state
// slice B0 [S][64] fits in LDS for S = 256.  No atomics; every sum has a fixed
// order, so results are bitwise reproducible for a given tile length.
#include "race_internal.h"

namespace race {
namespace {

constexpr int kStageTokens = 32;  // tokens staged per step in the reduction kernels
constexpr int kValuChunk = 32;    // sub-chunk of the causal output pass
constexpr int kMapTokens = 32;    // tokens per workgroup of the map kernel

template <typename TIn>
__device__ __forceinline__ float ld(const TIn* __restrict__ p, int64_t i) {
    return to_f32(p[i]);
}

// ---------------------------------------------------------------------------
// Per (tile, stream, column slice): rec[a*Wb + c] = sum_t x[t][a] * y[t][c],
// rec[Wa*Wb + a] = sum_t x[t][a] (slice 0 only).  Thread (tr, tc) =
// (tid / 16, tid % 16) owns rows a = tr + 16 i, i < MI, and slice columns
// tc + 16 j, j < 4, accumulating in registers over the tile's tokens in order.
template <typename TIn, int MI>
__global__ __launch_bounds__(kThreads) void tile_outer_sums_kernel(
    const TIn* __restrict__ x, const TIn* __restrict__ y, float* __restrict__ records, int64_t T,
    int tile, int64_t tiles, int64_t rec, int Wa, int Wb) {
    extern __shared__ float smem[];
    constexpr int kWaPad = MI * 16;
    float* xs = smem;                          // [kStageTokens][kWaPad]
    float* ys = xs + kStageTokens * kWaPad;    // [kStageTokens][kSliceCols]
    const int tid = threadIdx.x;
    const int tr = tid >> 4, tc = tid & 15;
    const int64_t n = blockIdx.y;
    const int64_t ti = blockIdx.x;
    const int c0 = blockIdx.z * kSliceCols;
    const int ncols = min(kSliceCols, Wb - c0);
    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const TIn* xn = x + n * T * Wa;
    const TIn* yn = y + n * T * Wb;

    float acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    float asum = 0.f;

    for (int64_t t0 = t_begin; t0 < t_end; t0 += kStageTokens) {
        const int cnt = int(min<int64_t>(kStageTokens, t_end - t0));
        __syncthreads();
        for (int e = tid; e < kStageTokens * kWaPad; e += kThreads) {
            const int i = e / kWaPad, a = e - i * kWaPad;
            xs[e] = (i < cnt && a < Wa) ? ld(xn, (t0 + i) * Wa + a) : 0.f;
        }
        for (int e = tid; e < kStageTokens * kSliceCols; e += kThreads) {
            const int i = e / kSliceCols, c = e - i * kSliceCols;
            ys[e] = (i < cnt && c < ncols) ? ld(yn, (t0 + i) * Wb + c0 + c) : 0.f;
        }
        __syncthreads();
        for (int i = 0; i < cnt; ++i) {
            float yv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) yv[j] = ys[i * kSliceCols + tc + 16 * j];
#pragma unroll
            for (int ii = 0; ii < MI; ++ii) {
                const float xv = xs[i * kWaPad + tr + 16 * ii];
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[ii][j] = fmaf(xv, yv[j], acc[ii][j]);
            }
        }
        if (blockIdx.z == 0 && tid < Wa)
            for (int i = 0; i < cnt; ++i) asum += xs[i * kWaPad + tid];
    }

    float* r = records + (n * tiles + ti) * rec;
#pragma unroll
    for (int ii = 0; ii < MI; ++ii) {
        const int a = tr + 16 * ii;
        if (a >= Wa) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = tc + 16 * j;
            if (c < ncols) r[int64_t(a) * Wb + c0 + c] = acc[ii][j];
        }
    }
    if (blockIdx.z == 0 && tid < Wa) r[int64_t(Wa) * Wb + tid] = asum;
}

// ---------------------------------------------------------------------------
// Exclusive scan of the tile records over tiles, element-parallel like the
// reference's scan (docs/causal_v2_design.md:242-261) but two-level so that a
// long run of tiles is not one serial chain of loads: a workgroup owns
// kThreads / groups record elements of one stream and splits the tiles into
// `groups` contiguous groups (8 for long runs; 1 for runs of at most 32 tiles,
// where each thread walks all of them and a workgroup covers 256 contiguous
// elements).  Thread (element, group) sums its group; the group sums meet in
// LDS; each thread then walks its group again writing
//     prefix(t) = sum of the earlier groups (in group order)
//               + the earlier tiles of its group (in tile order).
// Every sum has a fixed order, so the result is bitwise reproducible.  With
// `reverse` the tiles are scanned from the last to the first (the suffix
// sums of the causal backward): record t receives the sum over tiles > t.
// `init` (nullable) is a carried state added before the first tile; every
// thread reads its element before the group barrier and only the last group
// writes `state`, so `state` may be `init`.
constexpr int kScanGroupsMax = 8;
constexpr int kScanRegTiles = 16;  // tiles per group held in registers

__global__ __launch_bounds__(kThreads) void tile_scan_kernel(float* __restrict__ records,
                                                             float* state, const float* init,
                                                             int64_t tiles, int64_t rec, int used,
                                                             int reverse, int groups) {
    __shared__ float gsum[kThreads];
    const int elems = kThreads / groups;
    const int el = threadIdx.x % elems, gi = threadIdx.x / elems;
    const int e = blockIdx.x * elems + el;
    const int64_t n = blockIdx.y;
    const int64_t per = (tiles + groups - 1) / groups;
    const int64_t t_begin = gi * per;
    const int64_t t_end = min(tiles, t_begin + per);
    // Scan position t is record r[t * step].
    const int64_t step = reverse ? -rec : rec;
    float* r = records + n * tiles * rec + (reverse ? (tiles - 1) * rec : 0) + e;
    float run = (init && e < used) ? init[n * used + e] : 0.f;
    if (groups > 1 && per <= kScanRegTiles) {
        // A group of at most kScanRegTiles tiles stays in registers between
        // its sum and its prefix pass: the records are read once.
        float v[kScanRegTiles];
        float sum = 0.f;
        const int cnt = e < used ? int(max<int64_t>(0, t_end - t_begin)) : 0;
#pragma unroll
        for (int u = 0; u < kScanRegTiles; ++u) v[u] = u < cnt ? r[(t_begin + u) * step] : 0.f;
#pragma unroll
        for (int u = 0; u < kScanRegTiles; ++u) sum += v[u];
        gsum[gi * elems + el] = sum;
        __syncthreads();
        for (int j = 0; j < gi; ++j) run += gsum[j * elems + el];
#pragma unroll
        for (int u = 0; u < kScanRegTiles; ++u) {
            if (u < cnt) r[(t_begin + u) * step] = run;
            run += v[u];
        }
        if (e < used && state && gi == groups - 1) state[n * used + e] = run;
        return;
    }
    if (groups > 1) {
        float sum = 0.f;
        if (e < used) {
            int64_t t = t_begin;
            for (; t + 16 <= t_end; t += 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v[u] = r[(t + u) * step];
#pragma unroll
                for (int u = 0; u < 16; ++u) sum += v[u];
            }
            for (; t < t_end; ++t) sum += r[t * step];
        }
        gsum[gi * elems + el] = sum;
        __syncthreads();
        for (int j = 0; j < gi; ++j) run += gsum[j * elems + el];
    }
    if (e >= used) return;
    int64_t t = t_begin;
    for (; t + 16 <= t_end; t += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = r[(t + u) * step];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            r[(t + u) * step] = run;
            run += v[u];
        }
    }
    for (; t < t_end; ++t) {
        const float v = r[t * step];
        r[t * step] = run;
        run += v;
    }
    if (state && gi == groups - 1) state[n * used + e] = run;
}

// tile_scan_kernel for short runs (one group: a thread walks every tile) on
// 16-byte vectors: thread e takes record elements 4 e .. 4 e + 3, with the
// same fixed order per element (so the same results bit for bit) and a
// quarter of the load, store and add instructions.  Runs of at most
// kScanRegTiles tiles are loaded whole before any prefix is stored.  For
// records whose used length is a multiple of 4 (records, `init` and `state`
// 16-byte aligned); `state` may be `init` (each thread reads its elements
// first and writes them last).
__global__ __launch_bounds__(kThreads) void tile_scan4_kernel(float* __restrict__ records, float* state,
                                                              const float* init, int64_t tiles, int64_t rec,
                                                              int used4, int reverse) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int e = blockIdx.x * kThreads + threadIdx.x;
    if (e >= used4) return;
    const int64_t n = blockIdx.y;
    const int64_t step4 = (reverse ? -rec : rec) / 4;
    f4* r = reinterpret_cast<f4*>(records + n * tiles * rec + (reverse ? (tiles - 1) * rec : 0)) + e;
    f4 run = init ? reinterpret_cast<const f4*>(init + n * int64_t(used4) * 4)[e] : f4{0.f, 0.f, 0.f, 0.f};
    if (tiles <= kScanRegTiles) {
        f4 v[kScanRegTiles];
        const int cnt = int(tiles);
#pragma unroll
        for (int u = 0; u < kScanRegTiles; ++u) v[u] = u < cnt ? r[u * step4] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kScanRegTiles; ++u) {
            if (u < cnt) r[u * step4] = run;
            run += v[u];
        }
    } else {
        int64_t t = 0;
        for (; t + 16 <= tiles; t += 16) {
            f4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = r[(t + u) * step4];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                r[(t + u) * step4] = run;
                run += v[u];
            }
        }
        for (; t < tiles; ++t) {
            const f4 v = r[t * step4];
            r[t * step4] = run;
            run += v;
        }
    }
    if (state) reinterpret_cast<f4*>(state + n * int64_t(used4) * 4)[e] = run;
}

__device__ __forceinline__ float sum_over_tiles(const float* __restrict__ r, int64_t tiles,
                                                int64_t rec) {
    float sum = 0.f;
    int64_t t = 0;
    for (; t + 8 <= tiles; t += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = r[(t + u) * rec];
#pragma unroll
        for (int u = 0; u < 8; ++u) sum += v[u];
    }
    for (; t < tiles; ++t) sum += r[t * rec];
    return sum;
}

// Totals over tiles (fixed order) into the state ([S*d + S]) when it is
// given, and E = B / (A + eps).  The thread of B element (s, c) also sums
// A[s] in the same order as the thread of A element s, so E uses exactly the
// A that is stored.
__global__ __launch_bounds__(kThreads) void tile_reduce_kernel(
    const float* __restrict__ records, float* __restrict__ state, float* __restrict__ E,
    int64_t tiles, int64_t rec, int S, int d) {
    const int e = blockIdx.x * kThreads + threadIdx.x;
    const int64_t n = blockIdx.y;
    const int used = S * d + S;
    if (e >= used) return;
    const float* r = records + n * tiles * rec;
    const float sum = sum_over_tiles(r + e, tiles, rec);
    if (state) state[n * used + e] = sum;
    if (E && e < S * d) {
        const int s = e / d;
        const float a = sum_over_tiles(r + S * d + s, tiles, rec);
        E[n * S * d + e] = sum / (a + kEps);
    }
}

// dE[s][c] = sum over the tiles of the dE records (in tile order);
// E[s][c] = B[s][c] / (A[s] + eps) from the forward state;
// dB = dE / (A + eps); dA[s] = -sum_c dE[s][c] E[s][c] / (A[s] + eps).
// One wave per bucket row s (kThreads / 64 rows per workgroup): lanes over
// the columns c (d <= 128: at most two per lane), the row's tile records
// loaded together, its products summed by a fixed shuffle tree.
__global__ __launch_bounds__(kThreads) void bwd_finalize_kernel(
    const float* __restrict__ dE_records, const float* __restrict__ state, float* __restrict__ dB,
    float* __restrict__ dA, int64_t tiles, int64_t rec, int S, int d) {
    const int lane = threadIdx.x & 63;
    const int s = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int64_t n = blockIdx.y;
    if (s >= S) return;
    const float* r = dE_records + n * tiles * rec + int64_t(s) * d;
    const float* Bn = state + n * (S * d + S) + int64_t(s) * d;
    float* dBn = dB + (n * S + s) * d;
    const float den = state[n * (S * d + S) + S * d + s] + kEps;
    const bool lo = lane < d, hi = lane + 64 < d;
    const int c0 = lo ? lane : 0, c1 = hi ? lane + 64 : 0;  // in bounds either way
    const float g0 = lo ? sum_over_tiles(r + c0, tiles, rec) : 0.f;
    const float g1 = hi ? sum_over_tiles(r + c1, tiles, rec) : 0.f;
    const float e0 = lo ? Bn[c0] / den : 0.f, e1 = hi ? Bn[c1] / den : 0.f;
    if (lo) dBn[lane] = g0 / den;
    if (hi) dBn[lane + 64] = g1 / den;
    float acc = fmaf(g1, e1, g0 * e0);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) dA[n * S + s] = -acc / den;
}

// ---------------------------------------------------------------------------
// Causal output pass, one workgroup per (tile, stream, 64-column slice).
// Walks the tile in sub-chunks of kValuChunk tokens with the state slice
// (A0 [S], B0 [S][64]) in LDS, starting from the tile's exclusive prefix.
template <typename TIn>
__global__ __launch_bounds__(kThreads) void causal_output_valu_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    TIn* __restrict__ out, const float* __restrict__ records, int64_t T, int S, int d, int tile,
    int64_t tiles, int64_t rec) {
    extern __shared__ float smem[];
    constexpr int C = kValuChunk;
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y;
    const int64_t ti = blockIdx.x;
    const int c0 = blockIdx.z * kSliceCols;
    const int ncols = min(kSliceCols, d - c0);
    float* B0 = smem;                  // [S][64]
    float* A0 = B0 + S * kSliceCols;   // [S]
    float* W = A0 + S;                 // [C][S]: q, then w = q / (Abar + eps)
    float* Ks = W + C * S;             // [C][S]
    float* Vs = Ks + C * S;            // [C][64]
    float* P = Vs + C * kSliceCols;    // [C][C]: tril(W K^T)

    const float* r = records + (n * tiles + ti) * rec;
    for (int e = tid; e < S * kSliceCols; e += kThreads) {
        const int s = e / kSliceCols, c = e - s * kSliceCols;
        B0[e] = c < ncols ? r[int64_t(s) * d + c0 + c] : 0.f;
    }
    for (int s = tid; s < S; s += kThreads) A0[s] = r[int64_t(S) * d + s];

    const int64_t t_begin = ti * tile;
    const int64_t t_end = min(T, t_begin + tile);
    const TIn* qn = q + n * T * S;
    const TIn* kn = k + n * T * S;
    const TIn* vn = v + n * T * d;
    TIn* on = out + n * T * d;

    for (int64_t t0 = t_begin; t0 < t_end; t0 += C) {
        const int cnt = int(min<int64_t>(C, t_end - t0));
        __syncthreads();
        for (int e = tid; e < cnt * S; e += kThreads) {
            W[e] = ld(qn, t0 * S + e);
            Ks[e] = ld(kn, t0 * S + e);
        }
        for (int e = tid; e < cnt * kSliceCols; e += kThreads) {
            const int i = e / kSliceCols, c = e - i * kSliceCols;
            Vs[e] = c < ncols ? ld(vn, (t0 + i) * d + c0 + c) : 0.f;
        }
        __syncthreads();
        // Inclusive running mass per bucket and the rescaled queries.
        for (int s = tid; s < S; s += kThreads) {
            float run = A0[s];
            for (int i = 0; i < cnt; ++i) {
                run += Ks[i * S + s];
                W[i * S + s] = W[i * S + s] / (run + kEps);
            }
            A0[s] = run;
        }
        __syncthreads();
        // P = tril(W K^T), diagonal included.
        for (int e = tid; e < cnt * cnt; e += kThreads) {
            const int i = e / cnt, j = e - i * cnt;
            float acc = 0.f;
            if (j <= i)
                for (int s = 0; s < S; ++s) acc = fmaf(W[i * S + s], Ks[j * S + s], acc);
            P[i * C + j] = acc;
        }
        __syncthreads();
        // O = W B0 + P V.
        for (int e = tid; e < cnt * kSliceCols; e += kThreads) {
            const int i = e / kSliceCols, c = e - i * kSliceCols;
            if (c >= ncols) continue;
            float acc = 0.f;
            for (int s = 0; s < S; ++s) acc = fmaf(W[i * S + s], B0[s * kSliceCols + c], acc);
            for (int j = 0; j <= i; ++j) acc = fmaf(P[i * C + j], Vs[j * kSliceCols + c], acc);
            store_val(on + (t0 + i) * d + c0 + c, acc);
        }
        __syncthreads();
        // B0 += K^T V.
        for (int e = tid; e < S * kSliceCols; e += kThreads) {
            const int s = e / kSliceCols, c = e - s * kSliceCols;
            float acc = 0.f;
            for (int i = 0; i < cnt; ++i) acc = fmaf(Ks[i * S + s], Vs[i * kSliceCols + c], acc);
            B0[e] += acc;
        }
    }
}

// ---------------------------------------------------------------------------
// out[t][c] = sum_a x[t][a] * M[a][c] (+ bias[c]) for the map operand's M,
// one workgroup per (kMapTokens tokens, stream, 64-column slice).  Thread
// (i, tc) = (tid / 8, tid % 8) computes token i, slice columns tc + 8 j.
template <typename TIn>
__global__ __launch_bounds__(kThreads) void token_map_kernel(
    const TIn* __restrict__ x, TIn* __restrict__ out, const MapOperand op, int64_t T, int Wa,
    int Wb) {
    extern __shared__ float smem[];
    float* Ms = smem;                    // [Wa][64]
    float* xs = Ms + Wa * kSliceCols;    // [kMapTokens][Wa]
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y;
    const int c0 = blockIdx.z * kSliceCols;
    const int ncols = min(kSliceCols, Wb - c0);
    const int64_t t0 = int64_t(blockIdx.x) * kMapTokens;
    const int cnt = int(min<int64_t>(kMapTokens, T - t0));
    const float* Mn = op.m + n * op.stream;
    const float* dv = op.div ? op.div + n * op.div_stream : nullptr;
    float* sv = op.save && blockIdx.x == 0 ? op.save + n * op.save_stream : nullptr;
    for (int e = tid; e < Wa * kSliceCols; e += kThreads) {
        const int a = e / kSliceCols, c = e - a * kSliceCols;
        float v = 0.f;
        if (c < ncols) {
            const int64_t mi = a * op.row + (c0 + c) * op.col;
            v = Mn[mi];
            for (int t = 1; t < op.parts; ++t) v += Mn[mi + t * op.part_stride];
            if (sv) sv[mi] = v;
            if (dv) {
                const int di = op.div_by_col ? c0 + c : a;
                float q = dv[di];
                for (int t = 1; t < op.parts; ++t) q += dv[di + t * op.part_stride];
                if (sv && (op.div_by_col ? a == 0 : (c == 0 && blockIdx.z == 0)))
                    sv[op.save_div_off + di] = q;
                v = v / (q + kEps);
            }
        }
        Ms[e] = v;
    }
    const TIn* xn = x + n * T * Wa;
    for (int e = tid; e < cnt * Wa; e += kThreads) xs[e] = ld(xn, t0 * Wa + e);
    __syncthreads();
    const int i = tid >> 3, tc = tid & 7;
    if (i >= cnt) return;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int a = 0; a < Wa; ++a) {
        const float xv = xs[i * Wa + a];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(xv, Ms[a * kSliceCols + tc + 8 * j], acc[j]);
    }
    TIn* on = out + (n * T + t0 + i) * Wb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = tc + 8 * j;
        if (c < ncols) {
            float val = acc[j];
            if (op.bias) val += op.bias[n * op.bias_stream + c0 + c];
            store_val(on + c0 + c, val);
        }
    }
}

int rows_per_thread(int Wa) {
    const int need = (Wa + 15) / 16;
    int mi = 1;
    while (mi < need) mi *= 2;
    return mi;
}

}  // namespace

hipError_t launch_tile_outer_sums(const void* x, const void* y, float* records, const Problem& p,
                                  int Wa, int Wb, hipStream_t stream) {
    const int mi = rows_per_thread(Wa);
    const dim3 grid(unsigned(p.tiles), unsigned(p.N), unsigned((Wb + kSliceCols - 1) / kSliceCols));
    const size_t lds = size_t(kStageTokens) * (mi * 16 + kSliceCols) * sizeof(float);
#define RACE_OUTER(TIN, MI)                                                                      \
    tile_outer_sums_kernel<TIN, MI><<<grid, kThreads, lds, stream>>>(                            \
        static_cast<const TIN*>(x), static_cast<const TIN*>(y), records, p.T, p.tile, p.tiles, \
        p.rec, Wa, Wb)
#define RACE_OUTER_MI(TIN)                     \
    switch (mi) {                              \
        case 1: RACE_OUTER(TIN, 1); break;     \
        case 2: RACE_OUTER(TIN, 2); break;     \
        case 4: RACE_OUTER(TIN, 4); break;     \
        case 8: RACE_OUTER(TIN, 8); break;     \
        default: RACE_OUTER(TIN, 16); break;   \
    }
    if (p.dtype == RACE_BF16) {
        RACE_OUTER_MI(bf16_t)
    } else {
        RACE_OUTER_MI(float)
    }
#undef RACE_OUTER_MI
#undef RACE_OUTER
    return hipGetLastError();
}

hipError_t launch_tile_scan(float* records, float* state, const Problem& p, hipStream_t stream,
                            bool reverse) {
    const int used = p.S * p.d + p.S;
    const int groups = p.tiles <= 32 ? 1 : kScanGroupsMax;
    const int elems = kThreads / groups;
    // Short runs (one group: a thread walks every tile) on 16-byte vectors:
    // at the cfg5 shape (4 tiles, 33024-element records) 33 -> 25.5 us for
    // the forward's scan and 49.6 -> 26.0 us for the backward's reverse scan
    // of the block records.  Long runs keep the scalar kernel (cfg2, 64
    // tiles in 8 groups: 7.7-7.8 us against 8.1-8.3 on vectors).
    if (groups == 1 && used % 4 == 0 && p.rec % 4 == 0) {
        const int used4 = used / 4;
        const dim3 grid(unsigned((used4 + kThreads - 1) / kThreads), unsigned(p.N));
        tile_scan4_kernel<<<grid, kThreads, 0, stream>>>(records, state, p.init, p.tiles, p.rec, used4,
                                                         reverse ? 1 : 0);
        return hipGetLastError();
    }
    const dim3 grid(unsigned((used + elems - 1) / elems), unsigned(p.N));
    tile_scan_kernel<<<grid, kThreads, 0, stream>>>(records, state, p.init, p.tiles, p.rec, used,
                                                    reverse ? 1 : 0, groups);
    return hipGetLastError();
}

hipError_t launch_tile_reduce(const float* records, float* state, float* E, const Problem& p,
                              hipStream_t stream) {
    const int used = p.S * p.d + p.S;
    const dim3 grid(unsigned((used + kThreads - 1) / kThreads), unsigned(p.N));
    tile_reduce_kernel<<<grid, kThreads, 0, stream>>>(records, state, E, p.tiles, p.rec, p.S, p.d);
    return hipGetLastError();
}

hipError_t launch_bwd_finalize(const float* dE_records, const float* state, float* dB, float* dA,
                               const Problem& p, hipStream_t stream) {
    static_assert(kThreads % 64 == 0, "whole waves");
    const dim3 grid(unsigned((p.S + kThreads / 64 - 1) / (kThreads / 64)), unsigned(p.N));
    bwd_finalize_kernel<<<grid, kThreads, 0, stream>>>(dE_records, state, dB, dA, p.tiles, p.rec,
                                                       p.S, p.d);
    return hipGetLastError();
}

size_t causal_output_valu_lds_bytes(int S) {
    const int C = kValuChunk;
    return size_t(S * kSliceCols + S + 2 * C * S + C * kSliceCols + C * C) * sizeof(float);
}

hipError_t launch_causal_output_valu(const void* q, const void* k, const void* v, void* out,
                                     const float* records, const Problem& p, hipStream_t stream) {
    const dim3 grid(unsigned(p.tiles), unsigned(p.N), unsigned((p.d + kSliceCols - 1) / kSliceCols));
    const size_t lds = causal_output_valu_lds_bytes(p.S);
    if (p.dtype == RACE_BF16) {
        causal_output_valu_kernel<bf16_t><<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
            static_cast<const bf16_t*>(v), static_cast<bf16_t*>(out), records, p.T, p.S, p.d,
            p.tile, p.tiles, p.rec);
    } else {
        causal_output_valu_kernel<float><<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(q), static_cast<const float*>(k),
            static_cast<const float*>(v), static_cast<float*>(out), records, p.T, p.S, p.d, p.tile,
            p.tiles, p.rec);
    }
    return hipGetLastError();
}

size_t token_map_lds_bytes(int Wa) {
    return size_t(Wa * kSliceCols + kMapTokens * Wa) * sizeof(float);
}

hipError_t launch_token_map(const void* x, void* out, const MapOperand& op, const Problem& p,
                            int Wa, int Wb, hipStream_t stream) {
    const dim3 grid(unsigned((p.T + kMapTokens - 1) / kMapTokens), unsigned(p.N),
                    unsigned((Wb + kSliceCols - 1) / kSliceCols));
    const size_t lds = token_map_lds_bytes(Wa);
    if (p.dtype == RACE_BF16) {
        token_map_kernel<bf16_t><<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(x), static_cast<bf16_t*>(out), op, p.T, Wa, Wb);
    } else {
        token_map_kernel<float><<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(x), static_cast<float*>(out), op, p.T, Wa, Wb);
    }
    return hipGetLastError();
}

}  // namespace race
