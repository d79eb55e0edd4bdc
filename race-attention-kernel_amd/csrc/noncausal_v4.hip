// noncausal_v4.hip -- vector-ALU bucket reductions and token maps of the
// non-causal forward and backward for widths that are multiples of 4.
//
// The non-causal function (analysis/hot-path.md:157-162) and its VJP are two
// kinds of pass over the tokens:
//   reduction  R[a][b] = sum_t x[t][a] y[t][b],  colsum[a] = sum_t x[t][a]
//              (B = K^T V and A in the forward, dE = Q^T dOut in the backward)
//   map        out[t][c] = sum_a x[t][a] M[a][c] (+ bias[c])
//              (out = Q E, dQ = dOut E^T, dK = V dB^T + dA, dV = K dB)
// Both are fp32 vector-ALU code (no matrix cores): every thread owns a
// register tile (8 x 4 for 64-wide operands, 4 x 4 otherwise), operands are
// read from LDS as 16-byte vectors, and tokens are staged with 16-byte
// (fp32) or 8-byte (bf16) coalesced loads.  A reduction workgroup owns one
// chunk of one stream's tokens and writes the chunk's partial sums to a
// record; the records are added in chunk order (by the map that stages the
// matrix, by the backward's finalize, or by tile_reduce_kernel for long
// sequences), so results are bitwise reproducible.
#include "mfma_common.h"

namespace race {
namespace {

constexpr int kRedTokens = 32;   // tokens staged per step of a reduction (64 measured slower)
constexpr int kMapTokens4 = 64;  // tokens per map block (4-token tiles x 16)
constexpr int kMapBlocks = 4;    // map blocks per workgroup (M staged once)

// Four consecutive elements (16-byte aligned for fp32, 8-byte for bf16).
__device__ __forceinline__ float4 load4(const float* __restrict__ p) {
    return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ float4 load4(const bf16_t* __restrict__ p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                       __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

__device__ __forceinline__ void store4(float* __restrict__ p, const float4& v) {
    *reinterpret_cast<float4*>(p) = v;
}
__device__ __forceinline__ void store4(bf16_t* __restrict__ p, const float4& v) {
    uint2 u;
    u.x = uint32_t(f32_to_bf16(v.x)) | (uint32_t(f32_to_bf16(v.y)) << 16);
    u.y = uint32_t(f32_to_bf16(v.z)) | (uint32_t(f32_to_bf16(v.w)) << 16);
    *reinterpret_cast<uint2*>(p) = u;
}

// Cache policy of the token loads and of the fp32 token stores of these
// kernels (0 default, 2 nontemporal).  Nontemporal fp32 stores measured about
// 5% faster on the cfg4 maps; nontemporal loads no different.
#ifndef RACE_NC_LOAD_POLICY
#define RACE_NC_LOAD_POLICY 0
#endif
#ifndef RACE_NC_STORE_POLICY
#define RACE_NC_STORE_POLICY 2
#endif
constexpr int kNcLoadPolicy = RACE_NC_LOAD_POLICY;
constexpr int kNcStorePolicy = RACE_NC_STORE_POLICY;

// The same through a buffer view (offsets in bytes): out-of-range loads read
// zeros and out-of-range stores are dropped.  kOutside is past any view.
constexpr int kOutside = 0x7ffffff0;
template <typename TIn>
__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (std::is_same<TIn, float>::value) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNcLoadPolicy));
    } else {
        const uint2 u = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNcLoadPolicy));
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                           __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    }
}
template <typename TIn>
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, int off, const float4& v) {
    if constexpr (std::is_same<TIn, float>::value) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(mfma::u32x4, v), r, off, 0, kNcStorePolicy);
    } else {
        const mfma::u32x2 u{uint32_t(f32_to_bf16(v.x)) | (uint32_t(f32_to_bf16(v.y)) << 16),
                            uint32_t(f32_to_bf16(v.z)) | (uint32_t(f32_to_bf16(v.w)) << 16)};
        __builtin_amdgcn_raw_buffer_store_b64(u, r, off, 0, 0);
    }
}

// ---------------------------------------------------------------------------
// Reduction over one (chunk, stream).  Tile u = tid + kThreads m covers rows
// 4 (u / (Wb / 4)) .. + 3 and columns 4 (u % (Wb / 4)) .. + 3 of R.
// NV: 16-byte token vectors each thread stages per step; NT: tiles per thread.
template <typename TIn, int NV, int NT>
__global__ __launch_bounds__(kThreads) void outer_sums4_kernel(
    const TIn* __restrict__ x, const TIn* __restrict__ y, float* __restrict__ records, int64_t T,
    int chunk, int64_t chunks, int64_t rec, int Wa, int Wb) {
    extern __shared__ float smem[];
    float* xs = smem;                      // [2][kRedTokens][Wa]
    float* ys = xs + 2 * kRedTokens * Wa;  // [2][kRedTokens][Wb]
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y, ci = blockIdx.x;
    const int64_t t_begin = ci * chunk;
    const int64_t t_end = min(T, t_begin + chunk);
    const int va = Wa / 4, vb = Wb / 4, vrow = va + vb;
    const int nvec = kRedTokens * vrow;
    const int ntiles = va * vb;
    const TIn* xn = x + n * T * Wa;
    const TIn* yn = y + n * T * Wb;

    // One load per vector from a per-lane address (x or y row; a valid row
    // when out of range, zeroed when staged): branches around the loads, or
    // zeroing right after them, made the compiler wait for each load in turn.
    float4 pre[NV];
    auto fetch = [&](int64_t t0) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + m * kThreads;
            const int i = e / vrow, u = e - i * vrow;
            const int64_t t = e < nvec && t0 + i < t_end ? t0 + i : t_begin;
            pre[m] = load4(u < va ? xn + t * Wa + 4 * u : yn + t * Wb + 4 * (u - va));
        }
    };
    auto stash = [&](int buf, int64_t t0) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + m * kThreads;
            if (e < nvec) {
                const int i = e / vrow, u = e - i * vrow;
                const float4 val = t0 + i < t_end ? pre[m] : make_float4(0.f, 0.f, 0.f, 0.f);
                if (u < va)
                    store4(xs + (buf * kRedTokens + i) * Wa + 4 * u, val);
                else
                    store4(ys + (buf * kRedTokens + i) * Wb + 4 * (u - va), val);
            }
        }
    };

    float acc[NT][4][4];
    float csum[NT][4];
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            csum[m][r] = 0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[m][r][c] = 0.f;
        }

    fetch(t_begin);
    stash(0, t_begin);
    __syncthreads();
    int buf = 0;
    for (int64_t t0 = t_begin; t0 < t_end; t0 += kRedTokens) {
        const bool more = t0 + kRedTokens < t_end;
        if (more) fetch(t0 + kRedTokens);
        const float* xb = xs + buf * kRedTokens * Wa;
        const float* yb = ys + buf * kRedTokens * Wb;
        for (int i = 0; i < kRedTokens; ++i) {
#pragma unroll
            for (int m = 0; m < NT; ++m) {
                const int u = tid + m * kThreads;
                if (u < ntiles) {
                    const int a4 = u / vb, b4 = u - a4 * vb;
                    const float4 xv = *reinterpret_cast<const float4*>(xb + i * Wa + 4 * a4);
                    const float4 yv = *reinterpret_cast<const float4*>(yb + i * Wb + 4 * b4);
                    const float xr[4] = {xv.x, xv.y, xv.z, xv.w};
                    const float yc[4] = {yv.x, yv.y, yv.z, yv.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        csum[m][r] += xr[r];
#pragma unroll
                        for (int c = 0; c < 4; ++c) acc[m][r][c] = fmaf(xr[r], yc[c], acc[m][r][c]);
                    }
                }
            }
        }
        if (more) stash(buf ^ 1, t0 + kRedTokens);
        __syncthreads();
        buf ^= 1;
    }

    float* rp = records + (n * chunks + ci) * rec;
#pragma unroll
    for (int m = 0; m < NT; ++m) {
        const int u = tid + m * kThreads;
        if (u < ntiles) {
            const int a4 = u / vb, b4 = u - a4 * vb;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                store4(rp + int64_t(4 * a4 + r) * Wb + 4 * b4,
                       make_float4(acc[m][r][0], acc[m][r][1], acc[m][r][2], acc[m][r][3]));
                if (b4 == 0) rp[int64_t(Wa) * Wb + 4 * a4 + r] = csum[m][r];
            }
        }
    }
}

// Reductions with Wa = Wb = 64 (every reduction of the S = d = 64 shapes).
// Threads 0..127 take tokens 0..15 of each staged block of kRedTokens and
// threads 128..255 tokens 16..31; each owns an 8 x 4 tile of R (rows
// 8 (u / 16) .., columns 4 (u % 16) .., u = tid % 128), so three 16-byte LDS
// reads feed 32 FMAs.  The column sums of x are taken once per block, thread
// tid summing 8 tokens of column tid % 64.  At the end the two halves of R and
// the four token groups of the column sums are added in a fixed order through
// LDS, so results stay bitwise reproducible.
template <typename TIn>
__global__ __launch_bounds__(kThreads) void outer64_kernel(
    const TIn* __restrict__ x, const TIn* __restrict__ y, float* __restrict__ records, int64_t T,
    int chunk, int64_t chunks, int64_t rec) {
    constexpr int W = 64;
    constexpr int NV = kRedTokens * (2 * W / 4) / kThreads;  // 16-byte vectors per thread and block
    extern __shared__ float smem[];
    float* xs = smem;                      // [2][kRedTokens][W]
    float* ys = xs + 2 * kRedTokens * W;   // [2][kRedTokens][W]
    float* part = smem;                    // [W][W] + [4][W], after the loop
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y, ci = blockIdx.x;
    const int64_t t_begin = ci * chunk;
    const int64_t t_end = min(T, t_begin + chunk);
    const TIn* xn = x + n * T * W;
    const TIn* yn = y + n * T * W;
    const int half = tid >> 7, u = tid & 127;
    const int a8 = u >> 4, b4 = u & 15;
    const int ca = tid & 63, cg = tid >> 6;  // column-sum column and token group

    // Staging: vectors m < NV / 2 are x rows, the rest y rows, so each load
    // instruction reads one tensor (whole 256-byte rows, no divergence), and
    // rows past the chunk read as zero through the buffer views.
    static_assert(NV % 2 == 0 && (NV / 2) * kThreads == kRedTokens * (W / 4), "x, y halves");
    const int rows = int(t_end - t_begin);
    const auto xr = mfma::make_rsrc(xn + t_begin * W, int64_t(rows) * W * int64_t(sizeof(TIn)));
    const auto yr = mfma::make_rsrc(yn + t_begin * W, int64_t(rows) * W * int64_t(sizeof(TIn)));
    float4 pre[NV];
    auto fetch = [&](int r0) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + (m % (NV / 2)) * kThreads;
            const int i = e >> 4, v = e & 15;  // token, vector
            pre[m] = buf_load4<TIn>(m < NV / 2 ? xr : yr, ((r0 + i) * W + 4 * v) * int(sizeof(TIn)));
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + (m % (NV / 2)) * kThreads;
            const int i = e >> 4, v = e & 15;
            store4((m < NV / 2 ? xs : ys) + (buf * kRedTokens + i) * W + 4 * v, pre[m]);
        }
    };

    float acc[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = 0.f;
    float csum = 0.f;

    fetch(0);
    stash(0);
    __syncthreads();
    int buf = 0;
    for (int r0 = 0; r0 < rows; r0 += kRedTokens) {
        const bool more = r0 + kRedTokens < rows;
        if (more) fetch(r0 + kRedTokens);
        const float* xb = xs + (buf * kRedTokens + 16 * half) * W;
        const float* yb = ys + (buf * kRedTokens + 16 * half) * W;
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
            const float4 x0 = *reinterpret_cast<const float4*>(xb + i * W + 8 * a8);
            const float4 x1 = *reinterpret_cast<const float4*>(xb + i * W + 8 * a8 + 4);
            const float4 yv = *reinterpret_cast<const float4*>(yb + i * W + 4 * b4);
            const float xr[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const float yc[4] = {yv.x, yv.y, yv.z, yv.w};
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(xr[r], yc[c], acc[r][c]);
        }
        const float* xc = xs + (buf * kRedTokens + 8 * cg) * W + ca;
#pragma unroll
        for (int i = 0; i < 8; ++i) csum += xc[i * W];
        if (more) stash(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // Fixed-order combination: R = half 0 + half 1, colsum = groups 0 + 1 + 2 + 3.
    float* rp = records + (n * chunks + ci) * rec;
    float* cs = part + W * W;
    cs[cg * W + ca] = csum;
    if (half == 1) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
            store4(part + (8 * a8 + r) * W + 4 * b4, make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]));
    }
    __syncthreads();
    if (half == 0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const float4 o = *reinterpret_cast<const float4*>(part + (8 * a8 + r) * W + 4 * b4);
            store4(rp + (8 * a8 + r) * W + 4 * b4,
                   make_float4(acc[r][0] + o.x, acc[r][1] + o.y, acc[r][2] + o.z, acc[r][3] + o.w));
        }
    } else if (u < W) {
        rp[W * W + u] = ((cs[u] + cs[W + u]) + cs[2 * W + u]) + cs[3 * W + u];
    }
}

// ---------------------------------------------------------------------------
// Map over kMapBlocks blocks of kMapTokens4 tokens of one stream, for one
// slice of 64 output columns.  M slice [Wa][64] and the block's tokens,
// transposed ([Wa][kMapTokens4 + 4]), sit in LDS; thread (tt, cc) =
// (tid / 16, tid % 16) computes tokens 4 tt .. + 3, slice columns 4 cc .. + 3.
// In row a of the transposed tile, the group of tokens 4 g .. 4 g + 3 sits at
// group g ^ xsw(a): the staging stores of one instruction (16 rows 4 apart)
// then spread over the banks, and the 16-byte reads stay aligned.
// NV: 16-byte token vectors each thread stages per block.
__device__ __forceinline__ int xsw(int a) { return (a >> 2) & 7; }

// Sum of `parts` values `stride` apart, in order (parts = 1: one load).
__device__ __forceinline__ float sum_parts(const float* __restrict__ p, int parts, int64_t stride) {
    float v = p[0];
    for (int t = 1; t < parts; ++t) v += p[t * stride];
    return v;
}

// Parts (tile records) a slice stages with every load in flight at once: the
// non-causal forward folds at most this many per stream.
constexpr int kSliceParts = 4;

// Ms[a][c] = M[a][c0 + c] of the map operand for stream n (divided by its
// divisor when it has one) for the slice's columns c < ncols, zero beyond,
// a < Wa; the first token block's workgroups also save the undivided values
// when the operand asks for it.  The loads go out in groups of 8 before
// their LDS stores: a plain loop waited for each load before the next (one
// memory round trip per element).
__device__ __forceinline__ void stage_slice(float* __restrict__ Ms, const MapOperand& op,
                                            int64_t n, int Wa, int c0, int ncols) {
    constexpr int kRows = kThreads / kSliceCols;  // rows of the slice per pass
    const int c = threadIdx.x % kSliceCols, a0 = threadIdx.x / kSliceCols;
    const bool ok = c < ncols;
    const int cg = c0 + (ok ? c : 0);  // in bounds either way
    const float* col = op.m + n * op.stream + cg * op.col;
    const float* dv = op.div ? op.div + n * op.div_stream : nullptr;
    float* sv = op.save && blockIdx.x == 0 ? op.save + n * op.save_stream : nullptr;
    for (int ab = 0; ab < Wa; ab += 8 * kRows) {
        float v[8], q[8];
        if (op.parts <= kSliceParts) {
            // Every part of the 8 rows is requested before the sums (a loop
            // over the parts waited for each part in turn); the sums run in
            // part order, as sum_parts adds them.
            float vp[kSliceParts][8], qp[kSliceParts][8];
#pragma unroll
            for (int t = 0; t < kSliceParts; ++t) {
                const int64_t po = int64_t(min(t, op.parts - 1)) * op.part_stride;
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    const int a = min(ab + a0 + m * kRows, Wa - 1);  // clamped: no branch
                    vp[t][m] = col[a * op.row + po];
                    qp[t][m] = dv ? dv[(op.div_by_col ? cg : a) + po] : 0.f;
                }
            }
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                v[m] = vp[0][m];
                q[m] = qp[0][m];
#pragma unroll
                for (int t = 1; t < kSliceParts; ++t)
                    if (t < op.parts) {
                        v[m] += vp[t][m];
                        q[m] += qp[t][m];
                    }
            }
        } else {
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const int a = min(ab + a0 + m * kRows, Wa - 1);
                v[m] = sum_parts(col + a * op.row, op.parts, op.part_stride);
                q[m] = dv ? sum_parts(dv + (op.div_by_col ? cg : a), op.parts, op.part_stride) : 0.f;
            }
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int a = ab + a0 + m * kRows;
            if (a >= Wa) continue;
            Ms[a * kSliceCols + c] = ok ? (dv ? v[m] / (q[m] + kEps) : v[m]) : 0.f;
            if (sv && ok) {
                sv[a * op.row + cg * op.col] = v[m];
                // Each divisor once: by its column's threads in the first
                // slice (by column) or by column 0 of the first slice (by row).
                if (dv && (op.div_by_col ? a == 0 : (c == 0 && blockIdx.z == 0)))
                    sv[op.save_div_off + (op.div_by_col ? cg : a)] = q[m];
            }
        }
    }
}

// The bias of the slice's 4 columns 4 cc .. + 3 (zero past ncols or without
// a bias).
__device__ __forceinline__ float4 slice_bias(const MapOperand& op, int64_t n, int c0, int cc,
                                             int ncols) {
    if (!op.bias || 4 * cc >= ncols) return make_float4(0.f, 0.f, 0.f, 0.f);
    const float* bn = op.bias + n * op.bias_stream + c0 + 4 * cc;
    return make_float4(bn[0], 4 * cc + 1 < ncols ? bn[1] : 0.f, 4 * cc + 2 < ncols ? bn[2] : 0.f,
                       4 * cc + 3 < ncols ? bn[3] : 0.f);
}

template <typename TIn, int NV>
__global__ __launch_bounds__(kThreads) void map4_kernel(
    const TIn* __restrict__ x, TIn* __restrict__ out, const MapOperand op, int64_t T, int Wa,
    int Wb) {
    extern __shared__ float smem[];
    constexpr int TP = kMapTokens4 + 4;  // pitch of the transposed token tile
    float* Ms = smem;                    // [Wa][64]
    float* xt = Ms + Wa * kSliceCols;    // [Wa][TP]
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y;
    const int c0 = blockIdx.z * kSliceCols;
    const int ncols = min(kSliceCols, Wb - c0);
    const int va = Wa / 4;
    const int nvec = kMapTokens4 * va;
    const int tt = tid >> 4, cc = tid & 15;
    // Buffer views of the workgroup's rows (rows past T read as zero, their
    // stores are dropped): every load and store is unconditional, so the
    // compiler neither waits for each load in turn nor, with the block loop
    // unrolled, for the previous block's stores before using a prefetch.
    const int64_t wg_t0 = int64_t(blockIdx.x) * kMapBlocks * kMapTokens4;
    const int64_t wg_rows = min(T - wg_t0, int64_t(kMapBlocks) * kMapTokens4);
    const auto xr = mfma::make_rsrc(x + (n * T + wg_t0) * Wa, wg_rows * Wa * int64_t(sizeof(TIn)));
    const auto orr = mfma::make_rsrc(out + (n * T + wg_t0) * Wb, wg_rows * Wb * int64_t(sizeof(TIn)));

    // The next block's token vectors are loaded into registers while the
    // current block computes.
    float4 pre[NV];
    auto fetch = [&](int r0) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + m * kThreads;
            const int i = e / va, u = e - i * va;
            pre[m] = buf_load4<TIn>(xr, e < nvec ? ((r0 + i) * Wa + 4 * u) * int(sizeof(TIn)) : kOutside);
        }
    };
    // The first block's tokens are requested before the matrix slice is
    // staged, so the two round trips overlap.
    fetch(0);
    stage_slice(Ms, op, n, Wa, c0, ncols);
    const float4 bv = slice_bias(op, n, c0, cc, ncols);
#pragma unroll
    for (int blk = 0; blk < kMapBlocks; ++blk) {
        const int r0 = blk * kMapTokens4;
        if (r0 >= wg_rows) break;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + m * kThreads;
            if (e < nvec) {
                const int i = e / va, u = e - i * va;
                const int col = i ^ (xsw(4 * u) << 2);  // rows 4u .. 4u+3 share xsw
                xt[(4 * u + 0) * TP + col] = pre[m].x;
                xt[(4 * u + 1) * TP + col] = pre[m].y;
                xt[(4 * u + 2) * TP + col] = pre[m].z;
                xt[(4 * u + 3) * TP + col] = pre[m].w;
            }
        }
        __syncthreads();
        if (blk + 1 < kMapBlocks) fetch(r0 + kMapTokens4);
        float acc[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[r][0] = bv.x;
            acc[r][1] = bv.y;
            acc[r][2] = bv.z;
            acc[r][3] = bv.w;
        }
        for (int a = 0; a < Wa; ++a) {
            const float4 xv = *reinterpret_cast<const float4*>(xt + a * TP + 4 * (tt ^ xsw(a)));
            const float4 mv = *reinterpret_cast<const float4*>(Ms + a * kSliceCols + 4 * cc);
            const float xr[4] = {xv.x, xv.y, xv.z, xv.w};
            const float mc[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(xr[r], mc[c], acc[r][c]);
        }
        const bool col_ok = 4 * cc < ncols;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int off = ((r0 + 4 * tt + r) * Wb + c0 + 4 * cc) * int(sizeof(TIn));
            buf_store4<TIn>(orr, col_ok ? off : kOutside,
                            make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]));
        }
    }
}

// Maps with a 64-wide contraction (Wa = 64: every map of the S = d = 64
// shapes).  Each thread owns 8 tokens x 4 columns, so three 16-byte LDS reads
// feed 32 FMAs (4 x 4 tiles need two for 16), and the swizzled addresses are
// computed once per group of four contraction rows.  Blocks of 128 tokens, the
// same transposed and swizzled token tile as map4_kernel.
constexpr int kMap64Tokens = 128;
constexpr int kMap64Blocks = 4;

template <typename TIn>
__global__ __launch_bounds__(kThreads) void map64_kernel(
    const TIn* __restrict__ x, TIn* __restrict__ out, const MapOperand op, int64_t T, int Wb) {
    constexpr int Wa = 64;
    constexpr int TP = kMap64Tokens + 4;                   // pitch of the transposed token tile
    constexpr int NV = kMap64Tokens * (Wa / 4) / kThreads;  // 16-byte token vectors per thread
    extern __shared__ float smem[];
    float* Ms = smem;                  // [64][64]
    float* xt = Ms + Wa * kSliceCols;  // [64][TP]
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y;
    const int c0 = blockIdx.z * kSliceCols;
    const int ncols = min(kSliceCols, Wb - c0);
    const int tt = tid >> 4, cc = tid & 15;  // tokens 8 tt .. 8 tt + 7, columns 4 cc .. 4 cc + 3
    // Buffer views of the workgroup's rows: rows past T read as zero and
    // their stores are dropped, so every load and store is unconditional.
    // With the block loop unrolled the compiler then counts the stores
    // issued after each prefetch and waits for the prefetched tokens only; a
    // rolled loop with conditional stores waited for the previous block's
    // stores too (10% slower).
    const int64_t wg_t0 = int64_t(blockIdx.x) * kMap64Blocks * kMap64Tokens;
    const int64_t wg_rows = min(T - wg_t0, int64_t(kMap64Blocks) * kMap64Tokens);
    const auto xr = mfma::make_rsrc(x + (n * T + wg_t0) * Wa, wg_rows * Wa * int64_t(sizeof(TIn)));
    const auto orr = mfma::make_rsrc(out + (n * T + wg_t0) * Wb, wg_rows * Wb * int64_t(sizeof(TIn)));

    float4 pre[NV];
    auto fetch = [&](int r0) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + m * kThreads;
            const int i = e >> 4, u = e & 15;
            pre[m] = buf_load4<TIn>(xr, ((r0 + i) * Wa + 4 * u) * int(sizeof(TIn)));
        }
    };
    // The first block's tokens are requested before the matrix slice is
    // staged, so the two round trips overlap.
    fetch(0);
    stage_slice(Ms, op, n, Wa, c0, ncols);
    const float4 bv = slice_bias(op, n, c0, cc, ncols);
#pragma unroll
    for (int blk = 0; blk < kMap64Blocks; ++blk) {
        const int r0 = blk * kMap64Tokens;
        if (r0 >= wg_rows) break;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = tid + m * kThreads;
            const int i = e >> 4, u = e & 15;
            const int col = i ^ (xsw(4 * u) << 2);  // rows 4u .. 4u+3 share xsw
            xt[(4 * u + 0) * TP + col] = pre[m].x;
            xt[(4 * u + 1) * TP + col] = pre[m].y;
            xt[(4 * u + 2) * TP + col] = pre[m].z;
            xt[(4 * u + 3) * TP + col] = pre[m].w;
        }
        __syncthreads();
        if (blk + 1 < kMap64Blocks) fetch(r0 + kMap64Tokens);
        float acc[8][4];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            acc[r][0] = bv.x;
            acc[r][1] = bv.y;
            acc[r][2] = bv.z;
            acc[r][3] = bv.w;
        }
        // Rows 4 j .. 4 j + 3 share one swizzle: the group's addresses are
        // computed once and its four steps unrolled.
#pragma unroll 2
        for (int j = 0; j < Wa / 4; ++j) {
            const int sw = (j & 7) << 2;
            const float* xa = xt + 4 * j * TP;
            const int o0 = (8 * tt) ^ sw, o1 = (8 * tt + 4) ^ sw;
            const float* ma = Ms + 4 * j * kSliceCols + 4 * cc;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 x0 = *reinterpret_cast<const float4*>(xa + k * TP + o0);
                const float4 x1 = *reinterpret_cast<const float4*>(xa + k * TP + o1);
                const float4 mv = *reinterpret_cast<const float4*>(ma + k * kSliceCols);
                const float xr8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const float mc[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(xr8[r], mc[c], acc[r][c]);
            }
        }
        const bool col_ok = 4 * cc < ncols;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int off = ((r0 + 8 * tt + r) * Wb + c0 + 4 * cc) * int(sizeof(TIn));
            buf_store4<TIn>(orr, col_ok ? off : kOutside,
                            make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]));
        }
    }
}

// ---------------------------------------------------------------------------
// The backward at S = d = 64 in two passes, split the way the reference
// splits its non-causal backward (src/noncausal/kernels/race_bwd.cu:4-28:
// query side, bucket gradients, key side):
//   query side  dQ[t][s] = sum_c G[t][c] E[s][c]   (G = dOut)
//               dE[s][c] = sum_t Q[t][s] G[t][c]   (one record per tile)
//   key side    dB = dE / (A + eps), dA[s] = -sum_c dE[s][c] E[s][c] / (A[s] + eps)
//               dK[t][s] = sum_c V[t][c] dB[s][c] + dA[s],  dV[t][c] = sum_s K[t][s] dB[s][c]
// so dOut is read once, and the bucket gradients are formed by every key-side
// workgroup as it stages them (no separate finalize launch for up to
// kFoldParts tiles per stream).
//
// Both kernels walk their tokens in stages of kGradStage rows of two tensors,
// staged row-major in LDS with the next stage's rows in registers.  Map
// thread (tt, cc) = (tid / 16, tid % 16) computes tokens tt + 16 r (r < 4)
// and the 4 output columns 4 cc .. + 3; in a wave the four tt are adjacent
// rows, so the 16-byte slot j of row i is stored at slot j ^ (i & 3) and the
// four rows' reads fall in different banks.
constexpr int kGradStage = 64;
constexpr int kFoldParts = kKeyGradFoldParts;
constexpr int kGradBlocks = 3;  // workgroups per CU the two passes are built for (LDS allows 3)
// Rows of dB a key-side thread forms per round of record loads (16 in all;
// 8 per round measured the same as 4 at cfg4, 16 spills).
#ifndef RACE_KEY_GRAD_ROWS
#define RACE_KEY_GRAD_ROWS 4
#endif
constexpr int kKeyGradRows = RACE_KEY_GRAD_ROWS;

// The slot of a stage row (16-byte slots XORed by row & 3).
__device__ __forceinline__ int row_slot(int i, int j) { return j ^ (i & 3); }

template <typename TIn>
struct GradStage {
    static constexpr int W = 64;
    static constexpr int NV = kGradStage * (W / 4) / kThreads;  // 16-byte vectors per tensor and thread
    float4 pa[NV], pb[NV];
    __device__ __forceinline__ void fetch(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, int r0) {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = threadIdx.x + m * kThreads;
            const int i = e >> 4, v = e & 15;
            pa[m] = buf_load4<TIn>(ra, ((r0 + i) * W + 4 * v) * int(sizeof(TIn)));
        }
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = threadIdx.x + m * kThreads;
            const int i = e >> 4, v = e & 15;
            pb[m] = buf_load4<TIn>(rb, ((r0 + i) * W + 4 * v) * int(sizeof(TIn)));
        }
    }
    // a rows plain (swizzle_a false) or swizzled, b rows swizzled.
    template <bool kSwizzleA>
    __device__ __forceinline__ void stash(float* __restrict__ as, float* __restrict__ bs) const {
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            const int e = threadIdx.x + m * kThreads;
            const int i = e >> 4, v = e & 15;
            store4(as + i * W + 4 * (kSwizzleA ? row_slot(i, v) : v), pa[m]);
            store4(bs + i * W + 4 * row_slot(i, v), pb[m]);
        }
    }
};

// Query side: one workgroup per (tile, stream).  LDS: E transposed (pitch
// kEtPitch), the stage's Q rows (plain) and G rows (swizzled).  Reduction:
// threads 0..127 take tokens 0..15 of every 32, 128..255 tokens 16..31, each
// an 8 x 4 tile of dE (rows 8 (u / 16) .., columns 4 (u % 16) .., u = tid %
// 128), the two halves added in a fixed order at the end: outer64_kernel's
// order, so the records are the same whichever kernel forms them.  A ragged last tile reads
// zero rows past T (buffer views), which add nothing, and drops their stores.
constexpr int kEtPitch = 68;

template <typename TIn>
__global__ __launch_bounds__(kThreads, kGradBlocks) void query_grad64_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ g, TIn* __restrict__ dq,
    const float* __restrict__ state, float* __restrict__ records, int64_t T, int chunk,
    int64_t chunks, int64_t rec) {
    constexpr int W = 64, ST = kGradStage;
    extern __shared__ float smem[];
    float* Et = smem;                // [64 c][kEtPitch]: Et[c][s] = E[s][c]
    float* qs = Et + W * kEtPitch;   // [ST][64]
    float* gs = qs + ST * W;         // [ST][64], swizzled
    float* part = qs;                // [64][64] after the loop
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y, ci = blockIdx.x;
    const int64_t t_begin = ci * chunk;
    const int rows = int(min(T, t_begin + chunk) - t_begin);
    const int64_t es = sizeof(TIn);
    const auto qr = mfma::make_rsrc(q + (n * T + t_begin) * W, int64_t(rows) * W * es);
    const auto gr = mfma::make_rsrc(g + (n * T + t_begin) * W, int64_t(rows) * W * es);
    const auto dr = mfma::make_rsrc(dq + (n * T + t_begin) * W, int64_t(rows) * W * es);

    GradStage<TIn> st;
    st.fetch(qr, gr, 0);
    // E[s][c] = B[s][c] / (A[s] + eps) from the state, transposed into LDS:
    // lane c of wave w takes rows s = w + 4 m (coalesced loads, all issued
    // before the first division).
    {
        const int c = tid & 63, s0 = tid >> 6;
        const float* sn = state + n * (W * W + W);
        float b[16], a[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            b[m] = sn[(s0 + 4 * m) * W + c];
            a[m] = sn[W * W + s0 + 4 * m];
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) Et[c * kEtPitch + s0 + 4 * m] = b[m] / (a[m] + kEps);
    }

    const int half = tid >> 7, u = tid & 127;
    const int a8 = u >> 4, b4 = u & 15;
    const int tt = tid >> 4, cc = tid & 15;
    float acc[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = 0.f;

    for (int r0 = 0; r0 < rows; r0 += ST) {
        __syncthreads();
        st.template stash<false>(qs, gs);
        __syncthreads();
        if (r0 + ST < rows) st.fetch(qr, gr, r0 + ST);
        // dE partial over this thread's 32 tokens of the stage: of each 32
        // tokens, half 0 takes the first 16 and half 1 the next 16, in order
        // (outer64_kernel's split, so the records agree bit for bit).  The
        // next token's operands are read while the current token's products
        // run (two register sets).
#pragma unroll 2
        for (int i = 0; i < ST / 2; i += 2) {
            // Two tokens' operands are read before their products run.
            float4 x0[2], x1[2], yv[2];
#pragma unroll
            for (int u2 = 0; u2 < 2; ++u2) {
                const int ii = i + u2;
                const int t = 32 * (ii >> 4) + 16 * half + (ii & 15);
                x0[u2] = *reinterpret_cast<const float4*>(qs + t * W + 8 * a8);
                x1[u2] = *reinterpret_cast<const float4*>(qs + t * W + 8 * a8 + 4);
                yv[u2] = *reinterpret_cast<const float4*>(gs + t * W + 4 * row_slot(t, b4));
            }
#pragma unroll
            for (int u2 = 0; u2 < 2; ++u2) {
                const float xr[8] = {x0[u2].x, x0[u2].y, x0[u2].z, x0[u2].w,
                                     x1[u2].x, x1[u2].y, x1[u2].z, x1[u2].w};
                const float yc[4] = {yv[u2].x, yv[u2].y, yv[u2].z, yv[u2].w};
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(xr[r], yc[c], acc[r][c]);
            }
        }
        // dQ for tokens tt + 16 r, buckets 4 cc .. + 3 (contraction over c in
        // order, as the map kernels do).
        float mo[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c) mo[r][c] = 0.f;
#pragma unroll 2
        for (int j = 0; j < W / 4; ++j) {
            // The group's eight operand vectors are read before its products.
            float4 gv[4], ev[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                gv[r] = *reinterpret_cast<const float4*>(gs + (tt + 16 * r) * W + 4 * row_slot(tt, j));
#pragma unroll
            for (int k = 0; k < 4; ++k)
                ev[k] = *reinterpret_cast<const float4*>(Et + (4 * j + k) * kEtPitch + 4 * cc);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float ec[4] = {ev[k].x, ev[k].y, ev[k].z, ev[k].w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float gk = k == 0 ? gv[r].x : k == 1 ? gv[r].y : k == 2 ? gv[r].z : gv[r].w;
#pragma unroll
                    for (int c = 0; c < 4; ++c) mo[r][c] = fmaf(gk, ec[c], mo[r][c]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
            buf_store4<TIn>(dr, ((r0 + tt + 16 * r) * W + 4 * cc) * int(es),
                            make_float4(mo[r][0], mo[r][1], mo[r][2], mo[r][3]));
    }

    // dE = half 0 + half 1 into the tile's record (B part; A part unused).
    float* rp = records + (n * chunks + ci) * rec;
    __syncthreads();
    if (half == 1) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
            store4(part + (8 * a8 + r) * W + 4 * b4, make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]));
    }
    __syncthreads();
    if (half == 0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const float4 o = *reinterpret_cast<const float4*>(part + (8 * a8 + r) * W + 4 * b4);
            store4(rp + (8 * a8 + r) * W + 4 * b4,
                   make_float4(acc[r][0] + o.x, acc[r][1] + o.y, acc[r][2] + o.z, acc[r][3] + o.w));
        }
    }
}

// Key side: one workgroup per (tile, stream).  LDS: dB [s][c] with the
// 16-byte slot j of row s at j ^ ((s / 4) & 15) (the dK reads take rows
// 4 cc .. + 3 for 16 cc at once, the dV reads whole rows: both spread over
// the banks), dA [64], the stage's K and V rows (swizzled).  dB and dA come
// from `parts` dE records (summed in order) and the state with the
// arithmetic of bwd_finalize_kernel, or, with `ready`, from dB ([N][64][64])
// and dA ([N][64]) formed by it.
template <typename TIn>
__global__ __launch_bounds__(kThreads, kGradBlocks) void key_grad64_kernel(
    const TIn* __restrict__ k, const TIn* __restrict__ v, TIn* __restrict__ dk,
    TIn* __restrict__ dv, const float* __restrict__ dE_records, int parts, int64_t rec,
    const float* __restrict__ state, const float* __restrict__ dB_ready,
    const float* __restrict__ dA_ready, int64_t T, int chunk) {
    constexpr int W = 64, ST = kGradStage;
    extern __shared__ float smem[];
    float* dBs = smem;           // [64][64], swizzled
    float* dAs = dBs + W * W;    // [64]
    float* ks = dAs + W;         // [ST][64], swizzled
    float* vs = ks + ST * W;     // [ST][64], swizzled
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.y;
    const int64_t t_begin = int64_t(blockIdx.x) * chunk;
    const int rows = int(min(T, t_begin + chunk) - t_begin);
    const int64_t es = sizeof(TIn);
    const auto kr = mfma::make_rsrc(k + (n * T + t_begin) * W, int64_t(rows) * W * es);
    const auto vr = mfma::make_rsrc(v + (n * T + t_begin) * W, int64_t(rows) * W * es);
    const auto dkr = mfma::make_rsrc(dk + (n * T + t_begin) * W, int64_t(rows) * W * es);
    const auto dvr = mfma::make_rsrc(dv + (n * T + t_begin) * W, int64_t(rows) * W * es);
    auto db_at = [](int s, int c) { return s * W + 4 * ((c >> 2) ^ ((s >> 2) & 15)) + (c & 3); };

    GradStage<TIn> st;
    st.fetch(kr, vr, 0);
    {
        // Lane c of wave w forms rows s = w + 4 m.
        const int c = tid & 63, s0 = tid >> 6;
        if (dB_ready) {
            const float* bn = dB_ready + n * W * W;
            float b[16], a[16];
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                b[m] = bn[(s0 + 4 * m) * W + c];
                a[m] = dA_ready[n * W + s0 + 4 * m];
            }
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                dBs[db_at(s0 + 4 * m, c)] = b[m];
                if (c == 0) dAs[s0 + 4 * m] = a[m];
            }
        } else {
            const float* sn = state + n * (W * W + W);
            const float* rn = dE_records + n * int64_t(parts) * rec;
            // RACE_KEY_GRAD_ROWS rows at a time: every part, B and A value
            // requested before the sums.
#pragma unroll
            for (int mb = 0; mb < 16; mb += kKeyGradRows) {
                float gp[kFoldParts][kKeyGradRows], b[kKeyGradRows], a[kKeyGradRows];
#pragma unroll
                for (int m = 0; m < kKeyGradRows; ++m) {
                    const int s = s0 + 4 * (mb + m);
#pragma unroll
                    for (int p = 0; p < kFoldParts; ++p)
                        gp[p][m] = rn[int64_t(min(p, parts - 1)) * rec + s * W + c];
                    b[m] = sn[s * W + c];
                    a[m] = sn[W * W + s];
                }
#pragma unroll
                for (int m = 0; m < kKeyGradRows; ++m) {
                    const int s = s0 + 4 * (mb + m);
                    float gs = 0.f;
#pragma unroll
                    for (int p = 0; p < kFoldParts; ++p)
                        if (p < parts) gs += gp[p][m];
                    const float den = a[m] + kEps;
                    const float e = b[m] / den;
                    dBs[db_at(s, c)] = gs / den;
                    float dsum = fmaf(0.f, 0.f, gs * e);
#pragma unroll
                    for (int off = 32; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off);
                    if (c == 0) dAs[s] = -dsum / den;
                }
            }
        }
    }

    // Waves 0-1 form dK and waves 2-3 dV, each thread an 8 x 4 register tile:
    // tokens tt + 8 r (r < 8) and columns 4 cc .. 4 cc + 3, the contraction in
    // order (so the gradients are those of one thread per 4 x 4 tile doing
    // both maps).  Per 128 FMAs a thread reads 4 dB vectors (one per lane
    // and instruction) and 8 token vectors (4 rows per wave: broadcast), half
    // the dB traffic of 4 x 4 tiles, which held the passes at the LDS rate.
    const int half = __builtin_amdgcn_readfirstlane(tid >> 7);
    const int tt = (tid & 127) >> 4, cc = tid & 15;
    for (int r0 = 0; r0 < rows; r0 += ST) {
        __syncthreads();
        st.template stash<true>(ks, vs);
        __syncthreads();
        if (r0 + ST < rows) st.fetch(kr, vr, r0 + ST);
        float o[8][4];
        if (half == 0) {
            // dK[t][4 cc + i] = dA + sum_c V[t][c] dB[4 cc + i][c].
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float bias = dAs[4 * cc + i];
#pragma unroll
                for (int r = 0; r < 8; ++r) o[r][i] = bias;
            }
#pragma unroll 2
            for (int j = 0; j < W / 4; ++j) {
                float4 xv[8], bv[4];
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    xv[r] = *reinterpret_cast<const float4*>(vs + (tt + 8 * r) * W + 4 * row_slot(tt, j));
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    bv[i] = *reinterpret_cast<const float4*>(dBs + (4 * cc + i) * W + 4 * (j ^ cc));
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const float x = kk == 0 ? xv[r].x : kk == 1 ? xv[r].y : kk == 2 ? xv[r].z : xv[r].w;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float b = kk == 0 ? bv[i].x : kk == 1 ? bv[i].y : kk == 2 ? bv[i].z : bv[i].w;
                            o[r][i] = fmaf(x, b, o[r][i]);
                        }
                    }
            }
#pragma unroll
            for (int r = 0; r < 8; ++r)
                buf_store4<TIn>(dkr, ((r0 + tt + 8 * r) * W + 4 * cc) * int(es),
                                make_float4(o[r][0], o[r][1], o[r][2], o[r][3]));
        } else {
            // dV[t][4 cc + c] = sum_s K[t][s] dB[s][4 cc + c].
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) o[r][c] = 0.f;
#pragma unroll 2
            for (int j = 0; j < W / 4; ++j) {
                float4 xv[8], bv[4];
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    xv[r] = *reinterpret_cast<const float4*>(ks + (tt + 8 * r) * W + 4 * row_slot(tt, j));
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    bv[kk] = *reinterpret_cast<const float4*>(dBs + (4 * j + kk) * W + 4 * (cc ^ j));
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const float bc[4] = {bv[kk].x, bv[kk].y, bv[kk].z, bv[kk].w};
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const float x = kk == 0 ? xv[r].x : kk == 1 ? xv[r].y : kk == 2 ? xv[r].z : xv[r].w;
#pragma unroll
                        for (int c = 0; c < 4; ++c) o[r][c] = fmaf(x, bc[c], o[r][c]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 8; ++r)
                buf_store4<TIn>(dvr, ((r0 + tt + 8 * r) * W + 4 * cc) * int(es),
                                make_float4(o[r][0], o[r][1], o[r][2], o[r][3]));
        }
    }
}

int pow2_at_least(int x) {
    int m = 1;
    while (m < x) m *= 2;
    return m;
}

}  // namespace

bool v4_widths(int Wa, int Wb) { return Wa % 4 == 0 && Wb % 4 == 0; }

hipError_t launch_outer_sums4(const void* x, const void* y, float* records, const Problem& p,
                              int Wa, int Wb, hipStream_t stream) {
    if (Wa == 64 && Wb == 64) {
        const dim3 grid64(unsigned(p.tiles), unsigned(p.N));
        // The double-buffered staging; the final partial sums reuse it.
        const size_t lds64 = size_t(2 * 2 * kRedTokens * 64) * sizeof(float);
        static_assert(64 * 64 + 4 * 64 <= 2 * 2 * kRedTokens * 64, "part fits the staging");
        if (p.dtype == RACE_BF16)
            outer64_kernel<bf16_t><<<grid64, kThreads, lds64, stream>>>(
                static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(y), records, p.T, p.tile,
                p.tiles, p.rec);
        else
            outer64_kernel<float><<<grid64, kThreads, lds64, stream>>>(
                static_cast<const float*>(x), static_cast<const float*>(y), records, p.T, p.tile,
                p.tiles, p.rec);
        return hipGetLastError();
    }
    const int nv = pow2_at_least((kRedTokens * (Wa + Wb) / 4 + kThreads - 1) / kThreads);
    const int nt = pow2_at_least((Wa / 4 * (Wb / 4) + kThreads - 1) / kThreads);
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    const size_t lds = size_t(2 * kRedTokens * (Wa + Wb)) * sizeof(float);
#define RACE_OS4(TIN, NV, NT)                                                                    \
    outer_sums4_kernel<TIN, NV, NT><<<grid, kThreads, lds, stream>>>(                            \
        static_cast<const TIN*>(x), static_cast<const TIN*>(y), records, p.T, p.tile, p.tiles, \
        p.rec, Wa, Wb)
#define RACE_OS4_NT(TIN, NV)                      \
    switch (nt) {                                 \
        case 1: RACE_OS4(TIN, NV, 1); break;      \
        case 2: RACE_OS4(TIN, NV, 2); break;      \
        case 4: RACE_OS4(TIN, NV, 4); break;      \
        case 8: RACE_OS4(TIN, NV, 8); break;      \
        default: return hipErrorInvalidValue;     \
    }
#define RACE_OS4_NV(TIN)                          \
    switch (nv) {                                 \
        case 1: RACE_OS4_NT(TIN, 1) break;        \
        case 2: RACE_OS4_NT(TIN, 2) break;        \
        case 4: RACE_OS4_NT(TIN, 4) break;        \
        case 8: RACE_OS4_NT(TIN, 8) break;        \
        case 16: RACE_OS4_NT(TIN, 16) break;      \
        default: return hipErrorInvalidValue;     \
    }
    if (p.dtype == RACE_BF16) {
        RACE_OS4_NV(bf16_t)
    } else {
        RACE_OS4_NV(float)
    }
#undef RACE_OS4_NV
#undef RACE_OS4_NT
#undef RACE_OS4
    return hipGetLastError();
}

size_t query_grad64_lds_bytes() {
    return size_t(64 * kEtPitch + 2 * kGradStage * 64) * sizeof(float);
}
size_t key_grad64_lds_bytes() { return size_t(64 * 64 + 64 + 2 * kGradStage * 64) * sizeof(float); }

hipError_t launch_query_grad64(const void* q, const void* g, void* dq, const float* state,
                               float* records, const Problem& p, hipStream_t stream) {
    if (p.S != 64 || p.d != 64) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    const size_t lds = query_grad64_lds_bytes();
    if (p.dtype == RACE_BF16)
        query_grad64_kernel<bf16_t><<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(g), static_cast<bf16_t*>(dq),
            state, records, p.T, p.tile, p.tiles, p.rec);
    else
        query_grad64_kernel<float><<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(q), static_cast<const float*>(g), static_cast<float*>(dq),
            state, records, p.T, p.tile, p.tiles, p.rec);
    return hipGetLastError();
}

hipError_t launch_key_grad64(const void* k, const void* v, void* dk, void* dv,
                             const float* dE_records, const float* state, const float* dB_ready,
                             const float* dA_ready, const Problem& p, hipStream_t stream) {
    if (p.S != 64 || p.d != 64) return hipErrorInvalidValue;
    if (!dB_ready && (p.tiles > kKeyGradFoldParts || !dE_records || !state)) return hipErrorInvalidValue;
    const dim3 grid(unsigned(p.tiles), unsigned(p.N));
    const size_t lds = key_grad64_lds_bytes();
    const int parts = int(p.tiles);
    if (p.dtype == RACE_BF16)
        key_grad64_kernel<bf16_t><<<grid, kThreads, lds, stream>>>(
            static_cast<const bf16_t*>(k), static_cast<const bf16_t*>(v), static_cast<bf16_t*>(dk),
            static_cast<bf16_t*>(dv), dE_records, parts, p.rec, state, dB_ready, dA_ready, p.T, p.tile);
    else
        key_grad64_kernel<float><<<grid, kThreads, lds, stream>>>(
            static_cast<const float*>(k), static_cast<const float*>(v), static_cast<float*>(dk),
            static_cast<float*>(dv), dE_records, parts, p.rec, state, dB_ready, dA_ready, p.T, p.tile);
    return hipGetLastError();
}

size_t map4_lds_bytes(int Wa) {
    if (Wa == 64) return size_t(Wa * kSliceCols + Wa * (kMap64Tokens + 4)) * sizeof(float);
    return size_t(Wa * kSliceCols + Wa * (kMapTokens4 + 4)) * sizeof(float);
}

hipError_t launch_map4(const void* x, void* out, const MapOperand& op, const Problem& p, int Wa,
                       int Wb, hipStream_t stream) {
    if (Wa == 64) {
        const int64_t per_wg64 = int64_t(kMap64Blocks) * kMap64Tokens;
        const dim3 grid64(unsigned((p.T + per_wg64 - 1) / per_wg64), unsigned(p.N),
                          unsigned((Wb + kSliceCols - 1) / kSliceCols));
        const size_t lds64 = map4_lds_bytes(64);
        if (p.dtype == RACE_BF16)
            map64_kernel<bf16_t><<<grid64, kThreads, lds64, stream>>>(
                static_cast<const bf16_t*>(x), static_cast<bf16_t*>(out), op, p.T, Wb);
        else
            map64_kernel<float><<<grid64, kThreads, lds64, stream>>>(
                static_cast<const float*>(x), static_cast<float*>(out), op, p.T, Wb);
        return hipGetLastError();
    }
    const int64_t per_wg = int64_t(kMapBlocks) * kMapTokens4;
    const dim3 grid(unsigned((p.T + per_wg - 1) / per_wg), unsigned(p.N),
                    unsigned((Wb + kSliceCols - 1) / kSliceCols));
    const size_t lds = map4_lds_bytes(Wa);
    const int nv = pow2_at_least((kMapTokens4 * (Wa / 4) + kThreads - 1) / kThreads);
#define RACE_MAP4(TIN, NV)                                                                     \
    map4_kernel<TIN, NV><<<grid, kThreads, lds, stream>>>(                                     \
        static_cast<const TIN*>(x), static_cast<TIN*>(out), op, p.T, Wa, Wb)
#define RACE_MAP4_NV(TIN)                      \
    switch (nv) {                              \
        case 1: RACE_MAP4(TIN, 1); break;      \
        case 2: RACE_MAP4(TIN, 2); break;      \
        case 4: RACE_MAP4(TIN, 4); break;      \
        case 8: RACE_MAP4(TIN, 8); break;      \
        case 16: RACE_MAP4(TIN, 16); break;    \
        default: return hipErrorInvalidValue;  \
    }
    if (p.dtype == RACE_BF16) {
        RACE_MAP4_NV(bf16_t)
    } else {
        RACE_MAP4_NV(float)
    }
#undef RACE_MAP4_NV
#undef RACE_MAP4
    return hipGetLastError();
}

}  // namespace race
