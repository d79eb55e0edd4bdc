// race_internal.h -- shared device helpers and launcher declarations of the
// MI355X RACE attention library.  Not part of the ABI (include/race_mi355x.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "race_mi355x.h"

namespace race {

// Denominator offset of the per-bucket normalization (src/race_baseline.py:47).
constexpr float kEps = 1e-6f;
constexpr int kThreads = 256;   // every kernel runs 4 wave64s per workgroup
constexpr int kSliceCols = 64;  // V/out columns per workgroup in the VALU kernels

// bf16 is carried as its bit pattern.
using bf16_t = uint16_t;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(uint32_t(x) << 16); }

// Round-to-nearest-even fp32 -> bf16 (IEEE rounding of the top 16 bits);
// NaN stays NaN (quiet bit set).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return bf16_t(u >> 16);
}

__device__ __forceinline__ void store_val(float* p, float x) { *p = x; }
__device__ __forceinline__ void store_val(bf16_t* p, float x) { *p = f32_to_bf16(x); }

// Floats in one tile record: B [S][d] then A [S], padded to 64 floats so every
// record starts 256-byte aligned.
inline int64_t record_floats(int64_t S, int64_t d) { return ((S * d + S + 63) / 64) * 64; }

// LDS per workgroup on gfx950 (MI355X), the one target of this library.
constexpr int kGfx950LdsBytes = 160 * 1024;
inline int64_t state_floats(int64_t S, int64_t d) { return S * d + S; }

// Problem description handed from the API layer to the launchers (all sizes
// validated by the API layer before any launch).
struct Problem {
    int64_t N, T;
    int S, d;
    int dtype;       // race_dtype
    int kernel;      // race_kernel as requested
    int tile;        // tokens per tile (multiple of RACE_SUB_CHUNK_TOKENS)
    int64_t tiles;   // ceil(T / tile)
    int64_t rec;     // record_floats(S, d)
    bool single = false;  // the one-read causal forward (single_pass.hip) runs
    // Causal forward continued from a carried state ([N][S*d+S], B then A):
    // the scan starts every stream from it instead of zero.  Null otherwise.
    const float* init = nullptr;
};

// Optional hipEventRecord after each launch (race_fwd_profiled).
struct Marks {
    hipEvent_t* events = nullptr;
    int max = 0;
    int n = 0;
    hipError_t mark(hipStream_t stream) {
        if (!events) return hipSuccess;
        if (n >= max) return hipErrorInvalidValue;
        return hipEventRecord(events[n++], stream);
    }
};

// ---- VALU kernels (valu_kernels.hip): any supported shape, fp32 math ----

// Per (stream, tile) sums: rec[a*Wb + c] = sum_t x[t][a] * y[t][c] and
// rec[Wa*Wb + a] = sum_t x[t][a], over the tokens of the tile.
hipError_t launch_tile_outer_sums(const void* x, const void* y, float* records, const Problem& p,
                                  int Wa, int Wb, hipStream_t stream);
// In-place exclusive scan of the records over tiles (fixed tile order),
// starting from p.init when it is not null; the inclusive total goes to state
// ([N][S*d+S]) when it is not null (state may be p.init).  With `reverse` the
// scan runs from the last tile to the first.
hipError_t launch_tile_scan(float* records, float* state, const Problem& p, hipStream_t stream,
                            bool reverse = false);
// Totals over tiles into `state` ([N][S*d+S]) when not null, and E = B /
// (A + eps) into `E` ([N][S][d]).
hipError_t launch_tile_reduce(const float* records, float* state, float* E, const Problem& p,
                              hipStream_t stream);
// Causal output pass from the scanned records.
hipError_t launch_causal_output_valu(const void* q, const void* k, const void* v, void* out,
                                     const float* records, const Problem& p, hipStream_t stream);
// The matrix of a token map for stream n:
//     M[a][c] = m[n * stream + a * row + c * col]
// divided by (div[n * div_stream + (div_by_col ? c : a)] + eps) when div is
// given (E = B / (A + eps) read straight from a state), and bias[n *
// bias_stream + c] added to every output row when bias is given.  With
// parts > 1 every read of m and div is the sum, in order, of `parts` values
// part_stride apart (per-tile records summed on the fly).  When save is
// given, the workgroups of the first token block also write the (summed,
// undivided) values to save[n * save_stream + a * row + c * col] and the
// divisors to save[n * save_stream + save_div_off + (div_by_col ? c : a)].
struct MapOperand {
    const float* m = nullptr;
    int64_t stream = 0, row = 0, col = 0;
    int parts = 1;
    int64_t part_stride = 0;
    const float* div = nullptr;
    int64_t div_stream = 0;
    bool div_by_col = false;
    const float* bias = nullptr;
    int64_t bias_stream = 0;
    float* save = nullptr;
    int64_t save_stream = 0, save_div_off = 0;
};
// out[n][t][c] = sum_a x[n][t][a] * M[a][c] (+ bias[c]) for the operand's M.
hipError_t launch_token_map(const void* x, void* out, const MapOperand& op, const Problem& p,
                            int Wa, int Wb, hipStream_t stream);
// The causal op continued from init ([N][S*d+S]) token by token in one
// launch (decode.hip); the advanced state goes to `state`, which may be init.
hipError_t launch_decode(const void* q, const void* k, const void* v, void* out,
                         const float* init, float* state, const Problem& p, hipStream_t stream);
// Dynamic LDS of the VALU output pass and map kernels.
size_t causal_output_valu_lds_bytes(int S);
size_t token_map_lds_bytes(int Wa);
// Backward finalize: dE = the sum of the tile records of Q^T dOut ([N][tiles]
// [rec], fixed order), E = B / (A + eps) from the forward state ([N][S*d+S]);
// dB = dE / (A + eps) into dB ([N][S][d]), dA into dA ([N][S]).
hipError_t launch_bwd_finalize(const float* dE_records, const float* state, float* dB, float* dA,
                               const Problem& p, hipStream_t stream);

// ---- MFMA kernels: mfma_direct.hip (one wave per tile, operands straight
// from global memory into registers) and mfma_causal.hip (workgroup-
// cooperative tiles staged through LDS, every supported shape) ----

// Register-direct per-tile totals: (S, d) in {(64, 64), (64, 128), (128, 64)}.
bool direct_sums_supported(int S, int d);
hipError_t launch_tile_sums_direct(const void* k, const void* v, float* records, const Problem& p,
                                   hipStream_t stream);
// Register-direct causal output pass: S = d = 64, bf16.
bool direct_output_supported(int S, int d, int dtype);
// Tiles per compute unit the direct output pass wants resident (one wave64 per SIMD).
int direct_output_tiles_per_cu();
// Tiles per compute unit the MFMA causal path of this problem wants.
int mfma_tiles_per_cu(int S, int d, int dtype, int kernel);
hipError_t launch_causal_output_direct(const void* q, const void* k, const void* v, void* out,
                                       const float* records, const Problem& p, hipStream_t stream);

// ---- non-causal reductions and maps for widths that are multiples of 4
// (noncausal_v4.hip); the kernels above take every other width ----
bool v4_widths(int Wa, int Wb);
// Same records as launch_tile_outer_sums (per tile of p.tile tokens).
hipError_t launch_outer_sums4(const void* x, const void* y, float* records, const Problem& p,
                              int Wa, int Wb, hipStream_t stream);
// Same result as launch_token_map.
hipError_t launch_map4(const void* x, void* out, const MapOperand& op, const Problem& p, int Wa,
                       int Wb, hipStream_t stream);
size_t map4_lds_bytes(int Wa);
// The backward at S = d = 64 as a query-side pass (dQ, and the dE tile
// records into `records`, one per tile of p.tile tokens) and a key-side pass
// (dK, dV).  The key side forms dB and dA from the dE records and the state
// itself for at most kKeyGradFoldParts tiles per stream (dB_ready null), or
// reads them from dB_ready ([N][64][64]) and dA_ready ([N][64]).
constexpr int kKeyGradFoldParts = 4;
hipError_t launch_query_grad64(const void* q, const void* g, void* dq, const float* state,
                               float* records, const Problem& p, hipStream_t stream);
hipError_t launch_key_grad64(const void* k, const void* v, void* dk, void* dv,
                             const float* dE_records, const float* state, const float* dB_ready,
                             const float* dA_ready, const Problem& p, hipStream_t stream);

// ---- causal backward (causal_bwd.hip): fp32 vector-ALU kernels ----

// Sub-chunk length (32 or 16) of the causal backward kernels for (S, d) under
// `lds_limit_bytes` of LDS per workgroup, or 0 if the state does not fit.
int causal_bwd_chunk(int S, int d, int lds_limit_bytes);
// One column group of the vector-ALU causal backward walks (every term is
// linear in the value columns).  The launches then take p.d = the group's
// width, V, dOut and dV already offset to column c0, and these:
struct BwdCols {
    int64_t ld = 0;        // row stride, in elements, of V, dOut and dV (the full d)
    int c0 = 0;            // first column of the group
    int fwd_d = 0;         // row length of B0 in the forward prefix records (the full d)
    int64_t fwd_rec = 0;   // stride of those records (record_floats(S, full d))
    // fp32 running sums of dQ and dK over the groups, read before this group
    // adds to them (null for the first) and written after (null to skip).
    const float* acc_q_in = nullptr;
    float* acc_q_out = nullptr;
    const float* acc_k_in = nullptr;
    float* acc_k_out = nullptr;
};
// The single group: every column at once.
inline BwdCols all_columns(const Problem& p) {
    BwdCols c;
    c.ld = p.d;
    c.fwd_d = p.d;
    c.fwd_rec = p.rec;
    return c;
}
// Forward walk: dQ (nullable, caller dtype; the running sum over the groups
// when one is kept), dq32 [N][T][S] fp32 (this group's dQ), apre
// [N][tiles][tile / C][S] (running mass at every sub-chunk start) and the
// per-tile suffix totals (Z [S][d], Y [S]) into bwd_records, from the
// forward's scanned prefix records.
hipError_t launch_causal_bwd_dq(const void* q, const void* k, const void* v, const void* g,
                                void* dQ, float* dq32, float* apre, const float* fwd_records,
                                float* bwd_records, const Problem& p, int C, const BwdCols& cols,
                                hipStream_t stream);
// Backward walk from the suffix state at every tile end: dK, dV (each
// nullable; dK the running sum over the groups when one is kept).
hipError_t launch_causal_bwd_dkv(const void* q, const void* k, const void* v, const void* g,
                                 const float* dq32, const float* apre,
                                 const float* suffix_records, void* dK, void* dV, const Problem& p,
                                 int C, const BwdCols& cols, hipStream_t stream);

// Matrix-core kernels of the causal backward (mfma_bwd.hip): 64 x 64 blocks
// (S = d = 64, or one block of S and d multiples of 64: bucket group m, value
// group h), 32-token sub-chunks, the same buffers as the vector-ALU kernels.
// With fp32 tokens the dQ kernel writes dQ only through dq32 (dQ must be null).
struct BwdBlock {
    int ldq = 64;          // row stride of probsQ, probsK, dQ and dK (the full S)
    int ldv = 64;          // row stride of V, dOut and dV (the full d)
    int s0 = 0, c0 = 0;    // the block's first bucket and value column
    int fwd_d = 64;        // row length of B in the forward records (the full d)
    int64_t fwd_a = 4096;  // offset of A in a forward record (full S * full d)
    int64_t fwd_rec = 0;   // stride of the forward records
    // Several blocks (blocked = 1): fp32 running sums of dQ, dK (rows of ldq)
    // and dV (rows of ldv), at the block's first column, to which the kernels
    // add the block's part (the first addend writes them; a null sum is a
    // gradient not asked for); with fin_* set, the last addend goes to the
    // caller's gradient (dtype, same strides) instead.  One block (blocked =
    // 0): the gradients are written as they are.
    int blocked = 0;
    float* acc_q = nullptr;
    float* acc_k = nullptr;
    float* acc_v = nullptr;
    void* fin_q = nullptr;
    void* fin_k = nullptr;
    void* fin_v = nullptr;
    int q_first = 1, k_first = 1, v_first = 1;
    int alpha = 1;  // B3: the terms of alpha = -W dQ (and Y) belong to this block
};
// Shapes the blocks cover: S in {64, 128, 256}, d in {64, 128}.
bool causal_bwd_mfma_supported(int S, int d);
// The single block of an S = d = 64 problem.
BwdBlock single_block(const Problem& p);
// p is the block's problem (S = d = 64 and its record size); q, k, v, g point
// at the block's first column; dq32, apre and bwd_records are the block's own
// (rows of 64).  dv = 128 (bf16 blocks only): one walk over both value groups
// of a d = 128 problem, the bucket group's whole dQ at once, with the suffix
// records of value group h at bwd_records + h * N * tiles * rec (Y, the
// totals of alpha, in group 0's records and zero in group 1's).
hipError_t launch_causal_bwd_dq_mfma(const void* q, const void* k, const void* v, const void* g,
                                     void* dQ, float* dq32, float* apre, const float* fwd_records,
                                     float* bwd_records, const Problem& p, const BwdBlock& blk,
                                     hipStream_t stream, int dv = 64);
// dK and dV: the caller's gradients (one block, rows of 64), or through the
// block's running sums.  With blk.alpha = 0 the block leaves out the terms
// of alpha = -W dQ (dQ is not read): a walk over both value groups put
// them, for the whole dQ, into value group 0's block.
hipError_t launch_causal_bwd_dkv_mfma(const void* q, const void* k, const void* v, const void* g,
                                      const float* dq32, const float* apre,
                                      const float* suffix_records, void* dK, void* dV,
                                      const Problem& p, const BwdBlock& blk, hipStream_t stream);
// How one forward-walk launch covers `pairs` consecutive 128-bucket blocks:
// block b's outputs lie b times these strides (in elements of each buffer)
// past the pointers the launch is given.
struct DqWidePairs {
    int pairs = 1;
    int64_t hi_ps = 0;   // dq_hi (bf16)
    int64_t lo_ps = 0;   // dq_lo (bf16)
    int64_t ap_ps = 0;   // apre (floats)
    int64_t rec_ps = 0;  // bwd_records (floats)
    // 1: a workgroup walks every tile of its stream in order from a zero
    // prefix (items are streams; fwd_records is not read); 0: one tile,
    // from its forward record.
    int whole = 0;
};
// Workgroups per launch-order group of the block walks: gfx950 hands
// consecutive workgroups of a launch to its eight XCDs in turn, so
// workgroups kWideXcds apart run on the same XCD.
constexpr int kWideXcds = 8;
// Workgroup x of a forward-walk launch over `pairs` blocks walks item
// (stream n, tile ti: item = n tiles + ti; or stream n) of block `block`: groups of
// kWideXcds items, each listed once per block, so the workgroups of one
// item (the same V and dOut rows) are kWideXcds apart.  item is -1 for the
// padding past the last item.
struct WideItem {
    int64_t item;
    int block;
};
__host__ __device__ inline WideItem wide_item(int64_t x, int pairs, int64_t items) {
    const int64_t per = int64_t(kWideXcds) * pairs;
    const int64_t grp = x / per, in = x % per;
    const int64_t item = grp * kWideXcds + in % kWideXcds;
    return {item < items ? item : -1, int(in / kWideXcds)};
}
// The forward walk (B1) over 128-bucket x 128-column blocks (bf16 tokens,
// d = 128; block b holds buckets s0 + 128 b .. s0 + 128 b + 127, with q and k
// pointing at bucket s0 of the full tensors and fwd_records the full
// problem's): dQ of those buckets whole as bf16 (dq_hi, rows of ld_hi: the
// caller's dQ at bucket s0, or workspace) with the bf16 rounding of each
// remainder (dq_lo, rows of 128; null when no backward walk follows), which
// the backward walk reads back as hi + lo; the running mass
// [N][tiles][tile / 32][128]; the suffix records of the block's four 64 x 64
// parts, (group g2, value half h) at bwd_records + (2 g2 + h) N tiles rec.
// Block b's outputs are offset by b times pp's strides.
hipError_t launch_causal_bwd_dq_wide(const void* q, const void* k, const void* v, const void* g, void* dq_hi,
                                     int ld_hi, void* dq_lo, float* apre, const float* fwd_records,
                                     float* bwd_records, const Problem& p, int s0, const DqWidePairs& pp,
                                     hipStream_t stream);
// The backward walk over the same block: the buffers its forward walk wrote
// and dV's accumulation.
struct BwdWide {
    int ldq = 0;                 // row stride of probsQ, probsK, dK (the full S)
    const void* dq_hi = nullptr; // dQ of the block as bf16, rows of ld_hi
    int ld_hi = 0;
    const void* dq_lo = nullptr; // the bf16 remainders, rows of 128
    const float* apre = nullptr; // running mass per sub-chunk, rows of 128
    const float* rec[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};  // scanned suffix records (g2, value half)
    float* acc_v = nullptr;  // dV's fp32 running sum (rows of 128), or null
    void* fin_v = nullptr;   // the caller's dV (bf16) for the last addend, or null
    int v_first = 1;         // the first addend writes acc_v without reading it
};
// dK of the block's buckets whole (q, k and dK point at its first bucket) and
// its part of dV; p is the whole problem.
hipError_t launch_causal_bwd_dkv_wide(const void* q, const void* k, const void* v, const void* g, void* dK,
                                      const Problem& p, const BwdWide& wb, hipStream_t stream);
// The forward's tile sums (K1) on the matrix cores for the shapes
// mfma_causal_supported takes, into records of p.rec floats.
hipError_t launch_tile_sums_mfma(const void* k, const void* v, float* records, const Problem& p,
                                 hipStream_t stream);

// ---- bucket-probability front end (hashing.hip) ----
bool hash_shape_ok(int64_t rows, int dk, int L, int K);
size_t hash_lds_bytes(int dk, int L, int K);
hipError_t launch_hash_probs(const void* x, const float* planes_T, void* probs, int64_t rows,
                            int dk, int L, int K, int dtype, hipStream_t stream);
// dx of the hashing for the upstream gradient dprobs (same limits).
hipError_t launch_hash_probs_bwd(const void* x, const float* planes_T, const void* dprobs, void* dx,
                                int64_t rows, int dk, int L, int K, int dtype, hipStream_t stream);

// ---- Algorithm 1 with the hashing inside (alg1.hip): bf16 q, k, v, out ----
struct Alg1Args {
    const void* q;
    const void* k;
    const void* v;
    const float* W;     // [L][P][D] fp32
    const float* beta;  // one fp32 value in device memory
    void* out;
    float* records;     // [N][tiles][rec]
    float* state;       // nullable: [N][S*D + S]
    int L, P;
};
// D in {64, 128}, P in 1..5, L in 1..4.
bool alg1_shape_ok(int D, int P, int L);
// Dynamic LDS of the output pass (0 if unsupported); variant 0 = hi/lo
// features, 1 = bf16 features.
size_t alg1_output_lds_bytes(int D, int P, int L, int variant);
// Output-pass workgroups resident per compute unit.
int alg1_blocks_per_cu(int D, int P, int L, int variant);
// Tile sums, scan (final state into a.state when not null) and output pass.
hipError_t launch_alg1(const Alg1Args& a, const Problem& p, int variant, hipStream_t stream,
                       Marks* marks);

// ---- the causal op with the hashing inside (hashed_causal.hip) ----
struct HashedArgs {
    const void* q;        // query rows [N][T][d] (p.dtype)
    const void* k;        // key rows [N][T][d]
    const void* v;        // values [N][T][d]
    const float* planes;  // hash planes [L*K][d] fp32, row j = l*K + k
    void* out;
    float* records;       // [N][tiles][rec]
    float* state;         // nullable: [N][S*d + S]
    int L, K;             // tables, planes per table (R = 2^K, S = L*R)
};
// K >= 2, L*K <= 64, and an MFMA specialization for (L * 2^K, d).
bool hashed_causal_supported(int L, int K, int d);
// Tile sums, scan (final state into a.state when not null) and output pass.
hipError_t launch_hashed_causal(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks);

// Whether the MFMA causal path has a specialization for (S, d).
bool mfma_causal_supported(int S, int d);
hipError_t launch_causal_mfma(const void* q, const void* k, const void* v, void* out,
                              float* records, float* state, const Problem& p, hipStream_t stream,
                              Marks* marks);

// ---- One-read causal forward (single_pass.hip): S = d = 64 ----
// Tiles of kSinglePassTile tokens; the workspace holds the records, then one
// flag word per (stream, tile) (rounded up to 64 words), then the control
// words (per-XCD ticket counters and an error word).
constexpr int kSinglePassTile = 128;
constexpr int64_t kSinglePassCtlWords = 64;
inline int64_t single_pass_flag_words(int64_t N, int64_t tiles) { return ((N * tiles + 63) / 64) * 64; }
// Shape and device conditions of the path (`cus`: the device's CU count).
bool single_pass_supported(const Problem& p, int cus);
// Zeroes the flag and control words, then one persistent launch of `cus`
// workgroups.  `words` = records + N * tiles * rec.  The final state goes to
// `state` when not null; `init` seeds the running sums when not null.
hipError_t launch_causal_single(const void* q, const void* k, const void* v, void* out,
                                float* records, int* words, float* state, const float* init,
                                const Problem& p, int cus, hipStream_t stream, Marks* marks);
// Index in `words` of the error word: nonzero once a bounded wait gave up
// (the affected output tiles and `state` then hold NaN).
int64_t single_pass_error_word(int64_t N, int64_t tiles);
// Test hook: while on, every launch arms the error word as already set, so
// every bounded wait gives up at once and every workgroup exits normally.
void single_pass_preset_give_up(bool on);

}  // namespace race
