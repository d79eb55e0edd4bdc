/*
 * race_mi355x.h -- C ABI of the MI355X (gfx950) per-bucket RACE attention op.
 *
 * The op is race_fused_fwd(probsQ, probsK, V, causal): the hot span of the
 * reference's BatchedACE.forward (src/race_baseline.py:45-51), which takes the
 * bucket probabilities the hashing produced (src/race_baseline.py:43-44) and
 * returns, per stream n and token t,
 *
 *     causal:      out[t] = sum_s probsQ[t,s] * B_t[s,:] / (A_t[s] + 1e-6)
 *                  A_t = sum_{j<=t} probsK[j],  B_t = sum_{j<=t} probsK[j] (x) V[j]
 *     non-causal:  the same with A, B summed over all T tokens
 *                  (analysis/hot-path.md:157-162).
 *
 * plus the backward of both w.r.t. probsQ, probsK and V.  The name is the
 * one of the upstream host wrapper the reference describes as taking
 * "probsK/probsQ precomputed in fp32 ([N,T,S])" (src/race_fused_fwd.cu:9-13).
 *
 * Layouts (row-major, contiguous, 16-byte aligned base pointers):
 *   probsQ, probsK, dQ, dK : [N][T][S], S = L*R, table-major (s = l*R + r),
 *                            i.e. the reference's [N,T,L,R] viewed as [N,T,S]
 *   V, out, dOut, dV       : [N][T][d]
 *   state                  : [N][S*d + S] fp32: B[s][c] at s*d + c, then A[s]
 *                            at S*d + s (the per-bucket sums over all T tokens)
 * All token tensors of one call share one dtype (RACE_F32 or RACE_BF16);
 * accumulation is fp32.
 *
 * Contract, mirroring the reference's torch-free launcher API
 * (src/causal_v2/kernels/race_causal_fwd.h:40-49, :99-130):
 *   - the caller allocates outputs and the workspace; nothing here allocates
 *     device memory or synchronizes the host;
 *   - every launch goes on the caller's stream, in order;
 *   - a function returns the first error it hits: RACE_ERROR_INVALID_VALUE
 *     (numerically hipErrorInvalidValue) for unsupported shapes, bad pointers,
 *     a too-small workspace or an invalid tile length, else the hipError_t of
 *     the failed HIP call;
 *   - results are bitwise reproducible for a fixed shape, kernel and tile
 *     length: no atomics, every sum has a fixed order;
 *   - N == 0 or T == 0 is a successful no-op (the state, if given, is zeroed).
 * Limits: 1 <= S <= 256, 1 <= d <= 128, N*T*max(S,d) < 2^62.
 */
#ifndef RACE_MI355X_H
#define RACE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RACE_ABI_VERSION 1

typedef int32_t race_status;
#define RACE_SUCCESS 0
#define RACE_ERROR_INVALID_VALUE 1 /* equals hipErrorInvalidValue */
#define RACE_ERROR_SCRATCH_TOO_SMALL 2 /* race_fwd_noalloc only; equals hipErrorOutOfMemory */
/* race_fwd_single_status only: a bounded wait of the one-read kernel gave up
 * (outside the range of HIP's error codes, which other calls pass through). */
#define RACE_ERROR_SINGLE_PASS_GAVE_UP 4096

typedef enum race_dtype {
    RACE_F32 = 0,
    RACE_BF16 = 1
} race_dtype;

/* Which kernels run.  AUTO picks the MFMA kernels where a specialization
 * exists for (S, d) and the VALU kernels otherwise.  VALU forces the fp32
 * vector-ALU kernels (the reference-shaped path, any supported shape); MFMA
 * forces the matrix-core kernels and fails with RACE_ERROR_INVALID_VALUE if
 * the shape has none.  The MFMA path runs one wave per tile where a tile's
 * working set fits (S = d = 64) and workgroup-cooperative tiles otherwise;
 * MFMA_WG forces the workgroup-cooperative kernels.  Mirrors the reference
 * binding's tensor_cores flag (src/causal_v2/kernels/torch_binding.cpp:252-254). */
typedef enum race_kernel {
    RACE_KERNEL_AUTO = 0,
    RACE_KERNEL_VALU = 1,
    RACE_KERNEL_MFMA = 2,
    RACE_KERNEL_MFMA_WG = 3,
    RACE_KERNEL_DECODE = 4, /* race_fwd_carry only: the one-launch token-serial kernel */
    /* Causal forward, S = d = 64, fp32 or bf16, N = 8 or 16, on an MI355X
     * with all 256 CUs: one persistent launch that reads every operand once
     * (tiles of 128 tokens; tile_tokens must be 0 or 128).  Anything else
     * returns RACE_ERROR_INVALID_VALUE. */
    RACE_KERNEL_SINGLE = 5,
    /* Causal forward (race_fwd, race_fwd_noalloc, the tile path of
     * race_fwd_carry) on the workgroup matrix-core kernels with every
     * product fp32-accurate for bf16 tokens too: W, the masked scores and the
     * carried state enter the products as bf16 hi + lo pairs, as they do for
     * fp32 tokens, so a bf16 result differs from the exact one by about its
     * own rounding.  No counterpart in the reference's per-bucket path; its
     * bf16 tensor-core Algorithm-1 kernel likewise carries B and its scores
     * as hi + lo pairs (race_causal_fwd_tc.cu:23-40).  fp32 tokens: the same
     * as MFMA_WG.
     * Shapes without matrix-core kernels, the non-causal op, the backward,
     * the hashed and the Algorithm-1 entry points return
     * RACE_ERROR_INVALID_VALUE. */
    RACE_KERNEL_MFMA_PRECISE = 6
} race_kernel;

/* Shape of one call.  Mirrors CausalShape
 * (src/causal_v2/kernels/race_causal_fwd.h:60-66) with the hashing
 * parameters replaced by the bucket layout the op consumes. */
typedef struct race_shape {
    int64_t num_streams; /* N = batch * heads */
    int64_t seq_len;     /* T */
    int32_t num_tables;  /* L */
    int32_t num_buckets; /* R, buckets per table */
    int32_t head_dim;    /* d */
    int32_t dtype;       /* race_dtype of every token tensor */
} race_shape;

/* Optional knobs; pass NULL for the defaults.  tile_tokens: 0 picks the tile
 * length (tokens per workgroup of the causal output pass) automatically; a
 * positive value must be a multiple of RACE_SUB_CHUNK_TOKENS.  Mirrors the
 * reference's tile_tokens override (torch_binding.cpp:109-122). */
typedef struct race_options {
    int32_t tile_tokens;
    int32_t kernel; /* race_kernel */
} race_options;

/* Tile lengths are multiples of this many tokens. */
#define RACE_SUB_CHUNK_TOKENS 64

/* ABI version of the loaded library (RACE_ABI_VERSION it was built with). */
int32_t race_abi_version(void);

/* Static description of a status code. */
const char* race_status_string(race_status status);

/* Whether the shape is supported at all (limits above), and whether an MFMA
 * specialization exists for it.  Pure host logic, no device calls. */
race_status race_shape_supported(const race_shape* shape, int32_t* supported, int32_t* has_mfma);

/* The tile length a call with these arguments uses.  Automatic selection
 * reads the current device's compute-unit count. */
race_status race_select_tile_tokens(const race_shape* shape, int32_t causal,
                                    const race_options* opts, int32_t* tile_tokens);

/* Workspace of race_fwd in bytes for these arguments.  The causal workspace
 * starts with the tile records [N][tiles][rec] fp32, rec = S*d + S rounded
 * up to a multiple of 64 floats, B then A as in `state`; after race_fwd
 * returns (and the stream reaches it) record (n, t) holds the exclusive
 * prefix state at the first token of tile t of stream n.  *tiles and
 * *record_floats (nullable) receive the layout. */
race_status race_fwd_workspace_bytes(const race_shape* shape, int32_t causal,
                                     const race_options* opts, size_t* bytes, int64_t* tiles,
                                     int64_t* record_floats);

/* race_fused_fwd(probsQ, probsK, V, causal) -> out.
 * Replaces the reference's src/race_baseline.py:45-51 (causal) and the
 * non-causal formula of analysis/hot-path.md:157-162.  state (nullable): the
 * per-bucket totals over all T tokens (causal: the final scan state, the
 * decode hand-off; non-causal: what race_noncausal_bwd needs). */
race_status race_fwd(const void* probsQ, const void* probsK, const void* V, void* out,
                     float* state, const race_shape* shape, int32_t causal,
                     const race_options* opts, void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* race_fwd with a hipEventRecord on `stream` before the first launch and
 * after every launch: events[0] .. events[*n_events - 1], at most max_events
 * (an error if the call makes more launches than max_events - 1).  A
 * profiling aid for per-kernel timing on the caller's stream; it has no
 * counterpart in the reference. */
race_status race_fwd_profiled(const void* probsQ, const void* probsK, const void* V, void* out,
                              float* state, const race_shape* shape, int32_t causal,
                              const race_options* opts, void* workspace, size_t workspace_bytes,
                              hipStream_t stream, hipEvent_t* events, int32_t max_events,
                              int32_t* n_events);

/* Status of the last RACE_KERNEL_SINGLE forward whose workspace this is
 * (workspace NULL: the current GPU's race_fwd_noalloc scratch).  Waits for
 * `stream`, then reads the kernel's error word.  The one-read kernel's
 * workgroups wait on flags other workgroups set, each wait bounded; a wait
 * that gives up sets the word, the output rows of every tile whose prefix
 * never arrived are NaN and `state` is NaN, and every other output is valid.
 * Returns RACE_SUCCESS when no wait gave up, RACE_ERROR_SINGLE_PASS_GAVE_UP
 * when one did, RACE_ERROR_INVALID_VALUE when the arguments do not name a
 * RACE_KERNEL_SINGLE causal call or the workspace is too small.  The
 * reference's causal forward has no cross-workgroup wait; like its
 * launchers (src/causal_v2/kernels/race_causal_fwd.h:48-49) this reports the
 * first error. */
race_status race_fwd_single_status(const race_shape* shape, const race_options* opts,
                                   const void* workspace, size_t workspace_bytes,
                                   hipStream_t stream);

/* Test hook of the one-read kernel, no counterpart in the reference: while
 * `on` is nonzero, every RACE_KERNEL_SINGLE launch in this process arms its
 * error word as already set, so every bounded wait gives up at once and every
 * workgroup exits normally (all outputs and `state` NaN, and
 * race_fwd_single_status reports RACE_ERROR_SINGLE_PASS_GAVE_UP). */
race_status race_single_pass_test_give_up(int32_t on);

/* Bytes of the per-GPU scratch array race_fwd_noalloc takes its workspace
 * from.  32 MiB: at the automatic tile length on a 256-CU MI355X the cfg2
 * shape (N = 8, S = d = 64) needs 17 MB of tile records for any T up to
 * 2^21; race_fwd_workspace_bytes gives the need of any other call. */
#define RACE_NOALLOC_SCRATCH_BYTES (32u << 20)

/* race_fwd for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  It has
 * no counterpart in the reference.  The workspace comes from a device array
 * of RACE_NOALLOC_SCRATCH_BYTES that the library holds per GPU until the
 * process ends; the call itself allocates nothing.  A call whose
 * race_fwd_workspace_bytes exceeds that returns RACE_ERROR_SCRATCH_TOO_SMALL
 * before touching the device.  Outputs, their layouts and their values are
 * race_fwd's (the same kernels and tile length give the same bits).  All
 * calls on one GPU share its array: calls that overlap on one GPU (different
 * streams, or host threads without ordering) race and must be serialized by
 * the caller. */
race_status race_fwd_noalloc(const void* probsQ, const void* probsK, const void* V, void* out,
                             float* state, const race_shape* shape, int32_t causal,
                             const race_options* opts, hipStream_t stream);

/* Calls of race_fwd_carry with at most this many tokens (and an automatic
 * kernel and tile length) run the decode kernel. */
#define RACE_DECODE_TOKENS 16

/* Workspace of race_fwd_carry in bytes (0 when the call runs the decode
 * kernel; race_fwd's causal workspace otherwise). */
race_status race_fwd_carry_workspace_bytes(const race_shape* shape, const race_options* opts,
                                           size_t* bytes);

/* The causal race_fused_fwd continued from a carried state: the carry of the
 * reference's chunked forward (src/race_chunked.py:54-63, A_state and B_state
 * taken into the next chunk), fed by the hand-off state
 * (src/causal_v2/kernels/race_causal_fwd.h:20-21; race_fwd's `state`).  For
 * the T tokens of this call,
 *     out[t] = sum_s probsQ[t,s] * (B0 + B_t)[s,:] / (A0[s] + A_t[s] + 1e-6)
 * with (B0, A0) = init_state ([N][S*d + S] fp32, B then A, 16-byte aligned)
 * and A_t, B_t the inclusive sums over this call's tokens.  state (nullable)
 * receives init_state plus the sums over all T tokens and may equal
 * init_state (an in-place step).  Splitting a sequence anywhere and carrying
 * the state gives the unsplit result up to fp32 rounding.  Short calls
 * (decode: T <= RACE_DECODE_TOKENS) run one launch with one workgroup per
 * stream and no workspace; longer ones run race_fwd's causal kernels with the
 * tile scan started from init_state.  The reference has no kernel for this. */
race_status race_fwd_carry(const void* probsQ, const void* probsK, const void* V, void* out,
                           const float* init_state, float* state, const race_shape* shape,
                           const race_options* opts, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* race_fwd_carry with the events of race_fwd_profiled (a profiling aid, no
 * counterpart in the reference). */
race_status race_fwd_carry_profiled(const void* probsQ, const void* probsK, const void* V,
                                    void* out, const float* init_state, float* state,
                                    const race_shape* shape, const race_options* opts,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream,
                                    hipEvent_t* events, int32_t max_events, int32_t* n_events);

/* Workspace of race_noncausal_bwd in bytes. */
race_status race_noncausal_bwd_workspace_bytes(const race_shape* shape, const race_options* opts,
                                               size_t* bytes);

/* Gradients of the non-causal forward w.r.t. probsQ, probsK and V for the
 * upstream gradient dOut, given the forward's state (B, A).  There is no
 * reference kernel for this (the reference's backward differentiates a
 * different, globally normalized function through the hash chain,
 * src/noncausal/kernels/race_bwd.h:1-30); the math is the VJP of
 * analysis/hot-path.md:157-162:
 *   dQ = dOut E^T, dE = Q^T dOut, dB = dE / (A + eps),
 *   dA[s] = -sum_c dE[s,c] E[s,c] / (A[s] + eps), dK = V dB^T + 1 dA^T,
 *   dV = K dB, with E = B / (A + eps).
 * Any of dQ, dK, dV may be NULL to skip it. */
race_status race_noncausal_bwd(const void* probsQ, const void* probsK, const void* V,
                               const void* dOut, const float* state, void* dQ, void* dK, void* dV,
                               const race_shape* shape, const race_options* opts, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* Workspace of race_causal_bwd in bytes, O(1) per token: the forward prefix
 * records and the suffix records (of the walk's column group or block), the
 * running mass at every sub-chunk start and dQ as the walks hand it over
 * (an fp32 copy, or bf16 remainders); with bf16 tokens on the matrix cores
 * also fp32 running sums of the gradients summed over blocks.  The size
 * depends on the shape, dtype, tile length and kernel option (a host
 * computation, no device needed). */
race_status race_causal_bwd_workspace_bytes(const race_shape* shape, const race_options* opts,
                                            size_t* bytes);

/* Gradients of the causal forward w.r.t. probsQ, probsK and V for the
 * upstream gradient dOut.  The reference has no kernel for this: its design
 * outline (docs/causal_v2_design.md:689-742, for the globally normalized
 * function) walks prefix states forward and suffix states backward, which is
 * what this does for the per-bucket function of src/race_baseline.py:45-51.
 * With A_i, B_i the inclusive prefix sums, r_i = 1 / (A_i + eps), W_i = q_i r_i
 * and g = dOut:
 *   dq_i[s] = r_i[s] <B_i[s][:], g_i>,   alpha_i = -W_i dq_i (elementwise),
 *   Z_j = sum_{i>=j} W_i (x) g_i,  Y_j = sum_{i>=j} alpha_i,
 *   dk_j[s] = <Z_j[s][:], v_j> + Y_j[s],  dv_j[c] = sum_s k_j[s] Z_j[s][c].
 * The forward prefix states are recomputed (tile totals and their scan), so
 * only the forward's inputs are needed; the 128 x 128 block walks below skip
 * that and walk each stream whole from its first token when N times the
 * 128-bucket blocks covers the device's CUs or a stream is one tile (as does
 * race_causal_bwd_from_records, which then reads no records).  Any of dQ,
 * dK, dV may be NULL to skip it.  Kernels: with S and d multiples of 64 (S <= 256, d <= 128) and
 * tiles of whole 32-token sub-chunks, the matrix cores (64 x 64 bucket x
 * value blocks; bf16 tokens with d = 128 and S = 128 or 256 in walks over
 * 128 x 128 blocks); otherwise the vector ALU, in column groups where the
 * state does not fit one workgroup's LDS (RACE_KERNEL_VALU forces it).
 * RACE_KERNEL_MFMA on a shape without matrix-core kernels, a shape no kernel
 * takes, and the other kernel options return RACE_ERROR_INVALID_VALUE. */
race_status race_causal_bwd(const void* probsQ, const void* probsK, const void* V,
                            const void* dOut, void* dQ, void* dK, void* dV,
                            const race_shape* shape, const race_options* opts, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* Workspace of race_causal_bwd_from_records in bytes: race_causal_bwd's
 * without the forward records region (the caller supplies those).
 * opts->tile_tokens must be the forward's tile length (explicit, > 0). */
race_status race_causal_bwd_from_records_workspace_bytes(const race_shape* shape,
                                                         const race_options* opts, size_t* bytes);

/* race_causal_bwd from the forward's scanned tile records instead of
 * recomputing them: fwd_records is race_fwd's workspace after a causal call
 * with the same inputs and tile length ([N][tiles][rec], the exclusive prefix
 * state at each tile start), and opts->tile_tokens must be that tile length
 * (explicit, > 0).  The workspace is at least
 * race_causal_bwd_from_records_workspace_bytes for the same opts.  Keeping
 * the records costs 4 * rec / tile bytes per stream-token (rec = S*d + S
 * rounded up to 64 floats): 32.5 B at S = d = 64 and a tile of 512, about
 * 2 KB at S = 256, d = 128 and the minimum tile of 64.  The backward then
 * skips its own tile totals and scan.  No counterpart in the reference,
 * which has no causal backward kernel. */
race_status race_causal_bwd_from_records(const void* probsQ, const void* probsK, const void* V,
                                         const void* dOut, const float* fwd_records, void* dQ,
                                         void* dK, void* dV, const race_shape* shape,
                                         const race_options* opts, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream);

/* The bucket probabilities the op consumes, from the token rows: the hashing
 * of the reference's BatchedACE.forward (src/race_baseline.py:41-44).  For
 * each of `rows` rows x (head_dim values) and table l < num_tables, with
 * K = planes_per_table, R = 2^K and planes_T [head_dim][num_tables * K] fp32
 * (the reference's planes_T buffer, src/race_baseline.py:27):
 *   u_k = tanh(<x, planes_T[:, l K + k]>) / sqrt(head_dim),
 *   probs[row][l][r] = softmax_r(sum_k u_k s_{r,k}),
 * s_r the r-th of itertools.product([-1, 1], repeat=K) (s_{r,k} = +1 iff bit
 * K-1-k of r is set).  x and probs share `dtype`.  Limits: head_dim <= 128,
 * K <= 8, num_tables * K <= 64, num_tables * 2^K <= 256. */
race_status race_hash_probs(const void* x, const float* planes_T, void* probs, int64_t rows,
                            int32_t head_dim, int32_t num_tables, int32_t planes_per_table,
                            int32_t dtype, hipStream_t stream);

/* Gradient of race_hash_probs w.r.t. the rows: given dprobs (the upstream
 * gradient, [rows][num_tables * 2^K], dtype of x) writes dx [rows][head_dim].
 * With z_k = 2 u_k and sigma_k = sigma(z_k) (recomputed from x), per table
 *   du_k = 2 (sum_{r: s_{r,k} = +1} g_r - sigma_k sum_r g_r),  g_r = dprobs_r probs_r,
 *   dx   = sum_k du_k (1 - tanh^2(<x, p_k>)) / sqrt(head_dim) p_k.
 * The planes are a buffer in the reference (src/race_baseline.py:27), so no
 * gradient w.r.t. them.  The reference has no kernel for this; autograd
 * differentiates its torch composition (src/race_baseline.py:41-44).  Limits
 * as race_hash_probs. */
race_status race_hash_probs_bwd(const void* x, const float* planes_T, const void* dprobs, void* dx,
                                int64_t rows, int32_t head_dim, int32_t num_tables,
                                int32_t planes_per_table, int32_t dtype, hipStream_t stream);

/* ------------------------------------------------------------------------
 * The causal op with the hashing inside: BatchedACE.forward's hashing and hot
 * span (src/race_baseline.py:41-51) in one op, the reference's fused forward
 * race_fused_fwd(K, Q, V, planes, L) (src/race_fused_fwd.cu:150-171, kernel
 * :80-146).  Token rows k_rows, q_rows, v: [N][T][d] (shape->head_dim = d =
 * d_k), one dtype; planes: [L*K][d] fp32 row-major (the reference's
 * `planes`, = BatchedACE's planes_T transposed); shape->num_tables = L and
 * shape->num_buckets = R = 2^planes_per_table.  The result is race_fwd
 * (causal) on probsQ = hash(q_rows), probsK = hash(k_rows) as race_hash_probs
 * defines them, without those probabilities ever written to memory.  The
 * workspace, its tile records and `state` are race_fwd's.  Limits:
 * planes_per_table K >= 2, L*K <= 64, S = L*2^K in {64, 128, 256},
 * d in {64, 128}; the kernel option may be AUTO or MFMA_WG (the workgroup
 * matrix-core kernels run). */
race_status race_hashed_fwd_workspace_bytes(const race_shape* shape, int32_t planes_per_table,
                                            const race_options* opts, size_t* bytes, int64_t* tiles,
                                            int64_t* record_floats);
race_status race_hashed_fwd(const void* k_rows, const void* q_rows, const void* v, const float* planes,
                            void* out, float* state, const race_shape* shape, int32_t planes_per_table,
                            const race_options* opts, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);
/* race_hashed_fwd with the events of race_fwd_profiled (a profiling aid, no
 * counterpart in the reference). */
race_status race_hashed_fwd_profiled(const void* k_rows, const void* q_rows, const void* v,
                                     const float* planes, void* out, float* state,
                                     const race_shape* shape, int32_t planes_per_table,
                                     const race_options* opts, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream, hipEvent_t* events,
                                     int32_t max_events, int32_t* n_events);

/* ------------------------------------------------------------------------
 * Algorithm 1 with the hashing inside: the reference's causal v2 forward,
 * race_causal_forward(q, k, v, planes, beta, ...)
 * (src/causal_v2/kernels/race_causal_fwd.h:6-10, :126-130), for bf16 token
 * rows.  Per stream and token t, with Phi(x) in R^S (S = L R, R = 2^P,
 * table-major) the L tables' corner probabilities
 *     Phi_l(x)[r] = softmax_r(beta sum_p tanh(<W[l][p], x>) c_{r,p}),
 * c_{r,p} = +1 iff bit P-1-p of r is set, and A_t, B_t the inclusive sums of
 * Phi(k_j) and Phi(k_j) (x) v_j over j <= t:
 *     out_t = (Phi(q_t) . B_t) / (Phi(q_t) . A_t)   (0 where that is 0).
 * Layouts: q, k, v, out [BH][T][D] bf16, 16-byte aligned; W [L][P][D] fp32,
 * 16-byte aligned; beta one fp32 value in device memory (read by the kernels,
 * so a trainable beta never needs a host sync).  Limits (the reference's,
 * race_causal_fwd.h:45-47): D in {64, 128}, P in 1..5, L in 1..4,
 * BH <= 65535, T <= INT_MAX - 4097.
 * ------------------------------------------------------------------------ */

/* Shape of one call; mirrors CausalShape (race_causal_fwd.h:60-66). */
typedef struct race_alg1_shape {
    int64_t batch_heads; /* BH */
    int64_t seq_len;     /* T */
    int32_t head_dim;    /* D */
    int32_t num_planes;  /* P, R = 2^P corners per table */
    int32_t num_tables;  /* L */
} race_alg1_shape;

/* Rounding of the matrix-core products; mirrors Variant
 * (race_causal_fwd.h:68-70).  FP32: the features Phi enter every product as
 * bf16 hi/lo pairs (fp32-accurate; the reference's v2a accuracy).  BF16: the
 * features are rounded to bf16 once, the carried state and the masked Gram
 * matrix stay hi/lo (the rounding points of the reference's v2b). */
typedef enum race_alg1_variant {
    RACE_ALG1_FP32 = 0,
    RACE_ALG1_BF16 = 1
} race_alg1_variant;

/* Tile lengths are multiples of this many tokens (the sub-chunk C). */
#define RACE_ALG1_SUB_CHUNK_TOKENS 64
/* Largest automatic tile length (race_causal_fwd.h:74). */
#define RACE_ALG1_MAX_AUTO_TILE 4096

/* Whether the shape is within the limits above.  Host logic only. */
race_status race_alg1_shape_supported(const race_alg1_shape* shape, int32_t* supported);

/* Dynamic LDS of the output pass in bytes for (D, P, L) and `variant`;
 * mirrors output_pass_smem_bytes (race_causal_fwd.h:82-83).  Host logic. */
race_status race_alg1_output_lds_bytes(const race_alg1_shape* shape, int32_t variant,
                                       size_t* bytes);

/* Tile length an automatic call uses on the current device (a multiple of
 * RACE_ALG1_SUB_CHUNK_TOKENS, at most RACE_ALG1_MAX_AUTO_TILE, the smallest
 * for short sequences); mirrors race_causal_select_tile_tokens
 * (race_causal_fwd.h:90-95). */
race_status race_alg1_select_tile_tokens(const race_alg1_shape* shape, int32_t variant,
                                         int32_t* tile_tokens);

/* Workspace of race_alg1_fwd in bytes for a tile length (0 = automatic):
 * the tile records [BH][tiles][rec] fp32, rec = S*D + S rounded up to 64
 * floats, B [S][D] then A [S].  After the call record (n, t) holds the
 * exclusive prefix state at the first token of tile t of stream n (the
 * reference's debug prefix states, torch_binding.cpp:186-203). */
race_status race_alg1_workspace_bytes(const race_alg1_shape* shape, int32_t variant,
                                      int32_t tile_tokens, size_t* bytes, int64_t* tiles,
                                      int64_t* record_floats);

/* The forward.  tile_tokens: 0 automatic, else a positive multiple of
 * RACE_ALG1_SUB_CHUNK_TOKENS.  final_state (nullable): [BH][S*D + S] fp32,
 * the state after all T tokens (race_causal_fwd.h:20-21, layout B then A).
 * Replaces race_causal_forward (race_causal_fwd.h:126-130). */
race_status race_alg1_fwd(const void* q, const void* k, const void* v, const float* W,
                          const float* beta, void* out, float* final_state,
                          const race_alg1_shape* shape, int32_t tile_tokens, int32_t variant,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

/* race_alg1_fwd continued from a carried state: init_state [BH][S*D + S]
 * fp32 (B then A, the final_state layout) holds the sums of Phi(k) (x) v and
 * Phi(k) over all earlier tokens, and every output of this call is
 * (Phi(q_t) . (B0 + B_t)) / (Phi(q_t) . (A0 + A_t)) with A_t, B_t the inclusive
 * sums over this call's tokens.  final_state (nullable) receives the state
 * after them and may equal init_state.  The reference hands final_state off
 * for incremental generation (race_causal_fwd.h:20-21) but has no launcher
 * that takes it back; this one seeds the tile scan with it.  Workspace as for
 * race_alg1_fwd. */
race_status race_alg1_fwd_carry(const void* q, const void* k, const void* v, const float* W,
                                const float* beta, void* out, const float* init_state,
                                float* final_state, const race_alg1_shape* shape,
                                int32_t tile_tokens, int32_t variant, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* race_alg1_fwd with hipEventRecord marks around every launch, as
 * race_fwd_profiled.  A profiling aid with no counterpart in the reference. */
race_status race_alg1_fwd_profiled(const void* q, const void* k, const void* v, const float* W,
                                   const float* beta, void* out, float* final_state,
                                   const race_alg1_shape* shape, int32_t tile_tokens,
                                   int32_t variant, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream, hipEvent_t* events, int32_t max_events,
                                   int32_t* n_events);

/* race_noncausal_bwd / race_causal_bwd with a hipEventRecord on `stream`
 * before the first launch and after every launch, as race_fwd_profiled does.
 * Profiling aids with no counterpart in the reference (used by bench.py). */
race_status race_noncausal_bwd_profiled(const void* probsQ, const void* probsK, const void* V,
                                        const void* dOut, const float* state, void* dQ, void* dK,
                                        void* dV, const race_shape* shape,
                                        const race_options* opts, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream,
                                        hipEvent_t* events, int32_t max_events, int32_t* n_events);
race_status race_causal_bwd_profiled(const void* probsQ, const void* probsK, const void* V,
                                     const void* dOut, void* dQ, void* dK, void* dV,
                                     const race_shape* shape, const race_options* opts,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream,
                                     hipEvent_t* events, int32_t max_events, int32_t* n_events);

#ifdef __cplusplus
}
#endif

#endif /* RACE_MI355X_H */
