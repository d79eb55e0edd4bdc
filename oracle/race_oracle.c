/*
 * race_oracle.c -- CPU restatement of per-bucket RACE attention, in fp64.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU path is compared
 * against; it is never linked into, loaded by or called from the product
 * library.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * The function being restated is the reference's BatchedACE.forward hot span
 * (src/race_baseline.py:45-51):
 *
 *     A_pref = probsK.cumsum(dim=1)                          # [N,T,L,R]
 *     B_pref = (probsK[..., None] * V[:, :, None, None]).cumsum(dim=1)
 *     E_pref = B_pref / (A_pref[..., None] + 1e-6)
 *     out    = bmm(probsQ.view(N*T, 1, S), E_pref.view(N*T, S, d))
 *
 * i.e. per stream n and token t, with q_t, k_t in R^S (S = L*R, table-major
 * s = l*R + r) and v_t in R^d:
 *
 *     A_t = sum_{j<=t} k_j,  B_t = sum_{j<=t} k_j (x) v_j,
 *     out_t[c] = sum_s q_t[s] * B_t[s][c] / (A_t[s] + eps).
 *
 * The non-causal variant (analysis/hot-path.md:157-162,
 * src/verify_factorization.py:74-78) uses the totals over all T tokens.
 *
 * Layouts (row-major, contiguous): q, k [N][T][S] fp32; v, out [N][T][d].
 * Inputs are fp32 (bf16 inputs are widened exactly by the caller); every
 * accumulation is fp64.  "state" records are [S*d + S] doubles: B[s][c] at
 * s*d + c, then A[s] at S*d + s.
 *
 * Four independent formulations are provided so that each pins the others:
 *   race_oracle_causal_recurrence  per-token scan (src/race_fused_fwd.cu:131-146,
 *                                   mirrored in src/test_kernel_math.py:32-39),
 *                                   optionally continued from a carried state
 *                                   (the carry of src/race_chunked.py:54-63)
 *   race_oracle_causal_chunked     carried state + chunk identity
 *                                   (src/race_chunked.py:41-63,
 *                                   docs/causal_v2_design.md:70-77)
 *   race_oracle_causal_tiled       the GPU decomposition: tile totals, exclusive
 *                                   scan over tiles, chunk walk inside a tile
 *                                   (src/causal_v2/reference.py:84-103,144-159)
 *   race_oracle_noncausal_fwd/bwd  full-sequence totals and the closed-form VJP
 *   race_oracle_causal_bwd         the closed-form VJP of the causal function (the
 *                                   reference has no kernel for it; its design
 *                                   outline is docs/causal_v2_design.md:689-742)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef int64_t i64;

static void set_threads(int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
}

/* Per-token recurrence.  For every token: A += k_t, B += k_t (x) v_t, then
 * out_t = sum_s (q_t[s] / (A[s] + eps)) * B[s][:].  init_state (nullable,
 * [N][S*d + S]) is the state before the first token (zero when null), as
 * chunked_forward carries A_state, B_state into its next chunk
 * (src/race_chunked.py:54-63); final_state (nullable) receives the state
 * after the last token. */
void race_oracle_causal_recurrence(const float* q, const float* k, const float* v, double* out,
                                   double* final_state, const double* init_state, i64 N, i64 T,
                                   i64 S, i64 d, double eps, int nthreads) {
    set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* A = (double*)calloc((size_t)S, sizeof(double));
        double* B = (double*)calloc((size_t)(S * d), sizeof(double));
        if (init_state) {
            const double* st = init_state + n * (S * d + S);
            memcpy(B, st, (size_t)(S * d) * sizeof(double));
            memcpy(A, st + S * d, (size_t)S * sizeof(double));
        }
        double* w = (double*)malloc((size_t)S * sizeof(double));
        double* o = (double*)malloc((size_t)d * sizeof(double));
        for (i64 t = 0; t < T; ++t) {
            const float* qt = q + (n * T + t) * S;
            const float* kt = k + (n * T + t) * S;
            const float* vt = v + (n * T + t) * d;
            for (i64 s = 0; s < S; ++s) {
                const double ks = kt[s];
                A[s] += ks;
                double* Bs = B + s * d;
                for (i64 c = 0; c < d; ++c) Bs[c] += ks * (double)vt[c];
                w[s] = (double)qt[s] / (A[s] + eps);
            }
            for (i64 c = 0; c < d; ++c) o[c] = 0.0;
            for (i64 s = 0; s < S; ++s) {
                const double ws = w[s];
                const double* Bs = B + s * d;
                for (i64 c = 0; c < d; ++c) o[c] += ws * Bs[c];
            }
            memcpy(out + (n * T + t) * d, o, (size_t)d * sizeof(double));
        }
        if (final_state) {
            double* st = final_state + n * (S * d + S);
            memcpy(st, B, (size_t)(S * d) * sizeof(double));
            memcpy(st + S * d, A, (size_t)S * sizeof(double));
        }
        free(A);
        free(B);
        free(w);
        free(o);
    }
}

/* One chunk of `clen` tokens on top of the carried state (A0, B0), by the
 * chunk identity:
 *   Abar_i = A0 + sum_{j<=i} k_j          (inclusive running mass, per bucket)
 *   W_i    = q_i / (Abar_i + eps)
 *   O_i    = W_i . B0 + sum_{j<=i} (W_i . k_j) v_j
 * then A0 = Abar_last, B0 += sum_j k_j (x) v_j. */
static void chunk_step(const float* q, const float* k, const float* v, double* out, double* A0,
                       double* B0, i64 clen, i64 S, i64 d, double eps, double* W, double* P) {
    double* run = (double*)malloc((size_t)S * sizeof(double));
    memcpy(run, A0, (size_t)S * sizeof(double));
    for (i64 i = 0; i < clen; ++i)
        for (i64 s = 0; s < S; ++s) {
            run[s] += (double)k[i * S + s];
            W[i * S + s] = (double)q[i * S + s] / (run[s] + eps);
        }
    for (i64 i = 0; i < clen; ++i)
        for (i64 j = 0; j < clen; ++j) {
            double acc = 0.0;
            if (j <= i)
                for (i64 s = 0; s < S; ++s) acc += W[i * S + s] * (double)k[j * S + s];
            P[i * clen + j] = acc;
        }
    for (i64 i = 0; i < clen; ++i)
        for (i64 c = 0; c < d; ++c) {
            double acc = 0.0;
            for (i64 s = 0; s < S; ++s) acc += W[i * S + s] * B0[s * d + c];
            for (i64 j = 0; j <= i; ++j) acc += P[i * clen + j] * (double)v[j * d + c];
            out[i * d + c] = acc;
        }
    for (i64 s = 0; s < S; ++s)
        for (i64 c = 0; c < d; ++c) {
            double acc = 0.0;
            for (i64 i = 0; i < clen; ++i) acc += (double)k[i * S + s] * (double)v[i * d + c];
            B0[s * d + c] += acc;
        }
    memcpy(A0, run, (size_t)S * sizeof(double));
    free(run);
}

/* Carried-state chunked forward (src/race_chunked.py:41-63): chunks of
 * `chunk` tokens, the last one possibly shorter. */
void race_oracle_causal_chunked(const float* q, const float* k, const float* v, double* out,
                                double* final_state, i64 N, i64 T, i64 S, i64 d, double eps,
                                i64 chunk, int nthreads) {
    set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* A0 = (double*)calloc((size_t)S, sizeof(double));
        double* B0 = (double*)calloc((size_t)(S * d), sizeof(double));
        double* W = (double*)malloc((size_t)(chunk * S) * sizeof(double));
        double* P = (double*)malloc((size_t)(chunk * chunk) * sizeof(double));
        for (i64 t0 = 0; t0 < T; t0 += chunk) {
            const i64 clen = (T - t0 < chunk) ? (T - t0) : chunk;
            const i64 base = n * T + t0;
            chunk_step(q + base * S, k + base * S, v + base * d, out + base * d, A0, B0, clen, S,
                       d, eps, W, P);
        }
        if (final_state) {
            double* st = final_state + n * (S * d + S);
            memcpy(st, B0, (size_t)(S * d) * sizeof(double));
            memcpy(st + S * d, A0, (size_t)S * sizeof(double));
        }
        free(A0);
        free(B0);
        free(W);
        free(P);
    }
}

/* The GPU decomposition, in fp64: (1) per-tile totals of k and k (x) v over
 * tiles of `tile` tokens, (2) an exclusive scan of the totals over tiles in
 * order, (3) per tile, a walk over chunks of `chunk` tokens starting from the
 * tile's exclusive prefix.  prefix_states (nullable) receives the scanned
 * records [N][tiles][S*d + S]; final_state (nullable) the totals over T. */
void race_oracle_causal_tiled(const float* q, const float* k, const float* v, double* out,
                              double* prefix_states, double* final_state, i64 N, i64 T, i64 S,
                              i64 d, double eps, i64 tile, i64 chunk, int nthreads) {
    set_threads(nthreads);
    const i64 tiles = (T + tile - 1) / tile;
    const i64 rec = S * d + S;
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* pref = (double*)calloc((size_t)(tiles * rec), sizeof(double));
        /* (1) tile totals */
        for (i64 t = 0; t < tiles; ++t) {
            double* r = pref + t * rec;
            const i64 b = t * tile, e = (b + tile < T) ? b + tile : T;
            for (i64 j = b; j < e; ++j) {
                const float* kj = k + (n * T + j) * S;
                const float* vj = v + (n * T + j) * d;
                for (i64 s = 0; s < S; ++s) {
                    r[S * d + s] += kj[s];
                    for (i64 c = 0; c < d; ++c) r[s * d + c] += (double)kj[s] * (double)vj[c];
                }
            }
        }
        /* (2) exclusive scan over tiles, element by element, in tile order */
        double* run = (double*)calloc((size_t)rec, sizeof(double));
        for (i64 t = 0; t < tiles; ++t) {
            double* r = pref + t * rec;
            for (i64 e = 0; e < rec; ++e) {
                const double tot = r[e];
                r[e] = run[e];
                run[e] += tot;
            }
        }
        if (final_state) memcpy(final_state + n * rec, run, (size_t)rec * sizeof(double));
        /* (3) chunk walk inside each tile */
        double* A0 = (double*)malloc((size_t)S * sizeof(double));
        double* B0 = (double*)malloc((size_t)(S * d) * sizeof(double));
        double* W = (double*)malloc((size_t)(chunk * S) * sizeof(double));
        double* P = (double*)malloc((size_t)(chunk * chunk) * sizeof(double));
        for (i64 t = 0; t < tiles; ++t) {
            memcpy(B0, pref + t * rec, (size_t)(S * d) * sizeof(double));
            memcpy(A0, pref + t * rec + S * d, (size_t)S * sizeof(double));
            const i64 b = t * tile, e = (b + tile < T) ? b + tile : T;
            for (i64 t0 = b; t0 < e; t0 += chunk) {
                const i64 clen = (e - t0 < chunk) ? (e - t0) : chunk;
                const i64 base = n * T + t0;
                chunk_step(q + base * S, k + base * S, v + base * d, out + base * d, A0, B0, clen,
                           S, d, eps, W, P);
            }
        }
        if (prefix_states) memcpy(prefix_states + n * tiles * rec, pref,
                                  (size_t)(tiles * rec) * sizeof(double));
        free(pref);
        free(run);
        free(A0);
        free(B0);
        free(W);
        free(P);
    }
}

/* Non-causal forward: A = sum_j k_j, B = sum_j k_j (x) v_j, E = B / (A + eps)
 * row-wise, out_t = q_t . E.  state (nullable) receives (B, A) per stream. */
void race_oracle_noncausal_fwd(const float* q, const float* k, const float* v, double* out,
                               double* state, i64 N, i64 T, i64 S, i64 d, double eps,
                               int nthreads) {
    set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* A = (double*)calloc((size_t)S, sizeof(double));
        double* B = (double*)calloc((size_t)(S * d), sizeof(double));
        for (i64 j = 0; j < T; ++j) {
            const float* kj = k + (n * T + j) * S;
            const float* vj = v + (n * T + j) * d;
            for (i64 s = 0; s < S; ++s) {
                A[s] += kj[s];
                for (i64 c = 0; c < d; ++c) B[s * d + c] += (double)kj[s] * (double)vj[c];
            }
        }
        double* E = (double*)malloc((size_t)(S * d) * sizeof(double));
        for (i64 s = 0; s < S; ++s)
            for (i64 c = 0; c < d; ++c) E[s * d + c] = B[s * d + c] / (A[s] + eps);
        for (i64 t = 0; t < T; ++t) {
            const float* qt = q + (n * T + t) * S;
            double* o = out + (n * T + t) * d;
            for (i64 c = 0; c < d; ++c) o[c] = 0.0;
            for (i64 s = 0; s < S; ++s)
                for (i64 c = 0; c < d; ++c) o[c] += (double)qt[s] * E[s * d + c];
        }
        if (state) {
            memcpy(state + n * (S * d + S), B, (size_t)(S * d) * sizeof(double));
            memcpy(state + n * (S * d + S) + S * d, A, (size_t)S * sizeof(double));
        }
        free(A);
        free(B);
        free(E);
    }
}

/* Non-causal backward, the closed-form VJP of race_oracle_noncausal_fwd for
 * the upstream gradient g = dOut:
 *   dQ = g E^T;  dE = Q^T g;  dB = dE / (A + eps);
 *   dA[s] = -sum_c dE[s][c] E[s][c] / (A[s] + eps);
 *   dK = V dB^T + 1 dA^T;  dV = K dB. */
void race_oracle_noncausal_bwd(const float* q, const float* k, const float* v, const float* g,
                               double* dq, double* dk, double* dv, i64 N, i64 T, i64 S, i64 d,
                               double eps, int nthreads) {
    set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* A = (double*)calloc((size_t)S, sizeof(double));
        double* B = (double*)calloc((size_t)(S * d), sizeof(double));
        double* dE = (double*)calloc((size_t)(S * d), sizeof(double));
        for (i64 j = 0; j < T; ++j) {
            const float* kj = k + (n * T + j) * S;
            const float* vj = v + (n * T + j) * d;
            const float* qj = q + (n * T + j) * S;
            const float* gj = g + (n * T + j) * d;
            for (i64 s = 0; s < S; ++s) {
                A[s] += kj[s];
                for (i64 c = 0; c < d; ++c) {
                    B[s * d + c] += (double)kj[s] * (double)vj[c];
                    dE[s * d + c] += (double)qj[s] * (double)gj[c];
                }
            }
        }
        double* E = (double*)malloc((size_t)(S * d) * sizeof(double));
        double* dB = (double*)malloc((size_t)(S * d) * sizeof(double));
        double* dA = (double*)calloc((size_t)S, sizeof(double));
        for (i64 s = 0; s < S; ++s) {
            const double den = A[s] + eps;
            for (i64 c = 0; c < d; ++c) {
                E[s * d + c] = B[s * d + c] / den;
                dB[s * d + c] = dE[s * d + c] / den;
                dA[s] -= dE[s * d + c] * E[s * d + c] / den;
            }
        }
        for (i64 t = 0; t < T; ++t) {
            const float* gt = g + (n * T + t) * d;
            const float* vt = v + (n * T + t) * d;
            const float* kt = k + (n * T + t) * S;
            double* dqt = dq + (n * T + t) * S;
            double* dkt = dk + (n * T + t) * S;
            double* dvt = dv + (n * T + t) * d;
            for (i64 s = 0; s < S; ++s) {
                double aq = 0.0, ak = dA[s];
                for (i64 c = 0; c < d; ++c) {
                    aq += (double)gt[c] * E[s * d + c];
                    ak += (double)vt[c] * dB[s * d + c];
                }
                dqt[s] = aq;
                dkt[s] = ak;
            }
            for (i64 c = 0; c < d; ++c) {
                double acc = 0.0;
                for (i64 s = 0; s < S; ++s) acc += (double)kt[s] * dB[s * d + c];
                dvt[c] = acc;
            }
        }
        free(A);
        free(B);
        free(dE);
        free(E);
        free(dB);
        free(dA);
    }
}

/* Causal backward, the closed-form VJP of the causal function for the
 * upstream gradient g = dOut.  With the inclusive prefix sums A_i, B_i,
 * r_i = 1 / (A_i + eps) and W_i = q_i * r_i (elementwise over buckets):
 *   dq_i[s]    = r_i[s] * <B_i[s][:], g_i>
 *   alpha_i[s] = -W_i[s] * dq_i[s]                  (dLoss/dA_i)
 *   Z_j        = sum_{i>=j} W_i (x) g_i,  Y_j = sum_{i>=j} alpha_i   (suffix sums)
 *   dk_j[s]    = <Z_j[s][:], v_j> + Y_j[s]
 *   dv_j[c]    = sum_s k_j[s] Z_j[s][c]
 * One forward pass over the tokens (prefix sums) stores W and alpha; one
 * backward pass accumulates the suffix sums. */
void race_oracle_causal_bwd(const float* q, const float* k, const float* v, const float* g,
                            double* dq, double* dk, double* dv, i64 N, i64 T, i64 S, i64 d,
                            double eps, int nthreads) {
    set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* A = (double*)calloc((size_t)S, sizeof(double));
        double* B = (double*)calloc((size_t)(S * d), sizeof(double));
        double* W = (double*)malloc((size_t)(T * S) * sizeof(double));
        double* alpha = (double*)malloc((size_t)(T * S) * sizeof(double));
        for (i64 t = 0; t < T; ++t) {
            const float* qt = q + (n * T + t) * S;
            const float* kt = k + (n * T + t) * S;
            const float* vt = v + (n * T + t) * d;
            const float* gt = g + (n * T + t) * d;
            double* dqt = dq + (n * T + t) * S;
            for (i64 s = 0; s < S; ++s) {
                const double ks = kt[s];
                A[s] += ks;
                double* Bs = B + s * d;
                double u = 0.0;
                for (i64 c = 0; c < d; ++c) {
                    Bs[c] += ks * (double)vt[c];
                    u += Bs[c] * (double)gt[c];
                }
                const double r = 1.0 / (A[s] + eps);
                dqt[s] = r * u;
                W[t * S + s] = (double)qt[s] * r;
                alpha[t * S + s] = -W[t * S + s] * dqt[s];
            }
        }
        double* Z = (double*)calloc((size_t)(S * d), sizeof(double));
        double* Y = (double*)calloc((size_t)S, sizeof(double));
        for (i64 t = T - 1; t >= 0; --t) {
            const float* kt = k + (n * T + t) * S;
            const float* vt = v + (n * T + t) * d;
            const float* gt = g + (n * T + t) * d;
            double* dkt = dk + (n * T + t) * S;
            double* dvt = dv + (n * T + t) * d;
            for (i64 s = 0; s < S; ++s) {
                const double ws = W[t * S + s];
                double* Zs = Z + s * d;
                double acc = 0.0;
                for (i64 c = 0; c < d; ++c) {
                    Zs[c] += ws * (double)gt[c];
                    acc += Zs[c] * (double)vt[c];
                }
                Y[s] += alpha[t * S + s];
                dkt[s] = acc + Y[s];
            }
            for (i64 c = 0; c < d; ++c) {
                double acc = 0.0;
                for (i64 s = 0; s < S; ++s) acc += (double)kt[s] * Z[s * d + c];
                dvt[c] = acc;
            }
        }
        free(A);
        free(B);
        free(W);
        free(alpha);
        free(Z);
        free(Y);
    }
}

/* ------------------------------------------------------------------------
 * Algorithm 1 with the hashing inside (the reference's causal v2 forward,
 * src/causal_v2/kernels/race_causal_fwd.h:6-10; ground truth
 * src/causal_v2/reference.py:100-128).  Token rows q, k, v are [N][T][D];
 * the planes W are [L][P][D].  The feature map of a row x, table-major
 * (s = l R + r, R = 2^P), is the direct length-R softmax of
 * src/noncausal/reference.py:89-100:
 *     u_p        = tanh(<W[l][p], x>)
 *     phi_l[r]   = softmax_r(beta sum_p u_p c_{r,p}),
 * c_{r,p} = +1 iff bit P-1-p of r is set (plane 0 the most significant,
 * src/noncausal/reference.py:66-77).  With A_t, B_t the inclusive sums of
 * phi(k_j) and phi(k_j) (x) v_j over j <= t:
 *     global normalization (perbucket = 0):
 *         out_t = (phi(q_t) . B_t) / (phi(q_t) . A_t), 0 where the
 *         denominator is exactly 0 (src/causal_v2/reference.py:81-86);
 *     per-bucket normalization (perbucket = 1, the bridge to
 *     src/race_baseline.py:45-51, src/causal_v2/reference.py:144-159):
 *         out_t = sum_s phi(q_t)[s] B_t[s][:] / (A_t[s] + eps).
 * prefix (nullable, tile > 0): [N][ceil(T / tile)][S*D + S], the state before
 * the first token of every tile (B then A); final_state (nullable):
 * [N][S*D + S], the state after the last token.
 */
static void alg1_features(const float* x, const float* W, double beta, i64 D, i64 L, i64 P,
                          double* u, double* phi) {
    const i64 R = (i64)1 << P;
    for (i64 l = 0; l < L; ++l) {
        for (i64 p = 0; p < P; ++p) {
            const float* w = W + (l * P + p) * D;
            double acc = 0.0;
            for (i64 c = 0; c < D; ++c) acc += (double)w[c] * (double)x[c];
            u[p] = tanh(acc);
        }
        double* ph = phi + l * R;
        double mx = -INFINITY;
        for (i64 r = 0; r < R; ++r) {
            double lg = 0.0;
            for (i64 p = 0; p < P; ++p) lg += ((r >> (P - 1 - p)) & 1) ? u[p] : -u[p];
            ph[r] = beta * lg;
            if (ph[r] > mx) mx = ph[r];
        }
        double sum = 0.0;
        for (i64 r = 0; r < R; ++r) {
            ph[r] = exp(ph[r] - mx);
            sum += ph[r];
        }
        for (i64 r = 0; r < R; ++r) ph[r] /= sum;
    }
}

void race_oracle_alg1_causal(const float* q, const float* k, const float* v, const float* W,
                             double beta, double* out, double* prefix, double* final_state, i64 N,
                             i64 T, i64 D, i64 L, i64 P, int perbucket, double eps, i64 tile,
                             int nthreads) {
    const i64 S = L * ((i64)1 << P), rec = S * D + S;
    const i64 tiles = tile > 0 ? (T + tile - 1) / tile : 0;
    set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 n = 0; n < N; ++n) {
        double* st = (double*)calloc((size_t)rec, sizeof(double));  /* B [S][D] then A [S] */
        double* fq = (double*)malloc((size_t)S * sizeof(double));
        double* fk = (double*)malloc((size_t)S * sizeof(double));
        double* u = (double*)malloc((size_t)P * sizeof(double));
        double* o = (double*)malloc((size_t)D * sizeof(double));
        double* B = st;
        double* A = st + S * D;
        for (i64 t = 0; t < T; ++t) {
            if (prefix && tile > 0 && t % tile == 0)
                memcpy(prefix + (n * tiles + t / tile) * rec, st, (size_t)rec * sizeof(double));
            const float* vt = v + (n * T + t) * D;
            alg1_features(k + (n * T + t) * D, W, beta, D, L, P, u, fk);
            alg1_features(q + (n * T + t) * D, W, beta, D, L, P, u, fq);
            for (i64 s = 0; s < S; ++s) {
                A[s] += fk[s];
                double* Bs = B + s * D;
                for (i64 c = 0; c < D; ++c) Bs[c] += fk[s] * (double)vt[c];
            }
            for (i64 c = 0; c < D; ++c) o[c] = 0.0;
            double den = 0.0;
            for (i64 s = 0; s < S; ++s) {
                const double ws = perbucket ? fq[s] / (A[s] + eps) : fq[s];
                const double* Bs = B + s * D;
                for (i64 c = 0; c < D; ++c) o[c] += ws * Bs[c];
                den += fq[s] * A[s];
            }
            double* ot = out + (n * T + t) * D;
            for (i64 c = 0; c < D; ++c)
                ot[c] = perbucket ? o[c] : (den == 0.0 ? 0.0 : o[c] / den);
        }
        if (final_state) memcpy(final_state + n * rec, st, (size_t)rec * sizeof(double));
        free(st);
        free(fq);
        free(fk);
        free(u);
        free(o);
    }
}
