// race_api.hip -- the extern "C" entry points of include/race_mi355x.h:
// argument validation, tile selection, workspace carving and launch order.
//
// Mirrors the reference's torch-free launcher contract
// (src/causal_v2/kernels/race_causal_fwd.h:40-49): caller-owned outputs and
// workspace, one stream, no allocation, no host synchronization, first error
// returned, hipErrorInvalidValue for anything the kernels do not support.
#include <atomic>
#include <climits>
#include <mutex>

#include "race_internal.h"

namespace race {
namespace {

constexpr int64_t kMaxStreams = 65535;  // grid.y
// Longest automatic tile: the MFMA causal forward takes up to 16384 tokens
// (fewer tile records; measured faster at cfg3), every other path 4096.
constexpr int kMaxAutoTile = 16384;
constexpr int kMaxAutoTileOther = 4096;
// Causal backward of bf16 tokens with d = 128 and S = 128 or 256: backward
// walks over 128-bucket x 128-column blocks (causal_bwd_dkv_wide_kernel).
#ifndef RACE_BWD_WIDE_WALKS
#define RACE_BWD_WIDE_WALKS 1
#endif
constexpr bool kBwdWideWalks = RACE_BWD_WIDE_WALKS != 0;

int64_t round64(int64_t floats) { return ((floats + 63) / 64) * 64; }

bool shape_ok(const race_shape* sh) {
    if (!sh) return false;
    if (sh->num_streams < 0 || sh->num_streams > kMaxStreams) return false;
    if (sh->seq_len < 0 || sh->seq_len > int64_t(INT_MAX) - kMaxAutoTile) return false;
    if (sh->num_tables < 1 || sh->num_buckets < 1) return false;
    const int64_t S = int64_t(sh->num_tables) * sh->num_buckets;
    if (S > 256) return false;
    if (sh->head_dim < 1 || sh->head_dim > 128) return false;
    if (sh->dtype != RACE_F32 && sh->dtype != RACE_BF16) return false;
    const int64_t w = S > sh->head_dim ? S : sh->head_dim;
    if (sh->num_streams > 0 && sh->seq_len > 0 &&
        sh->num_streams * sh->seq_len > (int64_t(1) << 62) / w)
        return false;
    return true;
}

int sub(const race_shape* sh) { return sh->num_tables * sh->num_buckets; }

// Whether `tile` rows of `width` elements of `elem` bytes stay below 2^31
// bytes, the range of one buffer resource.
bool tile_fits_buffer(int64_t tile, int64_t width, int64_t elem) {
    return tile * width * elem < (int64_t(1) << 31);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int kernel_choice(const race_options* o) { return o ? o->kernel : RACE_KERNEL_AUTO; }

// Resolves which kernel family runs; INVALID_VALUE if the request cannot be met.
race_status resolve_kernel(const race_shape* sh, int causal, const race_options* o, bool* mfma) {
    const int k = kernel_choice(o);
    if (k != RACE_KERNEL_AUTO && k != RACE_KERNEL_VALU && k != RACE_KERNEL_MFMA &&
        k != RACE_KERNEL_MFMA_WG && k != RACE_KERNEL_SINGLE && k != RACE_KERNEL_MFMA_PRECISE)
        return RACE_ERROR_INVALID_VALUE;
    const bool has = causal && mfma_causal_supported(sub(sh), sh->head_dim);
    const bool forced = k == RACE_KERNEL_MFMA || k == RACE_KERNEL_MFMA_WG || k == RACE_KERNEL_SINGLE ||
                        k == RACE_KERNEL_MFMA_PRECISE;
    if (forced && !has) return RACE_ERROR_INVALID_VALUE;
    *mfma = forced || (k == RACE_KERNEL_AUTO && has);
    return RACE_SUCCESS;
}

// Device attributes the tile policies read on every call, cached per device
// (hipGetDevice is a thread-local read; the attribute query is not).
constexpr int kMaxCachedDevices = 64;
std::atomic<int> g_cu_count[kMaxCachedDevices];
std::atomic<int> g_lds_bytes[kMaxCachedDevices];

hipError_t cached_attribute(std::atomic<int>* table, hipDeviceAttribute_t attr, int* value) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    const bool cacheable = dev >= 0 && dev < kMaxCachedDevices;
    if (cacheable) {
        const int v = table[dev].load(std::memory_order_relaxed);
        if (v > 0) {
            *value = v;
            return hipSuccess;
        }
    }
    int v = 0;
    err = hipDeviceGetAttribute(&v, attr, dev);
    if (err != hipSuccess) return err;
    if (cacheable && v > 0) table[dev].store(v, std::memory_order_relaxed);
    *value = v;
    return hipSuccess;
}

hipError_t cu_count(int* cus) {
    return cached_attribute(g_cu_count, hipDeviceAttributeMultiprocessorCount, cus);
}

int pow2_floor(int64_t x) {
    int p = 1;
    while (int64_t(p) * 2 <= x && p < (1 << 30)) p *= 2;
    return p;
}

race_status resolve_tile(const race_shape* sh, int causal, const race_options* o, bool mfma,
                         int* tile) {
    if (kernel_choice(o) == RACE_KERNEL_SINGLE) {
        if (o->tile_tokens != 0 && o->tile_tokens != kSinglePassTile) return RACE_ERROR_INVALID_VALUE;
        *tile = kSinglePassTile;
        return RACE_SUCCESS;
    }
    if (o && o->tile_tokens != 0) {
        if (o->tile_tokens < 0 || o->tile_tokens % RACE_SUB_CHUNK_TOKENS != 0)
            return RACE_ERROR_INVALID_VALUE;
        *tile = o->tile_tokens;
        return RACE_SUCCESS;
    }
    const int64_t work = sh->num_streams * sh->seq_len;
    if (work == 0) {
        *tile = RACE_SUB_CHUNK_TOKENS;
        return RACE_SUCCESS;
    }
    int cus = 0;
    const hipError_t err = cu_count(&cus);
    if (err != hipSuccess) return err;
    if (cus < 1) cus = 1;
    // Aim for a few resident workgroups per compute unit so the output pass
    // streams HBM from every CU; longer tiles amortize the tile record
    // (4*(S*d+S) bytes read and written per tile) over more tokens.
    const int64_t per_cu =
        (causal && mfma) ? mfma_tiles_per_cu(sub(sh), sh->head_dim, sh->dtype, kernel_choice(o)) : 2;
    int t = pow2_floor(work / (per_cu * cus));
    const int cap = (causal && mfma) ? kMaxAutoTile : kMaxAutoTileOther;
    if (t < RACE_SUB_CHUNK_TOKENS) t = RACE_SUB_CHUNK_TOKENS;
    if (t > cap) t = cap;
    *tile = t;
    return RACE_SUCCESS;
}

race_status make_problem(const race_shape* sh, int causal, const race_options* o, bool* mfma,
                         Problem* p) {
    if (!shape_ok(sh)) return RACE_ERROR_INVALID_VALUE;
    race_status st = resolve_kernel(sh, causal, o, mfma);
    if (st != RACE_SUCCESS) return st;
    int tile = 0;
    st = resolve_tile(sh, causal, o, *mfma, &tile);
    if (st != RACE_SUCCESS) return st;
    // Kernels address a tile's rows through one buffer resource, whose range
    // is a 32-bit byte count.
    if (!tile_fits_buffer(tile, sub(sh) > sh->head_dim ? sub(sh) : sh->head_dim,
                          sh->dtype == RACE_BF16 ? 2 : 4))
        return RACE_ERROR_INVALID_VALUE;
    p->N = sh->num_streams;
    p->T = sh->seq_len;
    p->S = sub(sh);
    p->d = sh->head_dim;
    p->dtype = sh->dtype;
    p->kernel = kernel_choice(o);
    p->tile = tile;
    p->tiles = sh->seq_len == 0 ? 0 : (sh->seq_len + tile - 1) / tile;
    p->rec = record_floats(p->S, p->d);
    if (p->kernel == RACE_KERNEL_SINGLE) {
        int cus = 0;
        const hipError_t err = cu_count(&cus);
        if (err != hipSuccess) return err;
        if (!causal || !single_pass_supported(*p, cus)) return RACE_ERROR_INVALID_VALUE;
        p->single = true;
    }
    return RACE_SUCCESS;
}

// Workspace regions, in floats, each a multiple of 64 floats.
struct FwdLayout {
    int64_t records = 0;  // [N][tiles][rec]
    int64_t E = 0;        // non-causal: [N][S*d]
    int64_t words = 0;    // one-read causal forward: tile flags and control words (int32)
    int64_t total() const { return records + E + words; }
};

FwdLayout fwd_layout(const Problem& p, int causal) {
    FwdLayout l;
    l.records = p.N * p.tiles * p.rec;
    if (!causal) l.E = round64(p.N * p.S * p.d);
    if (p.single) l.words = single_pass_flag_words(p.N, p.tiles) + kSinglePassCtlWords;
    return l;
}

// Non-causal forwards with at most this many tiles per stream sum the tile
// records as the map stages its matrix (every map workgroup of a stream sums
// them again); longer ones reduce them once into E first.
constexpr int64_t kFoldTiles = 4;

struct BwdLayout {
    int64_t records = 0, dB = 0, dA = 0;
    int64_t total() const { return records + dB + dA; }
};

BwdLayout bwd_layout(const Problem& p) {
    BwdLayout l;
    l.records = p.N * p.tiles * p.rec;
    l.dB = round64(p.N * p.S * p.d);
    l.dA = round64(p.N * p.S);
    return l;
}

// Causal backward workspace: suffix records, the running mass at every
// sub-chunk start (sized for the shortest sub-chunk, 16 tokens), an fp32 copy
// of dQ and, unless the caller hands in the forward's records, the forward
// prefix records (last, so the two layouts share every other offset).
struct CausalBwdLayout {
    int64_t bwd = 0, apre = 0, dq32 = 0, fwd = 0, acc = 0;
    int64_t total() const { return bwd + apre + dq32 + fwd + acc; }
};

// Column groups of the vector-ALU causal backward: 1 where the state of
// every value column fits one workgroup's LDS, else the fewest groups of
// equal width that fit (each walk then takes one group; causal_bwd.hip), 0
// where none does.  *C gets the groups' sub-chunk length.
int causal_bwd_groups(int S, int d, int lds_limit, int* C) {
    for (int G = 1; G <= d; ++G) {
        if (d % G != 0) continue;
        const int c = causal_bwd_chunk(S, d / G, lds_limit);
        if (c != 0) {
            *C = c;
            return G;
        }
    }
    *C = 0;
    return 0;
}

// How a causal backward runs: on the matrix cores in 64 x 64 blocks (bucket
// group x value group; one block at S = d = 64; with bf16 tokens, d = 128 and
// S = 128 or 256, walks over 128 x 128 blocks), or on the vector ALU in
// column groups (0 groups: refused).  Planned for gfx950's LDS per
// workgroup, so the workspace query needs no device.
struct CausalBwdPlan {
    bool mfma = false;
    int mblocks = 1, hblocks = 1;  // bucket groups, value groups (matrix cores)
    int groups = 0, C = 0;         // column groups, sub-chunk (vector ALU)
    bool bf16 = false;
    bool blocked() const { return mfma && mblocks * hblocks > 1; }
    // bf16 with d = 128: one forward walk per bucket group over both value
    // groups (its dQ whole; no dQ running sum).
    bool wide() const { return blocked() && bf16 && hblocks == 2; }
    // ... and, with an even number of bucket groups (S = 128 or 256), one
    // backward walk per pair of them over every value column (their dK
    // whole; dV summed over the pairs).
    bool wide2() const { return wide() && mblocks % 2 == 0 && kBwdWideWalks; }
};

// The causal backward's kernel choices: automatic, vector ALU or matrix cores.
bool bwd_kernel_ok(int kernel) {
    return kernel == RACE_KERNEL_AUTO || kernel == RACE_KERNEL_VALU || kernel == RACE_KERNEL_MFMA;
}

CausalBwdPlan plan_causal_bwd(const Problem& p, int kernel) {
    CausalBwdPlan pl;
    pl.mfma = kernel != RACE_KERNEL_VALU && causal_bwd_mfma_supported(p.S, p.d) && p.tile % 32 == 0;
    pl.bf16 = p.dtype == RACE_BF16;
    if (pl.mfma) {
        pl.mblocks = p.S / 64;
        pl.hblocks = p.d / 64;
        pl.groups = 1;
        pl.C = 32;
    } else {
        pl.groups = causal_bwd_groups(p.S, p.d, kGfx950LdsBytes, &pl.C);
    }
    return pl;
}

// The running mass of one 128-bucket block walk: 128 floats per 32-token
// sub-chunk of each tile (the walks take tiles of whole sub-chunks).
int64_t wide_apre_floats(const Problem& p) { return round64(p.N * p.tiles * (p.tile / 32) * int64_t(128)); }

// Workspace of the causal backward: the forward prefix records unless given,
// the suffix records (of one column group, or of one 64 x 64 block: the
// groups and blocks take turns), the running mass every 16 tokens, dq32 (dQ,
// or the current group's or block's part of it); with blocks of bf16 tokens
// fp32 running sums of dQ, dK, dV; with several column groups of bf16 tokens
// the running sums of dQ and dK.
CausalBwdLayout causal_bwd_layout(const Problem& p, bool records_given, const CausalBwdPlan& pl) {
    CausalBwdLayout l;
    const int64_t NT = p.N * p.T;
    l.fwd = records_given ? 0 : p.N * p.tiles * p.rec;
    if (pl.wide2()) {
        // Per pair of bucket groups (one forward-walk launch covers them
        // all): the suffix records of its four 64 x 64 blocks, its running
        // mass, and dQ's bf16 remainders and bf16 part (128 buckets, 2 + 2
        // bytes); a dV running sum when there are several pairs.
        const int64_t pairs = pl.mblocks / 2;
        l.bwd = pairs * 4 * p.N * p.tiles * record_floats(64, 64);
        l.apre = pairs * wide_apre_floats(p);
        l.dq32 = round64(pairs * NT * 128);
        l.acc = pairs > 1 ? round64(NT * p.d) : 0;
        return l;
    }
    if (pl.blocked()) {
        // One walk over both value groups (bf16, d = 128) keeps the suffix
        // records of both groups.
        l.bwd = (pl.wide() ? 2 : 1) * p.N * p.tiles * record_floats(64, 64);
        l.apre = round64(p.N * p.tiles * (p.tile / 16) * int64_t(64));
        l.dq32 = round64(NT * 64);
        // bf16: fp32 running sums of dK and dV, and of dQ unless one walk
        // takes every value column.
        l.acc = p.dtype == RACE_BF16 ? (pl.wide() ? 1 : 2) * round64(NT * p.S) + round64(NT * p.d) : 0;
        return l;
    }
    const int groups = pl.groups > 1 ? pl.groups : 1;
    const int64_t rec_g = groups > 1 ? record_floats(p.S, p.d / groups) : p.rec;
    l.bwd = p.N * p.tiles * rec_g;
    l.apre = round64(p.N * p.tiles * (p.tile / 16) * int64_t(p.S));
    l.dq32 = round64(NT * p.S);
    l.acc = (groups > 1 && p.dtype == RACE_BF16) ? 2 * round64(NT * p.S) : 0;
    return l;
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

// p[0 .. n) = 0 (a no-op when p is null: an optional output not asked for).
hipError_t zero_fill(float* p, int64_t n, hipStream_t stream) {
    if (n <= 0 || !p) return hipSuccess;
    fill_zero_kernel<<<unsigned((n + kThreads - 1) / kThreads), kThreads, 0, stream>>>(p, n);
    return hipGetLastError();
}

// The reverse scan of suffix records kept as pr.N record streams (several
// arrays of N streams each, back to back), in launches of at most
// kMaxStreams streams (the scan's grid.y).
hipError_t scan_suffix_records(float* records, const Problem& pr, hipStream_t stream) {
    for (int64_t n0 = 0; n0 < pr.N; n0 += kMaxStreams) {
        Problem part = pr;
        part.N = pr.N - n0 < kMaxStreams ? pr.N - n0 : kMaxStreams;
        const hipError_t e = launch_tile_scan(records + n0 * pr.tiles * pr.rec, nullptr, part, stream, /*reverse=*/true);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

__global__ void copy_floats_kernel(const float* src, float* dst, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// dst = src elementwise (a no-op when dst is null or is src).
hipError_t copy_floats(const float* src, float* dst, int64_t n, hipStream_t stream) {
    if (n <= 0 || !dst || dst == src) return hipSuccess;
    copy_floats_kernel<<<unsigned((n + kThreads - 1) / kThreads), kThreads, 0, stream>>>(src, dst, n);
    return hipGetLastError();
}

hipError_t max_lds(int* bytes) {
    return cached_attribute(g_lds_bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, bytes);
}


// The non-causal reduction and map: the 16-byte-vector kernels when both
// widths are multiples of 4, the scalar ones otherwise.
hipError_t outer_sums(const void* x, const void* y, float* records, const Problem& p, int Wa,
                      int Wb, hipStream_t stream) {
    if (v4_widths(Wa, Wb)) return launch_outer_sums4(x, y, records, p, Wa, Wb, stream);
    return launch_tile_outer_sums(x, y, records, p, Wa, Wb, stream);
}

hipError_t token_map(const void* x, void* out, const MapOperand& op, const Problem& p, int Wa,
                     int Wb, hipStream_t stream) {
    if (v4_widths(Wa, Wb)) return launch_map4(x, out, op, p, Wa, Wb, stream);
    return launch_token_map(x, out, op, p, Wa, Wb, stream);
}

MapOperand map_operand(const float* m, int64_t stream, int64_t row, int64_t col) {
    MapOperand op;
    op.m = m;
    op.stream = stream;
    op.row = row;
    op.col = col;
    return op;
}

#define RACE_TRY(expr)                                   \
    do {                                                 \
        const hipError_t race_err_ = (expr);             \
        if (race_err_ != hipSuccess) return race_err_;   \
    } while (0)

}  // namespace
}  // namespace race

using namespace race;

extern "C" {

int32_t race_abi_version(void) { return RACE_ABI_VERSION; }

const char* race_status_string(race_status status) {
    if (status == RACE_SUCCESS) return "success";
    if (status == RACE_ERROR_INVALID_VALUE)
        return "invalid value: unsupported shape or kernel, null or misaligned pointer, "
               "workspace too small, or tile length not a positive multiple of "
               "RACE_SUB_CHUNK_TOKENS";
    if (status == RACE_ERROR_SINGLE_PASS_GAVE_UP)
        return "one-read forward gave up: a bounded wait of RACE_KERNEL_SINGLE expired; the "
               "output rows of the tiles whose prefix never arrived, and the state, are NaN";
    if (status == RACE_ERROR_SCRATCH_TOO_SMALL)
        return "scratch too small: the call needs more workspace than the "
               "RACE_NOALLOC_SCRATCH_BYTES race_fwd_noalloc holds per GPU; use race_fwd "
               "with a caller-allocated workspace (race_fwd_workspace_bytes), or a longer tile";
    return hipGetErrorString(static_cast<hipError_t>(status));
}

race_status race_shape_supported(const race_shape* shape, int32_t* supported, int32_t* has_mfma) {
    if (!shape || !supported) return RACE_ERROR_INVALID_VALUE;
    *supported = shape_ok(shape) ? 1 : 0;
    if (has_mfma)
        *has_mfma = (*supported && mfma_causal_supported(sub(shape), shape->head_dim)) ? 1 : 0;
    return RACE_SUCCESS;
}

race_status race_select_tile_tokens(const race_shape* shape, int32_t causal,
                                    const race_options* opts, int32_t* tile_tokens) {
    if (!tile_tokens) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    bool mfma = false;
    const race_status st = make_problem(shape, causal, opts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    *tile_tokens = p.tile;
    return RACE_SUCCESS;
}

race_status race_fwd_workspace_bytes(const race_shape* shape, int32_t causal,
                                     const race_options* opts, size_t* bytes, int64_t* tiles,
                                     int64_t* record_floats_out) {
    if (!bytes) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    bool mfma = false;
    const race_status st = make_problem(shape, causal, opts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    *bytes = size_t(fwd_layout(p, causal).total()) * sizeof(float);
    if (tiles) *tiles = p.tiles;
    if (record_floats_out) *record_floats_out = p.rec;
    return RACE_SUCCESS;
}

}  // extern "C"

namespace race {
namespace {

race_status fwd_impl(const void* probsQ, const void* probsK, const void* V, void* out, float* state,
                     const float* init, const race_shape* shape, int32_t causal,
                     const race_options* opts, void* workspace, size_t workspace_bytes,
                     hipStream_t stream, Marks* marks) {
    Problem p;
    bool mfma = false;
    race_status st = make_problem(shape, causal, opts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    if (state && !aligned16(state)) return RACE_ERROR_INVALID_VALUE;
    if (init && (!causal || !aligned16(init))) return RACE_ERROR_INVALID_VALUE;
    p.init = init;
    if (p.N == 0 || p.T == 0) {
        RACE_TRY(marks->mark(stream));
        if (init)
            RACE_TRY(copy_floats(init, state, p.N * state_floats(p.S, p.d), stream));
        else
            RACE_TRY(zero_fill(state, p.N * state_floats(p.S, p.d), stream));
        return marks->mark(stream);
    }
    if (!probsQ || !probsK || !V || !out) return RACE_ERROR_INVALID_VALUE;
    if (!aligned16(probsQ) || !aligned16(probsK) || !aligned16(V) || !aligned16(out))
        return RACE_ERROR_INVALID_VALUE;
    const FwdLayout l = fwd_layout(p, causal);
    if (!workspace || !aligned16(workspace) || workspace_bytes < size_t(l.total()) * sizeof(float))
        return RACE_ERROR_INVALID_VALUE;
    float* ws = static_cast<float*>(workspace);
    float* records = ws;

    if (causal) {
        if (p.single) {
            int cus = 0;
            RACE_TRY(cu_count(&cus));
            RACE_TRY(marks->mark(stream));
            return launch_causal_single(probsQ, probsK, V, out, records,
                                        reinterpret_cast<int*>(records + l.records), state, init, p,
                                        cus, stream, marks);
        }
        if (mfma) {
            RACE_TRY(marks->mark(stream));
            return launch_causal_mfma(probsQ, probsK, V, out, records, state, p, stream, marks);
        }
        int lds_limit = 0;
        RACE_TRY(max_lds(&lds_limit));
        if (causal_output_valu_lds_bytes(p.S) > size_t(lds_limit)) return RACE_ERROR_INVALID_VALUE;
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_tile_outer_sums(probsK, V, records, p, p.S, p.d, stream));
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_tile_scan(records, state, p, stream));
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_causal_output_valu(probsQ, probsK, V, out, records, p, stream));
        return marks->mark(stream);
    }

    RACE_TRY(marks->mark(stream));
    RACE_TRY(outer_sums(probsK, V, records, p, p.S, p.d, stream));
    RACE_TRY(marks->mark(stream));
    const int64_t Sd = int64_t(p.S) * p.d;
    if (p.tiles > kFoldTiles) {
        float* E = records + l.records;
        RACE_TRY(launch_tile_reduce(records, state, E, p, stream));
        RACE_TRY(marks->mark(stream));
        // out = q . E: M[a][c] = E[a*d + c].
        RACE_TRY(token_map(probsQ, out, map_operand(E, Sd, p.d, 1), p, p.S, p.d, stream));
        return marks->mark(stream);
    }
    // out = q . E with E[s][c] = B[s][c] / (A[s] + eps), B and A the sums of
    // the tile records in tile order, formed as the map stages its matrix
    // (M[a = s][c]); the first token block's workgroups also write the
    // totals to the state when it is asked for.
    MapOperand op = map_operand(records, p.tiles * p.rec, p.d, 1);
    op.parts = int(p.tiles);
    op.part_stride = p.rec;
    op.div = records + Sd;
    op.div_stream = p.tiles * p.rec;
    op.save = state;
    op.save_stream = Sd + p.S;
    op.save_div_off = Sd;
    RACE_TRY(token_map(probsQ, out, op, p, p.S, p.d, stream));
    return marks->mark(stream);
}

// race_fwd_carry runs the decode kernel when asked to, and by default for
// calls of at most RACE_DECODE_TOKENS tokens that leave the tile length
// automatic; otherwise the causal tile path with the scan seeded from init.
bool carry_runs_decode(const race_shape* sh, const race_options* o) {
    const int k = kernel_choice(o);
    if (k == RACE_KERNEL_DECODE) return true;
    return k == RACE_KERNEL_AUTO && (!o || o->tile_tokens == 0) && sh->seq_len <= RACE_DECODE_TOKENS;
}

// The decode kernel has no tiles; a tile length, if given, must still be a
// valid one.
bool decode_options_ok(const race_options* o) {
    return !o || (o->tile_tokens >= 0 && o->tile_tokens % RACE_SUB_CHUNK_TOKENS == 0);
}

race_status carry_impl(const void* probsQ, const void* probsK, const void* V, void* out,
                       const float* init, float* state, const race_shape* shape,
                       const race_options* opts, void* workspace, size_t workspace_bytes,
                       hipStream_t stream, Marks* marks) {
    if (!shape || !init || !aligned16(init)) return RACE_ERROR_INVALID_VALUE;
    if (state && !aligned16(state)) return RACE_ERROR_INVALID_VALUE;
    if (!carry_runs_decode(shape, opts))
        return fwd_impl(probsQ, probsK, V, out, state, init, shape, 1, opts, workspace,
                        workspace_bytes, stream, marks);
    if (!shape_ok(shape) || !decode_options_ok(opts)) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    p.N = shape->num_streams;
    p.T = shape->seq_len;
    p.S = sub(shape);
    p.d = shape->head_dim;
    p.dtype = shape->dtype;
    p.kernel = RACE_KERNEL_DECODE;
    p.tile = 0;
    p.tiles = 0;
    p.rec = record_floats(p.S, p.d);
    p.init = init;
    if (p.N == 0 || (p.T == 0 && (!state || state == init))) {
        RACE_TRY(marks->mark(stream));
        return marks->mark(stream);
    }
    if (p.T > 0) {
        if (!probsQ || !probsK || !V || !out) return RACE_ERROR_INVALID_VALUE;
        if (!aligned16(probsQ) || !aligned16(probsK) || !aligned16(V) || !aligned16(out))
            return RACE_ERROR_INVALID_VALUE;
    }
    RACE_TRY(marks->mark(stream));
    RACE_TRY(launch_decode(probsQ, probsK, V, out, init, state, p, stream));
    return marks->mark(stream);
}

race_status noncausal_bwd_impl(const void* probsQ, const void* probsK, const void* V,
                               const void* dOut, const float* state, void* dQ, void* dK, void* dV,
                               const race_shape* shape, const race_options* opts, void* workspace,
                               size_t workspace_bytes, hipStream_t stream, Marks* marks) {
    Problem p;
    bool mfma = false;
    race_status st = make_problem(shape, 0, opts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    if (p.N == 0 || p.T == 0) return RACE_SUCCESS;
    if (!state || !dOut || !aligned16(state) || !aligned16(dOut)) return RACE_ERROR_INVALID_VALUE;
    if (dQ && !aligned16(dQ)) return RACE_ERROR_INVALID_VALUE;
    if ((dQ || dK || dV) && (!probsQ || !aligned16(probsQ))) return RACE_ERROR_INVALID_VALUE;
    if (dK && (!V || !aligned16(V) || !aligned16(dK))) return RACE_ERROR_INVALID_VALUE;
    if (dV && (!probsK || !aligned16(probsK) || !aligned16(dV))) return RACE_ERROR_INVALID_VALUE;
    if (!dQ && !dK && !dV) return RACE_SUCCESS;
    const BwdLayout l = bwd_layout(p);
    if (!workspace || !aligned16(workspace) || workspace_bytes < size_t(l.total()) * sizeof(float))
        return RACE_ERROR_INVALID_VALUE;
    float* records = static_cast<float*>(workspace);
    float* dB = records + l.records;
    float* dA = dB + l.dB;
    const int64_t Sd = int64_t(p.S) * p.d;
    const int64_t state_stride = Sd + p.S;

    RACE_TRY(marks->mark(stream));
    // S = d = 64: the query side (dQ and the dE records, dOut read once) and,
    // with both dK and dV asked for, the key side each in one pass; the key
    // side forms dB and dA itself from up to kKeyGradFoldParts records per
    // stream, after the finalize otherwise.
    const bool w64 = p.S == 64 && p.d == 64;
    if (w64 && dQ && (dK || dV)) {
        RACE_TRY(launch_query_grad64(probsQ, dOut, dQ, state, records, p, stream));
        RACE_TRY(marks->mark(stream));
    }
    if (w64 && dK && dV) {
        if (!dQ) {
            RACE_TRY(outer_sums(probsQ, dOut, records, p, p.S, p.d, stream));
            RACE_TRY(marks->mark(stream));
        }
        if (p.tiles <= kKeyGradFoldParts) {
            RACE_TRY(launch_key_grad64(probsK, V, dK, dV, records, state, nullptr, nullptr, p, stream));
        } else {
            RACE_TRY(launch_bwd_finalize(records, state, dB, dA, p, stream));
            RACE_TRY(marks->mark(stream));
            RACE_TRY(launch_key_grad64(probsK, V, dK, dV, nullptr, nullptr, dB, dA, p, stream));
        }
        return marks->mark(stream);
    }
    const bool dE_done = w64 && dQ && (dK || dV);
    // dQ = dOut E^T: M[a = c][b = s] = E[s*d + c] = B[s*d + c] / (A[s] + eps),
    // read straight from the state.
    if (dQ && !dE_done) {
        MapOperand op = map_operand(state, state_stride, 1, p.d);
        op.div = state + Sd;
        op.div_stream = state_stride;
        op.div_by_col = true;
        RACE_TRY(token_map(dOut, dQ, op, p, p.d, p.S, stream));
        RACE_TRY(marks->mark(stream));
    }
    if (!dK && !dV) return RACE_SUCCESS;
    // dE = Q^T dOut as per-tile partials; the finalize adds them in a fixed
    // order.
    if (!dE_done) {
        RACE_TRY(outer_sums(probsQ, dOut, records, p, p.S, p.d, stream));
        RACE_TRY(marks->mark(stream));
    }
    RACE_TRY(launch_bwd_finalize(records, state, dB, dA, p, stream));
    RACE_TRY(marks->mark(stream));
    // dK = V dB^T + dA: M[a = c][b = s] = dB[s*d + c].
    if (dK) {
        MapOperand op = map_operand(dB, Sd, 1, p.d);
        op.bias = dA;
        op.bias_stream = p.S;
        RACE_TRY(token_map(V, dK, op, p, p.d, p.S, stream));
        RACE_TRY(marks->mark(stream));
    }
    // dV = K dB: M[a = s][b = c] = dB[s*d + c].
    if (dV) {
        RACE_TRY(token_map(probsK, dV, map_operand(dB, Sd, p.d, 1), p, p.S, p.d, stream));
        RACE_TRY(marks->mark(stream));
    }
    return RACE_SUCCESS;
}


}  // namespace
}  // namespace race

extern "C" {

race_status race_fwd(const void* probsQ, const void* probsK, const void* V, void* out,
                     float* state, const race_shape* shape, int32_t causal,
                     const race_options* opts, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
    Marks none;
    return fwd_impl(probsQ, probsK, V, out, state, nullptr, shape, causal, opts, workspace,
                    workspace_bytes, stream, &none);
}

race_status race_fwd_profiled(const void* probsQ, const void* probsK, const void* V, void* out,
                              float* state, const race_shape* shape, int32_t causal,
                              const race_options* opts, void* workspace, size_t workspace_bytes,
                              hipStream_t stream, hipEvent_t* events, int32_t max_events,
                              int32_t* n_events) {
    if (!events || max_events < 2 || !n_events) return RACE_ERROR_INVALID_VALUE;
    Marks marks;
    marks.events = events;
    marks.max = max_events;
    const race_status st = fwd_impl(probsQ, probsK, V, out, state, nullptr, shape, causal, opts,
                                    workspace, workspace_bytes, stream, &marks);
    *n_events = marks.n;
    return st;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free forward: race_fwd with its workspace taken from `scratch`,
// one file-scope device array per GPU, alive until the process ends.  In host
// code the name `scratch` is a host-side stand-in, not a device address:
// host code only ever uses the address hipGetSymbolAddress returns for the
// current device (kept per device below), in kernel arguments and copies.
// Every call on one GPU shares that GPU's array and leaves its contents
// behind; race_fwd writes every record it later reads, so nothing needs
// clearing first.  Calls that overlap on one GPU (other streams, other host
// threads without ordering) race on the array.
static __device__ __align__(256) float scratch[RACE_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace race {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxScratchDevices] = {};

// The device address of the current GPU's scratch array, looked up once per
// device with that device current.
hipError_t current_scratch(void** addr) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return err;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_addr[dev] = p;
    }
    *addr = g_scratch_addr[dev];
    return hipSuccess;
}

}  // namespace
}  // namespace race

extern "C" {

race_status race_fwd_noalloc(const void* probsQ, const void* probsK, const void* V, void* out,
                             float* state, const race_shape* shape, int32_t causal,
                             const race_options* opts, hipStream_t stream) {
    // The size check is host arithmetic and comes first, so an oversized call
    // is refused before any device is touched.
    size_t need = 0;
    race_status st = race_fwd_workspace_bytes(shape, causal, opts, &need, nullptr, nullptr);
    if (st != RACE_SUCCESS) return st;
    if (need > size_t(RACE_NOALLOC_SCRATCH_BYTES)) return RACE_ERROR_SCRATCH_TOO_SMALL;
    void* ws = nullptr;
    const hipError_t err = current_scratch(&ws);
    if (err != hipSuccess) return err;
    Marks none;
    return fwd_impl(probsQ, probsK, V, out, state, nullptr, shape, causal, opts, ws,
                    size_t(RACE_NOALLOC_SCRATCH_BYTES), stream, &none);
}

race_status race_fwd_single_status(const race_shape* shape, const race_options* opts,
                                   const void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
    if (!opts || opts->kernel != RACE_KERNEL_SINGLE) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    bool mfma = false;
    race_status st = make_problem(shape, 1, opts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    if (p.N == 0 || p.T == 0) return RACE_SUCCESS;  // nothing was launched
    const FwdLayout l = fwd_layout(p, 1);
    if (!workspace) {
        void* ws = nullptr;
        RACE_TRY(current_scratch(&ws));
        workspace = ws;
        workspace_bytes = size_t(RACE_NOALLOC_SCRATCH_BYTES);
    }
    if (!aligned16(workspace) || workspace_bytes < size_t(l.total()) * sizeof(float))
        return RACE_ERROR_INVALID_VALUE;
    const int* words = reinterpret_cast<const int*>(static_cast<const float*>(workspace) + l.records);
    int word = 0;
    RACE_TRY(hipMemcpyAsync(&word, words + single_pass_error_word(p.N, p.tiles), sizeof(int),
                            hipMemcpyDeviceToHost, stream));
    RACE_TRY(hipStreamSynchronize(stream));
    return word != 0 ? RACE_ERROR_SINGLE_PASS_GAVE_UP : RACE_SUCCESS;
}

race_status race_single_pass_test_give_up(int32_t on) {
    single_pass_preset_give_up(on != 0);
    return RACE_SUCCESS;
}

race_status race_fwd_carry_workspace_bytes(const race_shape* shape, const race_options* opts,
                                           size_t* bytes) {
    if (!bytes || !shape) return RACE_ERROR_INVALID_VALUE;
    if (carry_runs_decode(shape, opts)) {
        if (!decode_options_ok(opts) || !shape_ok(shape)) return RACE_ERROR_INVALID_VALUE;
        *bytes = 0;
        return RACE_SUCCESS;
    }
    return race_fwd_workspace_bytes(shape, 1, opts, bytes, nullptr, nullptr);
}

race_status race_fwd_carry(const void* probsQ, const void* probsK, const void* V, void* out,
                           const float* init_state, float* state, const race_shape* shape,
                           const race_options* opts, void* workspace, size_t workspace_bytes,
                           hipStream_t stream) {
    Marks none;
    return carry_impl(probsQ, probsK, V, out, init_state, state, shape, opts, workspace,
                      workspace_bytes, stream, &none);
}

race_status race_fwd_carry_profiled(const void* probsQ, const void* probsK, const void* V,
                                    void* out, const float* init_state, float* state,
                                    const race_shape* shape, const race_options* opts,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream,
                                    hipEvent_t* events, int32_t max_events, int32_t* n_events) {
    if (!events || max_events < 2 || !n_events) return RACE_ERROR_INVALID_VALUE;
    Marks marks;
    marks.events = events;
    marks.max = max_events;
    const race_status st = carry_impl(probsQ, probsK, V, out, init_state, state, shape, opts,
                                      workspace, workspace_bytes, stream, &marks);
    *n_events = marks.n;
    return st;
}

race_status race_noncausal_bwd_workspace_bytes(const race_shape* shape, const race_options* opts,
                                               size_t* bytes) {
    if (!bytes) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    bool mfma = false;
    const race_status st = make_problem(shape, 0, opts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    *bytes = size_t(bwd_layout(p).total()) * sizeof(float);
    return RACE_SUCCESS;
}

race_status race_noncausal_bwd(const void* probsQ, const void* probsK, const void* V,
                               const void* dOut, const float* state, void* dQ, void* dK, void* dV,
                               const race_shape* shape, const race_options* opts, void* workspace,
                               size_t workspace_bytes, hipStream_t stream) {
    Marks none;
    return noncausal_bwd_impl(probsQ, probsK, V, dOut, state, dQ, dK, dV, shape, opts, workspace,
                              workspace_bytes, stream, &none);
}

race_status race_noncausal_bwd_profiled(const void* probsQ, const void* probsK, const void* V,
                                        const void* dOut, const float* state, void* dQ, void* dK,
                                        void* dV, const race_shape* shape,
                                        const race_options* opts, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream,
                                        hipEvent_t* events, int32_t max_events,
                                        int32_t* n_events) {
    if (!events || max_events < 2 || !n_events) return RACE_ERROR_INVALID_VALUE;
    Marks marks;
    marks.events = events;
    marks.max = max_events;
    const race_status st = noncausal_bwd_impl(probsQ, probsK, V, dOut, state, dQ, dK, dV, shape,
                                              opts, workspace, workspace_bytes, stream, &marks);
    *n_events = marks.n;
    return st;
}

}  // extern "C"

namespace race {
namespace {

race_status causal_bwd_impl(const void* probsQ, const void* probsK, const void* V,
                            const void* dOut, const float* fwd_records, void* dQ, void* dK,
                            void* dV, const race_shape* shape, const race_options* opts,
                            void* workspace, size_t workspace_bytes, hipStream_t stream,
                            Marks* marks) {
    // The tile policy is the vector-ALU one; the kernel family is chosen here.
    const int kernel = kernel_choice(opts);
    if (!bwd_kernel_ok(kernel)) return RACE_ERROR_INVALID_VALUE;
    race_options topts = {opts ? opts->tile_tokens : 0, RACE_KERNEL_VALU};
    Problem p;
    bool mfma = false;
    race_status st = make_problem(shape, 0, &topts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    const CausalBwdPlan pl = plan_causal_bwd(p, kernel);
    const bool use_mfma = pl.mfma;
    if (kernel == RACE_KERNEL_MFMA && !use_mfma) return RACE_ERROR_INVALID_VALUE;
    // Saved forward records come with the forward's (explicit) tile length.
    if (fwd_records && (!opts || opts->tile_tokens <= 0 || !aligned16(fwd_records)))
        return RACE_ERROR_INVALID_VALUE;
    if (p.N == 0 || p.T == 0 || (!dQ && !dK && !dV)) return RACE_SUCCESS;
    if (!probsQ || !probsK || !V || !dOut) return RACE_ERROR_INVALID_VALUE;
    if (!aligned16(probsQ) || !aligned16(probsK) || !aligned16(V) || !aligned16(dOut))
        return RACE_ERROR_INVALID_VALUE;
    if ((dQ && !aligned16(dQ)) || (dK && !aligned16(dK)) || (dV && !aligned16(dV)))
        return RACE_ERROR_INVALID_VALUE;
    const int groups = pl.groups, C = pl.C;
    const CausalBwdLayout l = causal_bwd_layout(p, fwd_records != nullptr, pl);
    if (!workspace || !aligned16(workspace) || workspace_bytes < size_t(l.total()) * sizeof(float))
        return RACE_ERROR_INVALID_VALUE;
    if (groups == 0) return RACE_ERROR_INVALID_VALUE;
    float* bwd_rec = static_cast<float*>(workspace);
    float* apre = bwd_rec + l.bwd;
    float* dq32 = apre + l.apre;
    float* fwd_ws = dq32 + l.dq32;
    float* acc = fwd_ws + l.fwd;
    // B3 reads dQ back in fp32.  With one column group (or block) an fp32 dQ
    // is that copy: B1 writes it once, into the caller's buffer, and B3 reads
    // it from there.  With several, dq32 holds the current group's part.
    void* dq_out = dQ;
    if (dQ && p.dtype == RACE_F32 && groups == 1 && !pl.blocked()) {
        dq32 = static_cast<float*>(dQ);
        dq_out = nullptr;
    }

    // The bf16 128 x 128 block walks can start every stream at its first
    // token instead: when the streams times the blocks cover the CUs (one
    // forward-walk workgroup per CU fits) or a stream is one tile, each
    // forward walk goes through its whole stream, its prefix carried from
    // zero, and the forward's tile sums and scan are skipped.  At the cfg5
    // shape (N = 128, S = 256, 4 tiles) the step from the inputs went from
    // 3.49-3.50 to 3.21-3.23 ms (one box), the walks taking the same time as
    // tile by tile.  Saved records are then not read either.
    bool whole_streams = false;
    if (use_mfma && pl.wide2()) {
        int cus = 0;
        RACE_TRY(cu_count(&cus));
        whole_streams = p.tiles == 1 || p.N * (pl.mblocks / 2) >= cus;
    }
    // Prefix state at every tile start: the saved forward records, or the
    // forward's tile totals and scan again.
    RACE_TRY(marks->mark(stream));
    const float* fwd_rec = fwd_records;
    if (!fwd_rec && !whole_streams) {
        if (direct_sums_supported(p.S, p.d) && p.tile % 64 == 0)
            RACE_TRY(launch_tile_sums_direct(probsK, V, fwd_ws, p, stream));
        else if (mfma_causal_supported(p.S, p.d))
            RACE_TRY(launch_tile_sums_mfma(probsK, V, fwd_ws, p, stream));
        else
            RACE_TRY(launch_tile_outer_sums(probsK, V, fwd_ws, p, p.S, p.d, stream));
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_tile_scan(fwd_ws, nullptr, p, stream));
        RACE_TRY(marks->mark(stream));
        fwd_rec = fwd_ws;
    }
    if (use_mfma && !pl.blocked()) {
        const BwdBlock blk = single_block(p);
        RACE_TRY(launch_causal_bwd_dq_mfma(probsQ, probsK, V, dOut, dq_out, dq32, apre, fwd_rec,
                                           bwd_rec, p, blk, stream));
        RACE_TRY(marks->mark(stream));
        if (!dK && !dV) return RACE_SUCCESS;
        RACE_TRY(launch_tile_scan(bwd_rec, nullptr, p, stream, /*reverse=*/true));
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_causal_bwd_dkv_mfma(probsQ, probsK, V, dOut, dq32, apre, bwd_rec, dK, dV, p,
                                            blk, stream));
        return marks->mark(stream);
    }
    if (use_mfma) {
        // 64 x 64 blocks, bucket group m outer and value group h inner: dQ and
        // dK of group m are summed over h, dV of group h over m, in that fixed
        // order, in fp32 (the fp32 outputs themselves, or workspace for bf16
        // outputs, whose last addend writes the caller's buffers), inside the
        // kernels.
        Problem pb = p;
        pb.S = pb.d = 64;
        pb.rec = record_floats(64, 64);
        const bool f32 = p.dtype == RACE_F32;
        const int64_t es = f32 ? 4 : 2, NT = p.N * p.T;
        // bf16 running sums in the workspace: dQ (not for a walk over every
        // value column, whose dQ is whole), then dK, then dV.
        const int64_t q_sum = pl.wide() ? 0 : round64(NT * p.S);
        float* acc_q = f32 ? static_cast<float*>(dQ) : (dQ && !pl.wide() ? acc : nullptr);
        float* acc_k = f32 ? static_cast<float*>(dK) : (dK ? acc + q_sum : nullptr);
        float* acc_v = f32 ? static_cast<float*>(dV) : (dV ? acc + q_sum + round64(NT * p.S) : nullptr);
        auto col = [](void* base, int64_t c, int64_t es_) -> void* {
            return base ? static_cast<void*>(static_cast<char*>(base) + c * es_) : nullptr;
        };
        if (pl.wide2()) {
            // Per pair of bucket groups (buckets 128 mp ..): a forward walk
            // over its 128 buckets and every value column (its dQ whole,
            // straight to the caller's dQ; the suffix records of its four
            // 64 x 64 blocks), all pairs in one launch; one reverse scan of
            // every pair's records; then per pair a backward walk over the
            // same block: dK of its buckets whole, dV added to its running
            // sum over the pairs in pair order (the last pair writes the
            // caller's dV).
            const int pairs = pl.mblocks / 2;
            const int64_t rec_n = p.N * p.tiles * pb.rec;
            // The dq32 region holds dQ's bf16 remainders [pairs][N T][128]
            // and, when dQ is not asked for, its bf16 part after them.
            bf16_t* dq_lo_ws = reinterpret_cast<bf16_t*>(dq32);
            bf16_t* dq_hi_ws = dq_lo_ws + pairs * NT * 128;
            DqWidePairs pp;
            pp.pairs = pairs;
            pp.hi_ps = dQ ? 128 : NT * 128;  // the caller's dQ: the pair's first column
            pp.lo_ps = NT * 128;
            pp.ap_ps = wide_apre_floats(p);
            pp.rec_ps = 4 * rec_n;
            pp.whole = whole_streams ? 1 : 0;
            void* dq_hi0 = dQ ? dQ : static_cast<void*>(dq_hi_ws);
            const int ld_hi = dQ ? p.S : 128;
            RACE_TRY(launch_causal_bwd_dq_wide(probsQ, probsK, V, dOut, dq_hi0, ld_hi, dK || dV ? dq_lo_ws : nullptr,
                                               apre, fwd_rec, bwd_rec, p, 0, pp, stream));
            RACE_TRY(marks->mark(stream));
            if (!dK && !dV) return RACE_SUCCESS;
            Problem p4 = pb;
            p4.N = pairs * 4 * p.N;
            RACE_TRY(scan_suffix_records(bwd_rec, p4, stream));
            RACE_TRY(marks->mark(stream));
            for (int mp = 0; mp < pairs; ++mp) {
                BwdWide wb;
                wb.ldq = p.S;
                wb.dq_hi = static_cast<const bf16_t*>(dq_hi0) + mp * pp.hi_ps;
                wb.ld_hi = ld_hi;
                wb.dq_lo = dq_lo_ws + mp * pp.lo_ps;
                wb.apre = apre + mp * pp.ap_ps;
                for (int g2 = 0; g2 < 2; ++g2) {
                    wb.rec[g2][0] = bwd_rec + mp * pp.rec_ps + (2 * g2) * rec_n;
                    wb.rec[g2][1] = bwd_rec + mp * pp.rec_ps + (2 * g2 + 1) * rec_n;
                }
                wb.acc_v = dV && pairs > 1 ? acc : nullptr;
                wb.v_first = mp == 0;
                wb.fin_v = mp == pairs - 1 ? dV : nullptr;
                RACE_TRY(launch_causal_bwd_dkv_wide(static_cast<const char*>(probsQ) + 128 * mp * es,
                                                    static_cast<const char*>(probsK) + 128 * mp * es, V, dOut,
                                                    col(dK, 128 * mp, es), p, wb, stream));
                RACE_TRY(marks->mark(stream));
            }
            return RACE_SUCCESS;
        }
        if (pl.wide()) {
            // Per bucket group m: one forward walk over all 128 value columns
            // (dQ of group m whole, straight to the caller's dQ; the suffix
            // records of both value groups), one reverse scan of both record
            // arrays, then the backward walk of each value group, the terms
            // of alpha in group 0's.
            Problem p2 = pb;
            p2.N = 2 * p.N;  // both groups' records, scanned as 2N streams
            float* rec_h[2] = {bwd_rec, bwd_rec + p.N * p.tiles * pb.rec};
            for (int m = 0; m < pl.mblocks; ++m) {
                const bool last_m = m == pl.mblocks - 1;
                const void* qb = static_cast<const char*>(probsQ) + 64 * m * es;
                const void* kb = static_cast<const char*>(probsK) + 64 * m * es;
                BwdBlock b1;
                b1.ldq = p.S;
                b1.ldv = p.d;
                b1.s0 = 64 * m;
                b1.c0 = 0;
                b1.fwd_d = p.d;
                b1.fwd_a = int64_t(p.S) * p.d;
                b1.fwd_rec = p.rec;
                b1.blocked = 1;
                b1.acc_q = nullptr;  // dQ of group m is whole: written straight to the caller's dQ
                b1.q_first = 1;
                b1.fin_q = col(dQ, 64 * m, es);
                RACE_TRY(launch_causal_bwd_dq_mfma(qb, kb, V, dOut, nullptr, dq32, apre, fwd_rec, bwd_rec,
                                                   pb, b1, stream, 128));
                RACE_TRY(marks->mark(stream));
                if (!dK && !dV) continue;
                RACE_TRY(scan_suffix_records(bwd_rec, p2, stream));
                RACE_TRY(marks->mark(stream));
                for (int h = 0; h < 2; ++h) {
                    BwdBlock blk = b1;
                    blk.c0 = 64 * h;
                    blk.acc_q = nullptr;
                    blk.fin_q = nullptr;
                    blk.acc_k = acc_k ? acc_k + 64 * m : nullptr;
                    blk.acc_v = acc_v ? acc_v + 64 * h : nullptr;
                    blk.k_first = h == 0;
                    blk.v_first = m == 0;
                    blk.fin_k = h == 1 ? col(dK, 64 * m, es) : nullptr;
                    blk.fin_v = last_m ? col(dV, 64 * h, es) : nullptr;
                    blk.alpha = h == 0;
                    const void* vb = static_cast<const char*>(V) + 64 * h * es;
                    const void* gb = static_cast<const char*>(dOut) + 64 * h * es;
                    RACE_TRY(launch_causal_bwd_dkv_mfma(qb, kb, vb, gb, dq32, apre, rec_h[h], nullptr,
                                                        nullptr, pb, blk, stream));
                    RACE_TRY(marks->mark(stream));
                }
            }
            return RACE_SUCCESS;
        }
        for (int m = 0; m < pl.mblocks; ++m) {
            for (int h = 0; h < pl.hblocks; ++h) {
                const bool last_h = h == pl.hblocks - 1, last_m = m == pl.mblocks - 1;
                BwdBlock blk;
                blk.ldq = p.S;
                blk.ldv = p.d;
                blk.s0 = 64 * m;
                blk.c0 = 64 * h;
                blk.fwd_d = p.d;
                blk.fwd_a = int64_t(p.S) * p.d;
                blk.fwd_rec = p.rec;
                blk.blocked = 1;
                blk.acc_q = acc_q ? acc_q + 64 * m : nullptr;
                blk.acc_k = acc_k ? acc_k + 64 * m : nullptr;
                blk.acc_v = acc_v ? acc_v + 64 * h : nullptr;
                blk.q_first = h == 0;
                blk.k_first = h == 0;
                blk.v_first = m == 0;
                if (!f32) {
                    blk.fin_q = last_h ? col(dQ, 64 * m, es) : nullptr;
                    blk.fin_k = last_h ? col(dK, 64 * m, es) : nullptr;
                    blk.fin_v = last_m ? col(dV, 64 * h, es) : nullptr;
                }
                const void* qb = static_cast<const char*>(probsQ) + 64 * m * es;
                const void* kb = static_cast<const char*>(probsK) + 64 * m * es;
                const void* vb = static_cast<const char*>(V) + 64 * h * es;
                const void* gb = static_cast<const char*>(dOut) + 64 * h * es;
                RACE_TRY(launch_causal_bwd_dq_mfma(qb, kb, vb, gb, nullptr, dq32, apre, fwd_rec, bwd_rec,
                                                   pb, blk, stream));
                RACE_TRY(marks->mark(stream));
                if (!dK && !dV) continue;
                RACE_TRY(launch_tile_scan(bwd_rec, nullptr, pb, stream, /*reverse=*/true));
                RACE_TRY(marks->mark(stream));
                RACE_TRY(launch_causal_bwd_dkv_mfma(qb, kb, vb, gb, dq32, apre, bwd_rec, nullptr, nullptr,
                                                    pb, blk, stream));
                RACE_TRY(marks->mark(stream));
            }
        }
        return RACE_SUCCESS;
    }
    if (groups == 1) {
        const BwdCols cols = all_columns(p);
        RACE_TRY(launch_causal_bwd_dq(probsQ, probsK, V, dOut, dq_out, dq32, apre, fwd_rec, bwd_rec,
                                      p, C, cols, stream));
        RACE_TRY(marks->mark(stream));
        if (!dK && !dV) return RACE_SUCCESS;
        RACE_TRY(launch_tile_scan(bwd_rec, nullptr, p, stream, /*reverse=*/true));
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_causal_bwd_dkv(probsQ, probsK, V, dOut, dq32, apre, bwd_rec, dK, dV, p, C,
                                       cols, stream));
        return marks->mark(stream);
    }
    // Column groups, in order: each adds its dQ and dK to the fp32 running
    // sums (the fp32 outputs themselves, or workspace for bf16 outputs, whose
    // last group then writes the caller's buffers).
    Problem pg = p;
    pg.d = p.d / groups;
    pg.rec = record_floats(p.S, pg.d);
    const bool f32 = p.dtype == RACE_F32;
    const int64_t es = f32 ? 4 : 2;
    float* acc_q = f32 ? static_cast<float*>(dQ) : (dQ ? acc : nullptr);
    float* acc_k = f32 ? static_cast<float*>(dK) : (dK ? acc + round64(p.N * p.T * int64_t(p.S)) : nullptr);
    for (int gi = 0; gi < groups; ++gi) {
        const bool first = gi == 0, last = gi == groups - 1;
        BwdCols cols;
        cols.ld = p.d;
        cols.c0 = gi * pg.d;
        cols.fwd_d = p.d;
        cols.fwd_rec = p.rec;
        cols.acc_q_in = first ? nullptr : acc_q;
        cols.acc_q_out = (!f32 && last) ? nullptr : acc_q;
        cols.acc_k_in = first ? nullptr : acc_k;
        cols.acc_k_out = (!f32 && last) ? nullptr : acc_k;
        void* dq_t = (!f32 && last) ? dQ : nullptr;
        void* dk_t = (!f32 && last) ? dK : nullptr;
        const int64_t off = int64_t(cols.c0) * es;
        const void* vg = static_cast<const char*>(V) + off;
        const void* gg = static_cast<const char*>(dOut) + off;
        void* dvg = dV ? static_cast<void*>(static_cast<char*>(dV) + off) : nullptr;
        RACE_TRY(launch_causal_bwd_dq(probsQ, probsK, vg, gg, dq_t, dq32, apre, fwd_rec, bwd_rec, pg,
                                      C, cols, stream));
        RACE_TRY(marks->mark(stream));
        if (!dK && !dV) continue;
        RACE_TRY(launch_tile_scan(bwd_rec, nullptr, pg, stream, /*reverse=*/true));
        RACE_TRY(marks->mark(stream));
        RACE_TRY(launch_causal_bwd_dkv(probsQ, probsK, vg, gg, dq32, apre, bwd_rec, dk_t, dvg, pg, C,
                                       cols, stream));
        RACE_TRY(marks->mark(stream));
    }
    return RACE_SUCCESS;
}


}  // namespace
}  // namespace race

extern "C" {

race_status race_causal_bwd_workspace_bytes(const race_shape* shape, const race_options* opts,
                                            size_t* bytes) {
    if (!bytes || !bwd_kernel_ok(kernel_choice(opts))) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    bool mfma = false;
    // The backward uses the vector-ALU tile policy for both kernel families.
    race_options topts = {opts ? opts->tile_tokens : 0, RACE_KERNEL_VALU};
    const race_status st = make_problem(shape, 0, &topts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    *bytes = size_t(causal_bwd_layout(p, false, plan_causal_bwd(p, kernel_choice(opts))).total()) *
             sizeof(float);
    return RACE_SUCCESS;
}

race_status race_causal_bwd_from_records_workspace_bytes(const race_shape* shape,
                                                         const race_options* opts, size_t* bytes) {
    if (!bytes || !opts || opts->tile_tokens <= 0 || !bwd_kernel_ok(opts->kernel)) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    bool mfma = false;
    race_options topts = {opts->tile_tokens, RACE_KERNEL_VALU};
    const race_status st = make_problem(shape, 0, &topts, &mfma, &p);
    if (st != RACE_SUCCESS) return st;
    *bytes = size_t(causal_bwd_layout(p, true, plan_causal_bwd(p, kernel_choice(opts))).total()) *
             sizeof(float);
    return RACE_SUCCESS;
}

race_status race_causal_bwd(const void* probsQ, const void* probsK, const void* V,
                            const void* dOut, void* dQ, void* dK, void* dV,
                            const race_shape* shape, const race_options* opts, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
    Marks none;
    return causal_bwd_impl(probsQ, probsK, V, dOut, nullptr, dQ, dK, dV, shape, opts, workspace,
                           workspace_bytes, stream, &none);
}

race_status race_causal_bwd_from_records(const void* probsQ, const void* probsK, const void* V,
                                         const void* dOut, const float* fwd_records, void* dQ,
                                         void* dK, void* dV, const race_shape* shape,
                                         const race_options* opts, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream) {
    Marks none;
    if (!fwd_records) return RACE_ERROR_INVALID_VALUE;
    return causal_bwd_impl(probsQ, probsK, V, dOut, fwd_records, dQ, dK, dV, shape, opts,
                           workspace, workspace_bytes, stream, &none);
}

race_status race_causal_bwd_profiled(const void* probsQ, const void* probsK, const void* V,
                                     const void* dOut, void* dQ, void* dK, void* dV,
                                     const race_shape* shape, const race_options* opts,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream,
                                     hipEvent_t* events, int32_t max_events, int32_t* n_events) {
    if (!events || max_events < 2 || !n_events) return RACE_ERROR_INVALID_VALUE;
    Marks marks;
    marks.events = events;
    marks.max = max_events;
    const race_status st = causal_bwd_impl(probsQ, probsK, V, dOut, nullptr, dQ, dK, dV, shape, opts,
                                           workspace, workspace_bytes, stream, &marks);
    *n_events = marks.n;
    return st;
}

}  // extern "C"

extern "C" {

race_status race_hash_probs(const void* x, const float* planes_T, void* probs, int64_t rows,
                            int32_t head_dim, int32_t num_tables, int32_t planes_per_table,
                            int32_t dtype, hipStream_t stream) {
    if (!hash_shape_ok(rows, head_dim, num_tables, planes_per_table)) return RACE_ERROR_INVALID_VALUE;
    if (dtype != RACE_F32 && dtype != RACE_BF16) return RACE_ERROR_INVALID_VALUE;
    if (rows == 0) return RACE_SUCCESS;
    if (!x || !planes_T || !probs) return RACE_ERROR_INVALID_VALUE;
    if (!aligned16(x) || !aligned16(planes_T) || !aligned16(probs)) return RACE_ERROR_INVALID_VALUE;
    int lds_limit = 0;
    RACE_TRY(max_lds(&lds_limit));
    if (hash_lds_bytes(head_dim, num_tables, planes_per_table) > size_t(lds_limit))
        return RACE_ERROR_INVALID_VALUE;
    return launch_hash_probs(x, planes_T, probs, rows, head_dim, num_tables, planes_per_table,
                             dtype, stream);
}

race_status race_hash_probs_bwd(const void* x, const float* planes_T, const void* dprobs, void* dx,
                                int64_t rows, int32_t head_dim, int32_t num_tables,
                                int32_t planes_per_table, int32_t dtype, hipStream_t stream) {
    if (!hash_shape_ok(rows, head_dim, num_tables, planes_per_table)) return RACE_ERROR_INVALID_VALUE;
    if (dtype != RACE_F32 && dtype != RACE_BF16) return RACE_ERROR_INVALID_VALUE;
    if (rows == 0) return RACE_SUCCESS;
    if (!x || !planes_T || !dprobs || !dx) return RACE_ERROR_INVALID_VALUE;
    const int tier = num_tables * planes_per_table <= 16 ? 16 : num_tables * planes_per_table <= 32 ? 32 : 64;
    int lds_limit = 0;
    RACE_TRY(max_lds(&lds_limit));
    if (size_t(head_dim) * tier * sizeof(float) > size_t(lds_limit)) return RACE_ERROR_INVALID_VALUE;
    return launch_hash_probs_bwd(x, planes_T, dprobs, dx, rows, head_dim, num_tables,
                                 planes_per_table, dtype, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The causal op with the hashing inside (hashed_causal.hip): the fused
// forward of src/race_fused_fwd.cu:150-171, race_fused_fwd(K, Q, V, planes, L).

namespace race {
namespace {

// The problem of a hashed call: R = 2^K buckets per table, the workgroup MFMA
// kernels' tile policy.
race_status hashed_problem(const race_shape* sh, int32_t K, const race_options* o, Problem* p) {
    if (!shape_ok(sh)) return RACE_ERROR_INVALID_VALUE;
    if (K < 1 || K > 8 || sh->num_buckets != (1 << K)) return RACE_ERROR_INVALID_VALUE;
    if (!hashed_causal_supported(sh->num_tables, K, sh->head_dim)) return RACE_ERROR_INVALID_VALUE;
    const int k = kernel_choice(o);
    if (k != RACE_KERNEL_AUTO && k != RACE_KERNEL_MFMA && k != RACE_KERNEL_MFMA_WG)
        return RACE_ERROR_INVALID_VALUE;
    const race_options wg = {o ? o->tile_tokens : 0, RACE_KERNEL_MFMA_WG};
    bool mfma = false;
    return make_problem(sh, 1, &wg, &mfma, p);
}

race_status hashed_fwd_impl(const void* k_rows, const void* q_rows, const void* v, const float* planes,
                            void* out, float* state, const race_shape* shape, int32_t K,
                            const race_options* opts, void* workspace, size_t workspace_bytes,
                            hipStream_t stream, Marks* marks) {
    Problem p;
    const race_status st = hashed_problem(shape, K, opts, &p);
    if (st != RACE_SUCCESS) return st;
    if (state && !aligned16(state)) return RACE_ERROR_INVALID_VALUE;
    if (p.N == 0 || p.T == 0) {
        RACE_TRY(marks->mark(stream));
        RACE_TRY(zero_fill(state, p.N * state_floats(p.S, p.d), stream));
        return marks->mark(stream);
    }
    if (!k_rows || !q_rows || !v || !planes || !out) return RACE_ERROR_INVALID_VALUE;
    if (!aligned16(k_rows) || !aligned16(q_rows) || !aligned16(v) || !aligned16(planes) ||
        !aligned16(out))
        return RACE_ERROR_INVALID_VALUE;
    const FwdLayout l = fwd_layout(p, 1);
    if (!workspace || !aligned16(workspace) || workspace_bytes < size_t(l.total()) * sizeof(float))
        return RACE_ERROR_INVALID_VALUE;
    HashedArgs a;
    a.q = q_rows;
    a.k = k_rows;
    a.v = v;
    a.planes = planes;
    a.out = out;
    a.records = static_cast<float*>(workspace);
    a.state = state;
    a.L = shape->num_tables;
    a.K = K;
    RACE_TRY(marks->mark(stream));
    return launch_hashed_causal(a, p, stream, marks);
}

}  // namespace
}  // namespace race

extern "C" {

race_status race_hashed_fwd_workspace_bytes(const race_shape* shape, int32_t planes_per_table,
                                            const race_options* opts, size_t* bytes, int64_t* tiles,
                                            int64_t* record_floats_out) {
    if (!bytes) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    const race_status st = hashed_problem(shape, planes_per_table, opts, &p);
    if (st != RACE_SUCCESS) return st;
    *bytes = size_t(fwd_layout(p, 1).total()) * sizeof(float);
    if (tiles) *tiles = p.tiles;
    if (record_floats_out) *record_floats_out = p.rec;
    return RACE_SUCCESS;
}

race_status race_hashed_fwd(const void* k_rows, const void* q_rows, const void* v, const float* planes,
                            void* out, float* state, const race_shape* shape, int32_t planes_per_table,
                            const race_options* opts, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    Marks none;
    return hashed_fwd_impl(k_rows, q_rows, v, planes, out, state, shape, planes_per_table, opts,
                           workspace, workspace_bytes, stream, &none);
}

race_status race_hashed_fwd_profiled(const void* k_rows, const void* q_rows, const void* v,
                                     const float* planes, void* out, float* state,
                                     const race_shape* shape, int32_t planes_per_table,
                                     const race_options* opts, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream, hipEvent_t* events,
                                     int32_t max_events, int32_t* n_events) {
    if (!events || max_events < 2 || !n_events) return RACE_ERROR_INVALID_VALUE;
    Marks marks;
    marks.events = events;
    marks.max = max_events;
    const race_status st = hashed_fwd_impl(k_rows, q_rows, v, planes, out, state, shape,
                                           planes_per_table, opts, workspace, workspace_bytes, stream,
                                           &marks);
    *n_events = marks.n;
    return st;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Algorithm 1 with the hashing inside (alg1.hip), the reference's causal v2
// forward (src/causal_v2/kernels/race_causal_fwd.h:110-130).

namespace race {
namespace {

constexpr int kAlg1Chunk = RACE_ALG1_SUB_CHUNK_TOKENS;

bool alg1_shape_valid(const race_alg1_shape* sh) {
    if (!sh) return false;
    if (sh->batch_heads < 0 || sh->batch_heads > kMaxStreams) return false;
    if (sh->seq_len < 0 || sh->seq_len > int64_t(INT_MAX) - RACE_ALG1_MAX_AUTO_TILE - 1) return false;
    return alg1_shape_ok(sh->head_dim, sh->num_planes, sh->num_tables);
}

// Tile length: a few resident output-pass workgroups per CU, never below
// the sub-chunk and never above RACE_ALG1_MAX_AUTO_TILE (the reference's
// policy, race_causal_fwd.h:90-95, with this device's CU count).
race_status alg1_resolve_tile(const race_alg1_shape* sh, int variant, int32_t requested, int* tile) {
    if (requested != 0) {
        if (requested < 0 || requested % kAlg1Chunk != 0) return RACE_ERROR_INVALID_VALUE;
        *tile = requested;
        return RACE_SUCCESS;
    }
    const int64_t work = sh->batch_heads * sh->seq_len;
    if (work == 0) {
        *tile = kAlg1Chunk;
        return RACE_SUCCESS;
    }
    int cus = 0;
    RACE_TRY(cu_count(&cus));
    if (cus < 1) cus = 1;
    const int64_t per_cu =
        2 * int64_t(alg1_blocks_per_cu(sh->head_dim, sh->num_planes, sh->num_tables, variant));
    int t = pow2_floor(work / (per_cu * cus));
    if (t < kAlg1Chunk) t = kAlg1Chunk;
    if (t > RACE_ALG1_MAX_AUTO_TILE) t = RACE_ALG1_MAX_AUTO_TILE;
    *tile = t;
    return RACE_SUCCESS;
}

race_status alg1_problem(const race_alg1_shape* sh, int32_t variant, int32_t tile_tokens,
                         Problem* p) {
    if (!alg1_shape_valid(sh)) return RACE_ERROR_INVALID_VALUE;
    if (variant != RACE_ALG1_FP32 && variant != RACE_ALG1_BF16) return RACE_ERROR_INVALID_VALUE;
    int tile = 0;
    const race_status st = alg1_resolve_tile(sh, variant, tile_tokens, &tile);
    if (st != RACE_SUCCESS) return st;
    if (!tile_fits_buffer(tile, sh->head_dim, 2)) return RACE_ERROR_INVALID_VALUE;
    p->N = sh->batch_heads;
    p->T = sh->seq_len;
    p->S = sh->num_tables << sh->num_planes;
    p->d = sh->head_dim;
    p->dtype = RACE_BF16;
    p->kernel = RACE_KERNEL_MFMA;
    p->tile = tile;
    p->tiles = sh->seq_len == 0 ? 0 : (sh->seq_len + tile - 1) / tile;
    p->rec = record_floats(p->S, p->d);
    return RACE_SUCCESS;
}

race_status alg1_fwd_impl(const void* q, const void* k, const void* v, const float* W,
                          const float* beta, void* out, const float* init, float* final_state,
                          const race_alg1_shape* sh, int32_t tile_tokens, int32_t variant,
                          void* workspace, size_t workspace_bytes, hipStream_t stream,
                          Marks* marks) {
    Problem p;
    const race_status st = alg1_problem(sh, variant, tile_tokens, &p);
    if (st != RACE_SUCCESS) return st;
    if (final_state && !aligned16(final_state)) return RACE_ERROR_INVALID_VALUE;
    if (init && !aligned16(init)) return RACE_ERROR_INVALID_VALUE;
    p.init = init;
    if (p.N == 0 || p.T == 0) {
        RACE_TRY(marks->mark(stream));
        if (init)
            RACE_TRY(copy_floats(init, final_state, p.N * state_floats(p.S, p.d), stream));
        else
            RACE_TRY(zero_fill(final_state, p.N * state_floats(p.S, p.d), stream));
        return marks->mark(stream);
    }
    if (!q || !k || !v || !W || !beta || !out) return RACE_ERROR_INVALID_VALUE;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !aligned16(W))
        return RACE_ERROR_INVALID_VALUE;
    const size_t need = size_t(p.N * p.tiles * p.rec) * sizeof(float);
    if (!workspace || !aligned16(workspace) || workspace_bytes < need) return RACE_ERROR_INVALID_VALUE;
    int lds_limit = 0;
    RACE_TRY(max_lds(&lds_limit));
    if (alg1_output_lds_bytes(p.d, sh->num_planes, sh->num_tables, variant) > size_t(lds_limit))
        return RACE_ERROR_INVALID_VALUE;
    Alg1Args a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.W = W;
    a.beta = beta;
    a.out = out;
    a.records = static_cast<float*>(workspace);
    a.state = final_state;
    a.L = sh->num_tables;
    a.P = sh->num_planes;
    RACE_TRY(marks->mark(stream));
    return launch_alg1(a, p, variant, stream, marks);
}

}  // namespace
}  // namespace race

extern "C" {

race_status race_alg1_shape_supported(const race_alg1_shape* shape, int32_t* supported) {
    if (!shape || !supported) return RACE_ERROR_INVALID_VALUE;
    *supported = alg1_shape_valid(shape) ? 1 : 0;
    return RACE_SUCCESS;
}

race_status race_alg1_output_lds_bytes(const race_alg1_shape* shape, int32_t variant,
                                       size_t* bytes) {
    if (!bytes || !alg1_shape_valid(shape)) return RACE_ERROR_INVALID_VALUE;
    if (variant != RACE_ALG1_FP32 && variant != RACE_ALG1_BF16) return RACE_ERROR_INVALID_VALUE;
    *bytes = alg1_output_lds_bytes(shape->head_dim, shape->num_planes, shape->num_tables, variant);
    return RACE_SUCCESS;
}

race_status race_alg1_select_tile_tokens(const race_alg1_shape* shape, int32_t variant,
                                         int32_t* tile_tokens) {
    if (!tile_tokens) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    const race_status st = alg1_problem(shape, variant, 0, &p);
    if (st != RACE_SUCCESS) return st;
    *tile_tokens = p.tile;
    return RACE_SUCCESS;
}

race_status race_alg1_workspace_bytes(const race_alg1_shape* shape, int32_t variant,
                                      int32_t tile_tokens, size_t* bytes, int64_t* tiles,
                                      int64_t* record_floats_out) {
    if (!bytes) return RACE_ERROR_INVALID_VALUE;
    Problem p;
    const race_status st = alg1_problem(shape, variant, tile_tokens, &p);
    if (st != RACE_SUCCESS) return st;
    *bytes = size_t(p.N * p.tiles * p.rec) * sizeof(float);
    if (tiles) *tiles = p.tiles;
    if (record_floats_out) *record_floats_out = p.rec;
    return RACE_SUCCESS;
}

race_status race_alg1_fwd(const void* q, const void* k, const void* v, const float* W,
                          const float* beta, void* out, float* final_state,
                          const race_alg1_shape* shape, int32_t tile_tokens, int32_t variant,
                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
    Marks none;
    return alg1_fwd_impl(q, k, v, W, beta, out, nullptr, final_state, shape, tile_tokens, variant,
                         workspace, workspace_bytes, stream, &none);
}

race_status race_alg1_fwd_carry(const void* q, const void* k, const void* v, const float* W,
                                const float* beta, void* out, const float* init_state,
                                float* final_state, const race_alg1_shape* shape,
                                int32_t tile_tokens, int32_t variant, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
    if (!init_state) return RACE_ERROR_INVALID_VALUE;
    Marks none;
    return alg1_fwd_impl(q, k, v, W, beta, out, init_state, final_state, shape, tile_tokens,
                         variant, workspace, workspace_bytes, stream, &none);
}

race_status race_alg1_fwd_profiled(const void* q, const void* k, const void* v, const float* W,
                                   const float* beta, void* out, float* final_state,
                                   const race_alg1_shape* shape, int32_t tile_tokens,
                                   int32_t variant, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream, hipEvent_t* events, int32_t max_events,
                                   int32_t* n_events) {
    if (!events || max_events < 2 || !n_events) return RACE_ERROR_INVALID_VALUE;
    Marks marks;
    marks.events = events;
    marks.max = max_events;
    const race_status st = alg1_fwd_impl(q, k, v, W, beta, out, nullptr, final_state, shape, tile_tokens,
                                         variant, workspace, workspace_bytes, stream, &marks);
    *n_events = marks.n;
    return st;
}

}  // extern "C"
