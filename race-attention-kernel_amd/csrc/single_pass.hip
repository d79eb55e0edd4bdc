// single_pass.hip -- one-read causal forward for S = d = 64 on gfx950.
//
// The three-launch forward (mfma_causal.hip) reads K and V twice: once for
// the tile totals, again in the output pass.  This path reads every operand
// once.  A workgroup stages a tile's K and V in LDS while it forms the tile's
// totals (phase 1), publishes them, and walks the same LDS copy for the
// tile's output (phase 2) once the tile's exclusive prefix is known.  The
// prefixes come from kSpParts scanner workgroups per stream (each owning a
// quarter of every record) that add the tile totals in tile order -- the
// running sums of src/race_baseline.py:45-51 at tile granularity, in the
// fixed order of tile_scan_kernel -- so results do not depend on timing and
// repeat bit for bit.
//
// Placement.  Every stream is processed on one XCD (the hardware register
// XCC_ID names the XCD a workgroup runs on): tile totals, prefixes and flags
// then move through that XCD's L2, where a plain store that has completed
// (s_waitcnt vmcnt(0)) is visible to every other CU of the XCD.  XCD x takes
// the streams n = x, x + 8, ...; the host runs this path only when the
// stream count is 8 or 16, so the XCDs are evenly loaded and the scanners
// (kSpParts per stream) leave most of each XCD's 32 CUs to the tiles.
//
// Work order.  Each XCD has one ticket counter.  Its first tickets make
// their workgroups the scanners of the XCD's streams; later tickets name
// tiles, interleaved over the XCD's streams in tile order.  A workgroup
// holding a tile waits only for that tile's prefix, which needs the totals of
// earlier tiles of the stream.  Those were ticketed earlier, by workgroups
// that are running, and a workgroup waits only while each tile whose totals
// it has not yet published was ticketed after the tile it waits for.  So
// every wait points to an earlier ticket and none can close a cycle, whatever
// the number of resident workgroups (tests/test_single_pass_protocol.py
// emulates the protocol; dealing tiles out by launch index instead
// deadlocks there).  Every wait is still bounded: after kSpSpinLimit polls it sets
// the error word, and every later wait gives up at once, so the kernel always
// ends.  A give-up is never silent: a tile whose prefix wait gave up computes
// its output from a NaN prefix, so every output row of that tile is NaN, and a
// scanner that gave up writes NaN into `state`; the host reads the error word
// back with race_fwd_single_status.  The arming kernel can preset the error
// word (a test hook), which makes every wait give up at once.
//
// Pipeline of a tile workgroup.  Tiles are NSUB sub-chunks of C = 32 tokens.
// Step s stages sub-chunk s of the workgroup's tile sequence (phase 1) and
// runs the output of sub-chunk s - L (phase 2), L = R - 1, from a ring of R
// LDS slots, so a tile's totals are published L - NSUB steps before its
// output starts and the scanner's latency hides behind that lag.
#include <atomic>

#include "causal_geo.h"

namespace race {
namespace {

using namespace mfma;

constexpr int kSpS = 64, kSpD = 64, kSpC = 32, kSpNW = 4, kSpT = 64 * kSpNW;
constexpr int kSpXcds = 8;
constexpr int kSpWindow = 16;          // tiles a scanner takes in one round trip
constexpr int kSpSpinLimit = 1 << 16;  // polls before a wait gives up
constexpr int kSpParts = 4;           // scanner workgroups per stream
constexpr int kFlagTotals = 1, kFlagPrefix = 1 + kSpParts;
constexpr int kSpErr = kSpXcds;        // control word index of the error flag
constexpr int kSpLoadPolicy = kPolicyStream;  // every operand is read once
constexpr int kRecPolicy = 16;         // `sc1`: record reads miss the CU cache

template <typename TIn, int NSUB, int R>
struct SpGeo {
    using G = Geo<TIn, kSpS, kSpD, kSpC, kSpNW>;
    static constexpr int kSlotBytes = G::kKBytes + G::kVBytes;
    static constexpr int kLag = R - 1;
    static constexpr int kLds = R * kSlotBytes + G::kWBytes + G::kPBytes + G::kOBytes + G::kQBytes;
    static constexpr int kTile = kSpC * NSUB;
    static_assert(NSUB >= 2, "the next tile's ticket is taken two steps ahead");
    static_assert(kLag >= NSUB, "a tile's totals are complete before its output starts");
    static_assert((kLag + NSUB - 1) / NSUB + 2 <= 8, "live tiles fit the 8-entry tile ring");
};

// The XCD this workgroup runs on: hwreg(HW_REG_XCC_ID, 0, 4).
__device__ __forceinline__ int xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & (kSpXcds - 1); }

__device__ __forceinline__ int flag_load(const int* f) {
    return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_store(int* f, int v) {
    __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Completion of this wave's outstanding global stores (and loads).
__device__ __forceinline__ void drain_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// A use of x at this point: the compiler waits for the load that wrote it here.
__device__ __forceinline__ void settle(f32x4& x) { asm volatile("" : "+v"(x)); }

// Polls *f until it reaches `want`; false once the spin limit is spent here or
// the error word is set by any wave (checked first, so a preset error word
// fails every wait, ready or not).
__device__ __forceinline__ bool wait_flag(const int* f, int want, int* ctl) {
    for (int i = 0; i < kSpSpinLimit; ++i) {
        if (flag_load(ctl + kSpErr) != 0) return false;
        if (flag_load(f) >= want) return true;
        __builtin_amdgcn_s_sleep(2);
    }
    flag_store(ctl + kSpErr, 1);
    return false;
}

__device__ __forceinline__ float quiet_nan() { return __builtin_bit_cast(float, 0x7fc00000u); }

// A tile job: stream n and tile i of the job index v on an XCD with 2^mshift
// streams (one or two).  Kept in scalar registers: buffer resources built
// from vector registers cost a readfirstlane loop per load.
struct SpTile {
    int64_t n, i;
};
__device__ __forceinline__ SpTile sp_tile(int v, int x, int mshift) {
    const int n = __builtin_amdgcn_readfirstlane(x + kSpXcds * (v & ((1 << mshift) - 1)));
    const int i = __builtin_amdgcn_readfirstlane(v >> mshift);
    return SpTile{int64_t(n), int64_t(i)};
}

// ---------------------------------------------------------------------------
// Scanner of part `part` of stream n's records: the exclusive prefix of every
// tile, in place, in tile order.  A record is 1040 chunks of 16 bytes (B
// [64][64], then A [64]); kSpParts scanners share a stream, part p owning
// chunks [260 p, 260 p + 260): thread t owns chunk 260 p + t and, for t < 4,
// chunk 260 p + 256 + t.  Each part adds one to a tile's flag once its share
// of the prefix is stored, so a tile's prefix is whole at 1 + kSpParts.
__device__ __forceinline__ void sp_scan(float* __restrict__ records, int* __restrict__ flags,
                                        int* __restrict__ ctl, float* __restrict__ state,
                                        const float* __restrict__ init, int64_t n, int part,
                                        int64_t tiles, int64_t rec, int* bcast) {
    constexpr int kChunks = (kSpS * kSpD + kSpS) / 4;  // 1040
    constexpr int kPart = kChunks / kSpParts;           // 260
    constexpr int kExtra = kPart - kSpT;                // 4
    constexpr int kStateFloats = kSpS * kSpD + kSpS;
    static_assert(kChunks % kSpParts == 0 && kExtra > 0 && kExtra <= 64, "chunk ownership");
    const int tid = threadIdx.x, l = tid & 63;
    const bool w0 = tid < 64;
    const bool has_b = tid < kExtra;
    const int c0 = kPart * part + tid;
    const int c1 = kPart * part + kSpT + (tid & (kExtra - 1));  // threads past kExtra read a copy
    f32x4 run0 = {0.f, 0.f, 0.f, 0.f}, run1 = {0.f, 0.f, 0.f, 0.f};
    if (init) {
        const float* ip = init + n * kStateFloats;
        run0 = *reinterpret_cast<const f32x4*>(ip + 4 * c0);
        if (has_b) run1 = *reinterpret_cast<const f32x4*>(ip + 4 * c1);
    }
    int* fl = flags + n * tiles;
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(records + n * tiles * rec, tiles * rec * int64_t(sizeof(float)));

    // Wave 0 polls a window of flags; lane j holds the flag of tile pos + j.
    auto poll = [&](int64_t pos) {
        return (l < kSpWindow && pos + l < tiles) ? flag_load(fl + pos + l) : 0;
    };
    int64_t pos = 0;
    int f = w0 ? poll(0) : 0;
    int idle = 0;
    // An error word set before the scan starts (a wait elsewhere gave up, or
    // the test preset) stops it here: no prefix is published, so every tile
    // wait of the stream gives up too.
    const bool preset = __builtin_amdgcn_readfirstlane(flag_load(ctl + kSpErr)) != 0;
    while (!preset && pos < tiles) {
        if (w0) {
            const bool ready = l < kSpWindow && pos + l < tiles && f >= kFlagTotals;
            const uint64_t not_ready = __ballot(!ready);
            const int r = not_ready ? __builtin_ctzll(not_ready) : 64;
            if (l == 0) bcast[0] = r < kSpWindow ? r : kSpWindow;
        }
        __syncthreads();
        const int r = __builtin_amdgcn_readfirstlane(bcast[0]);
        if (r == 0) {
            bool give_up = false;
            if (w0) {
                give_up = ++idle >= kSpSpinLimit || flag_load(ctl + kSpErr) != 0;
                if (give_up && l == 0) flag_store(ctl + kSpErr, 1);
                __builtin_amdgcn_s_sleep(1);
                f = poll(pos);
            }
            if (w0 && l == 0) bcast[1] = give_up;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(bcast[1])) break;
            continue;
        }
        idle = 0;
        // The window's totals, every slot read (unconditional loads keep the
        // registers simple; slots at or past r are not used, slots past the
        // last tile read that tile again).  Byte offsets within the stream's
        // records stay below 2^31 (the host checks tiles * rec): the tile
        // part is uniform (soffset), the chunk part per thread.
        f32x4 x0[kSpWindow], x1[kSpWindow];
#pragma unroll
        for (int j = 0; j < kSpWindow; ++j) {
            const int soff = int((pos + j < tiles ? pos + j : tiles - 1) * rec * int64_t(sizeof(float)));
            x0[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, 16 * c0, soff, kRecPolicy));
            x1[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, 16 * c1, soff, kRecPolicy));
        }
#pragma unroll
        for (int j = 0; j < kSpWindow; ++j) {
            if (j < r) {
                const int soff = int((pos + j) * rec * int64_t(sizeof(float)));
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, run0), rr, 16 * c0, soff, 0);
                if (has_b) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, run1), rr, 16 * c1, soff, 0);
                run0 = run0 + x0[j];
                run1 = run1 + x1[j];
            }
        }
        if (w0) f = poll(pos + r);
        drain_vm();
        __syncthreads();
        if (w0 && l < r) __hip_atomic_fetch_add(fl + pos + l, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pos += r;
    }
    if (state) {
        // A scan that gave up leaves NaN, never a partial sum, in the state.
        if (pos != tiles) {
            const float nan = quiet_nan();
            run0 = f32x4{nan, nan, nan, nan};
            run1 = run0;
        }
        float* sp = state + n * kStateFloats;
        *reinterpret_cast<f32x4*>(sp + 4 * c0) = run0;
        if (has_b) *reinterpret_cast<f32x4*>(sp + 4 * c1) = run1;
    }
}

// ---------------------------------------------------------------------------
template <typename TIn, int NSUB, int R>
__global__ __launch_bounds__(kSpT, 1) void causal_single_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    TIn* __restrict__ out, float* __restrict__ records, int* __restrict__ flags, int* __restrict__ ctl,
    float* __restrict__ state, const float* __restrict__ init, int64_t T, int64_t tiles, int64_t rec,
    int N) {
    using SG = SpGeo<TIn, NSUB, R>;
    using G = typename SG::G;
    using PS = typename G::PS;
    using PK = typename G::PK;
    using PC = typename G::PC;
    using PD = typename G::PD;
    using OT = OutTile<TIn, kSpD, kSpC>;
    using QT = OutTile<TIn, kSpS, kSpC>;
    constexpr bool kSplit = G::kSplit;
    constexpr int S = kSpS, D = kSpD, C = kSpC, L = SG::kLag, TT = SG::kTile;
    constexpr int NSB = S / 16, NBI = C / 16, NKS = S / 32;
    constexpr int NLB = NBI * (NBI + 1) / 2;
    constexpr int es = int(sizeof(TIn));
    constexpr bool kQStage = G::kQStage;
    constexpr int kQChunks = C * QT::kChunks;
    constexpr int kQPer = (kQChunks + kSpT - 1) / kSpT;
    constexpr int kStoreP = std::is_same<TIn, float>::value ? kOutWgStorePolicyF32 : kOutStorePolicy;

    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* Slots = lds;
    unsigned char* Ws = Slots + R * SG::kSlotBytes;
    unsigned char* Ps = Ws + G::kWBytes;
    unsigned char* Os = Ps + G::kPBytes;
    unsigned char* Qs = Os + G::kOBytes;
    __shared__ int ring[8];   // tile jobs of the workgroup's tiles k, at k % 8 (-1: none)
    __shared__ int bcast[2];

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, lr = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int x = xcc_id();
    const int m = x < N ? (N - x + kSpXcds - 1) / kSpXcds : 0;
    if (m == 0) return;
    const int mshift = m > 1 ? 1 : 0;  // the host allows one or two streams per XCD
    const int jobs = int(int64_t(m) * tiles);  // the host keeps N * tiles below 2^31

    if (tid == 0) bcast[0] = atomicAdd(ctl + x, 1);
    __syncthreads();
    const int first = __builtin_amdgcn_readfirstlane(bcast[0]);
    __syncthreads();
    if (first < m * kSpParts) {
        sp_scan(records, flags, ctl, state, init, int64_t(x) + int64_t(kSpXcds) * (first / kSpParts),
                first % kSpParts, tiles, rec, bcast);
        return;
    }

    // ---- tile role ----
    const __amdgpu_buffer_rsrc_t none = make_rsrc(nullptr, 0);
    auto rows_of = [&](const SpTile& t) { return int(min<int64_t>(TT, T - t.i * TT)); };
    auto job_at = [&](int kk) { return __builtin_amdgcn_readfirstlane(ring[kk & 7]); };

    const bf16x8 tri0 = tril_frag(0, g, lr), tri1 = tril_frag(16, g, lr);
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = __bf16(1.0f);

    using QRegs = std::conditional_t<kQStage, uint4[kQPer], f32x4[NBI]>;
    auto load_q = [&](QRegs& qr, __amdgpu_buffer_rsrc_t qrs, int r0) {
        if constexpr (kQStage) {
#pragma unroll
            for (int i = 0; i < kQPer; ++i) {
                const int qi = tid + i * kSpT;
                if (kQChunks % kSpT == 0 || qi < kQChunks)
                    qr[i] = buf_load16<kSpLoadPolicy>(qrs, r0 * S * es + 16 * qi);
            }
        } else {
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi)
                qr[bi] = load_q4<TIn, kSpLoadPolicy>(qrs, ((r0 + 16 * bi + lr) * S + 16 * w + 4 * g) * es);
        }
    };

    int kmax = 1 << 30;  // number of tiles this workgroup holds, once a ticket runs out
    const int job0 = first - m * kSpParts;
    if (tid == 0) ring[0] = job0 < jobs ? job0 : -1;
    if (job0 >= jobs) kmax = 0;

    KVStage<TIn, S, D, C, kSpLoadPolicy, kSpNW> st;
    QRegs qr;
    if (kmax > 0) {
        const SpTile t0 = sp_tile(job0, x, mshift);
        const int rows = rows_of(t0);
        st.load(make_rsrc(k + (t0.n * T + t0.i * TT) * S, int64_t(rows) * S * es),
                make_rsrc(v + (t0.n * T + t0.i * TT) * D, int64_t(rows) * D * es), 0);
    }

    f32x4 gb[NSB];   // phase 1: tile totals B[16 sb + 4 g + r][16 w + lr]
    f32x4 ga;        // phase 1: A[16 w + 4 g + r] (every lr)
    f32x4 b0[NSB];   // phase 2: running B0[16 sb + 4 g + r][16 w + lr]
    float a0[4];     // phase 2: running A0[16 w + 4 g + r]
    int ticket = 0;  // thread 0: the next tile's ticket
    // The output tile's chunks on their way to global memory.  Live across
    // the loop, so their registers are written again only by the next
    // flush, a step later: a store's data registers cannot be overwritten
    // before the store completes, and registers reused right after the flush
    // made the next loads wait for it.
    typename OT::template Chunks<kSpT> och;
#pragma unroll
    for (int i = 0; i < OT::template Chunks<kSpT>::kPer; ++i) och.x[i] = make_uint4(0, 0, 0, 0);
    int* pending_flag = nullptr;                 // totals stored last step, flag not yet set
    __amdgpu_buffer_rsrc_t flush_o = none;       // output tile of the previous phase-2 step
    int flush_r0 = 0;
    bool flush_pending = false;

    for (int s = 0;; ++s) {
#pragma unroll
        for (int i = 0; i < OT::template Chunks<kSpT>::kPer; ++i)
            asm volatile("" : "+v"(och.x[i].x), "+v"(och.x[i].y), "+v"(och.x[i].z), "+v"(och.x[i].w));
        const int k1 = s / NSUB, j1 = s % NSUB;
        const bool p1 = k1 < kmax;
        const int s2 = s - L;
        const int k2 = s2 >= 0 ? s2 / NSUB : -1, j2 = s2 >= 0 ? s2 % NSUB : 0;
        const bool p2 = s2 >= 0 && k2 < kmax;
        // Done once phase 2 has passed the last tile (steps between the last
        // phase-1 and the first phase-2 sub-chunk of a tile have neither).
        if (s2 >= 0 && k2 >= kmax) break;

        // Release the totals stored last step: every wave's stores complete,
        // then one flag.
        if (pending_flag) drain_vm();
        __syncthreads();  // B1: slot s % R and the output tile are free
        if (pending_flag && tid == 0) flag_store(pending_flag, kFlagTotals);
        pending_flag = nullptr;
        // Phase 2's tile and, at its first sub-chunk, its exclusive prefix
        // (waited for after the release above, which other tiles' prefixes need).
        SpTile t2 = {0, 0};
        if (p2) {
            t2 = sp_tile(job_at(k2), x, mshift);
            if (j2 == 0) {
                const bool ready = wait_flag(flags + t2.n * tiles + t2.i, kFlagPrefix, ctl);
                const __amdgpu_buffer_rsrc_t pr =
                    make_rsrc(records + (t2.n * tiles + t2.i) * rec, rec * int64_t(sizeof(float)));
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        b0[sb][rr] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                   pr, ((16 * sb + 4 * g + rr) * D + 16 * w + lr) * 4, 0,
                                                                   kRecPolicy));
                f32x4 a = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, (S * D + 16 * w + 4 * g) * 4, 0, kRecPolicy));
                // Use the prefix here, once per tile: left pending, the
                // compiler waits for every load of the step where b0 and a0
                // are next read (they are loop-carried), i.e. for the
                // prefetches as well, on every step.
                settle(a);
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb) settle(b0[sb]);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) a0[rr] = a[rr];
                // A prefix that never arrived: NaN reaches every W and every
                // product of the tile, so each of its output rows is NaN.
                if (!ready) {
                    const float nan = quiet_nan();
#pragma unroll
                    for (int sb = 0; sb < NSB; ++sb) b0[sb] = f32x4{nan, nan, nan, nan};
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) a0[rr] = nan;
                }
            }
        }
        const int rows2 = p2 ? rows_of(t2) : 0;
        const int64_t base2 = t2.n * T + t2.i * TT;

        unsigned char* K1 = Slots + (s % R) * SG::kSlotBytes;
        unsigned char* V1 = K1 + G::kKBytes;
        unsigned char* K2 = Slots + ((s2 + R) % R) * SG::kSlotBytes;
        unsigned char* V2 = K2 + G::kKBytes;
        if (p1) st.store(K1, V1, nullptr);
        if (p1 && j1 == NSUB - 1 && tid == 0) {
            const int job = ticket - m * kSpParts;
            ring[(k1 + 1) & 7] = (k1 + 1 < kmax && job < jobs) ? job : -1;
        }
        f32x4 qc[NBI];
        if (p2) {
            if constexpr (kQStage) {
#pragma unroll
                for (int i = 0; i < kQPer; ++i) {
                    const int qi = tid + i * kSpT;
                    if (kQChunks % kSpT == 0 || qi < kQChunks)
                        *reinterpret_cast<uint4*>(Qs + QT::chunk_at(qi)) = qr[i];
                }
            } else {
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi) qc[bi] = qr[bi];
            }
        }
        // Order of this step's global traffic: the prefetched registers are
        // consumed above, then the ticket, the output and totals stores,
        // and last the next prefetch loads.  The compiler waits for all
        // outstanding operations (vmcnt(0)) when loads and stores are both
        // pending, so a store issued after a prefetch would hold up that
        // prefetch's use by a whole store round trip.
        if (p1 && j1 == NSUB - 2 && tid == 0) ticket = atomicAdd(ctl + x, 1);
        if (flush_pending) {
            OT::template read<kSpT>(Os, och);
            OT::template write<kStoreP, kSpT>(och, flush_o, flush_r0);
        }
        flush_pending = false;
        __syncthreads();  // B2

        if (p1 && j1 == NSUB - 1 && job_at(k1 + 1) < 0) kmax = k1 + 1;
        // Phase 1: tile totals over this sub-chunk.
        if (p1) {
            if (j1 == 0) {
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb) gb[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
                ga = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            bf16x8 vh, vl;
            PD::frag_tr(V1, 0, 16 * w, g, lr, vh, vl);
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb) {
                bf16x8 kh, kl;
                PK::frag_tr(K1, 0, 16 * sb, g, lr, kh, kl);
                gb[sb] = mfma3<kSplit>(kh, kl, vh, vl, gb[sb]);
                if (sb == w) {
                    if constexpr (kSplit) ga = mfma16(kl, ones, ga);
                    ga = mfma16(kh, ones, ga);
                }
            }
            if (j1 == NSUB - 1) {
                const SpTile t1 = sp_tile(job_at(k1), x, mshift);
                float* rp = records + (t1.n * tiles + t1.i) * rec;
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) rp[(16 * sb + 4 * g + rr) * D + 16 * w + lr] = gb[sb][rr];
                if (lr == 0) *reinterpret_cast<f32x4*>(rp + S * D + 16 * w + 4 * g) = ga;
                pending_flag = flags + t1.n * tiles + t1.i;
            }
        }

        // Prefetch step s + 1: phase 1's K and V, phase 2's Q.
        {
            const int n1 = (s + 1) / NSUB, m1 = (s + 1) % NSUB;
            if (n1 < kmax) {
                const SpTile t = sp_tile(job_at(n1), x, mshift);
                const int rows = rows_of(t);
                st.load(make_rsrc(k + (t.n * T + t.i * TT) * S, int64_t(rows) * S * es),
                        make_rsrc(v + (t.n * T + t.i * TT) * D, int64_t(rows) * D * es), C * m1);
            }
            const int sq = s + 1 - L;
            if (sq >= 0 && sq / NSUB < kmax) {
                const SpTile t = sp_tile(job_at(sq / NSUB), x, mshift);
                const int rows = rows_of(t);
                load_q(qr, make_rsrc(q + (t.n * T + t.i * TT) * S, int64_t(rows) * S * es), C * (sq % NSUB));
            }
        }

        // Phase 2, steps 1 + 2: running mass and W = Q / (Abar + eps).
        if (p2) {
            bf16x8 kh, kl;
            PK::frag_tr(K2, 0, 16 * w, g, lr, kh, kl);
            f32x4 last;
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
                f32x4 acc = {a0[0], a0[1], a0[2], a0[3]};
                const bf16x8& lf = bi == 0 ? tri0 : tri1;
                if constexpr (kSplit) acc = mfma16(kl, lf, acc);
                acc = mfma16(kh, lf, acc);
                const f32x4 qv = kQStage ? QT::get4(Qs, 16 * bi + lr, 16 * w + 4 * g) : qc[bi];
                uint2 hi, lo;
                split4<kSplit>(qv[0] * __builtin_amdgcn_rcpf(acc[0] + kEps),
                               qv[1] * __builtin_amdgcn_rcpf(acc[1] + kEps),
                               qv[2] * __builtin_amdgcn_rcpf(acc[2] + kEps),
                               qv[3] * __builtin_amdgcn_rcpf(acc[3] + kEps), hi, lo);
                PS::put4(Ws, 16 * bi + lr, 16 * w + 4 * g, hi, lo);
                last = acc;
            }
            // Inclusive mass at the sub-chunk's last row (zero rows past the tile add nothing).
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) a0[rr] = __shfl(last[rr], 16 * g + 15);
        }
        __syncthreads();  // B3

        // Phase 2, step 3: P^T blocks of the lower triangle, one per wave.
        if (p2 && w < NLB) {
            int bi = 0, rem = w;
            while (rem > bi) { rem -= bi + 1; ++bi; }
            f32x4 pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                bf16x8 ah, al, bh, bl;
                PK::frag(K2, 16 * rem + lr, kk, g, ah, al);
                PS::frag(Ws, 16 * bi + lr, kk, g, bh, bl);
                pacc = mfma3<kSplit>(ah, al, bh, bl, pacc);
            }
            if (rem == bi) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (4 * g + rr > lr) pacc[rr] = 0.f;
            }
            uint2 hi, lo;
            split4<kSplit>(pacc[0], pacc[1], pacc[2], pacc[3], hi, lo);
            PC::put4(Ps, 16 * bi + lr, 16 * rem + 4 * g, hi, lo);
        }
        __syncthreads();  // B4

        // Phase 2, steps 4 + 5: O^T = B0^T W^T + V^T P^T for c-block w, then B0 += K^T V.
        if (p2) {
            bf16x8 vh, vl;
            PD::frag_tr(V2, 0, 16 * w, g, lr, vh, vl);
            f32x4 o[NBI];
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) o[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
                const f32x4 x0 = b0[2 * kk], x1 = b0[2 * kk + 1];
                uint2 h0, l0, h1, l1;
                split4<kSplit>(x0[0], x0[1], x0[2], x0[3], h0, l0);
                split4<kSplit>(x1[0], x1[1], x1[2], x1[3], h1, l1);
                const bf16x8 bh = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                bf16x8 bl = bh;
                if constexpr (kSplit) bl = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
#pragma unroll
                for (int bi = 0; bi < NBI; ++bi) {
                    bf16x8 wh, wl;
                    PS::frag(Ws, 16 * bi + lr, kk, g, wh, wl);
                    o[bi] = mfma3<kSplit>(bh, bl, wh, wl, o[bi]);
                }
            }
#pragma unroll
            for (int bi = 0; bi < NBI; ++bi) {
                bf16x8 ph, pl;
                PC::frag(Ps, 16 * bi + lr, 0, g, ph, pl);
                if (bi == 0) {
                    // The upper half of this step is the block above the
                    // diagonal: zero, and never written to the P tile.
#pragma unroll
                    for (int e = 4; e < 8; ++e) {
                        ph[e] = __bf16(0.0f);
                        if constexpr (kSplit) pl[e] = __bf16(0.0f);
                    }
                }
                o[bi] = mfma3<kSplit>(vh, vl, ph, pl, o[bi]);
                OT::put(Os, 16 * bi + lr, 16 * w + 4 * g, o[bi]);
            }
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb) {
                bf16x8 kh, kl;
                PK::frag_tr(K2, 0, 16 * sb, g, lr, kh, kl);
                b0[sb] = mfma3<kSplit>(kh, kl, vh, vl, b0[sb]);
            }
            flush_o = make_rsrc(out + base2 * D, int64_t(rows2) * D * es);
            flush_r0 = C * j2;
            flush_pending = true;
        }
    }
    __syncthreads();
    if (flush_pending) {
        OT::template read<kSpT>(Os, och);
        OT::template write<kStoreP, kSpT>(och, flush_o, flush_r0);
    }
}

// Zeroes the tile flags and the control words ahead of the main kernel; the
// error word (index err_at) gets err_value, 0 unless the test hook presets it.
__global__ __launch_bounds__(kThreads) void single_arm_kernel(int* __restrict__ words, int64_t count,
                                                              int64_t err_at, int err_value) {
    for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += int64_t(gridDim.x) * kThreads)
        words[i] = i == err_at ? err_value : 0;
}

std::atomic<int> g_preset_give_up{0};

template <typename TIn, int NSUB, int R>
hipError_t launch_single(const void* q, const void* k, const void* v, void* out, float* records,
                         int* words, float* state, const float* init, const Problem& p, int cus,
                         hipStream_t stream, Marks* marks) {
    using SG = SpGeo<TIn, NSUB, R>;
    if (p.tile != SG::kTile) return hipErrorInvalidValue;
    const int64_t nflags = single_pass_flag_words(p.N, p.tiles);
    const int64_t count = nflags + kSinglePassCtlWords;
    single_arm_kernel<<<dim3(unsigned((count + kThreads - 1) / kThreads)), kThreads, 0, stream>>>(
        words, count, nflags + kSpErr, g_preset_give_up.load() ? 1 : 0);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (marks && (err = marks->mark(stream)) != hipSuccess) return err;
    causal_single_kernel<TIn, NSUB, R><<<dim3(unsigned(cus)), kSpT, SG::kLds, stream>>>(
        static_cast<const TIn*>(q), static_cast<const TIn*>(k), static_cast<const TIn*>(v),
        static_cast<TIn*>(out), records, words, words + nflags, state, init, p.T, p.tiles, p.rec,
        int(p.N));
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return marks ? marks->mark(stream) : hipSuccess;
}

}  // namespace

bool single_pass_supported(const Problem& p, int cus) {
    // One or two streams per XCD (N = 8 or 16), 32 CUs per XCD.
    if (p.S != kSpS || p.d != kSpD || p.N <= 0 || p.N % kSpXcds != 0 || p.N / kSpXcds > 2) return false;
    if (cus != 32 * kSpXcds) return false;
    if (p.dtype != RACE_F32 && p.dtype != RACE_BF16) return false;
    // Ticket and offset arithmetic: jobs and a stream's records in 32 bits.
    if (p.N * p.tiles >= (int64_t(1) << 31)) return false;
    if (p.tiles * p.rec * int64_t(sizeof(float)) >= (int64_t(1) << 31)) return false;
    return true;
}

int single_pass_tile() { return kSinglePassTile; }

int64_t single_pass_error_word(int64_t N, int64_t tiles) { return single_pass_flag_words(N, tiles) + kSpErr; }

void single_pass_preset_give_up(bool on) { g_preset_give_up.store(on ? 1 : 0); }

hipError_t launch_causal_single(const void* q, const void* k, const void* v, void* out,
                                float* records, int* words, float* state, const float* init,
                                const Problem& p, int cus, hipStream_t stream, Marks* marks) {
    if (!single_pass_supported(p, cus)) return hipErrorInvalidValue;
    if (p.dtype == RACE_BF16)
        return launch_single<bf16_t, 4, 14>(q, k, v, out, records, words, state, init, p, cus, stream, marks);
    return launch_single<float, 4, 7>(q, k, v, out, records, words, state, init, p, cus, stream, marks);
}

}  // namespace race
