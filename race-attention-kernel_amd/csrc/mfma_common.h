// mfma_common.h -- device helpers shared by the MFMA kernels of the RACE
// attention library (gfx950): bf16 hi/lo splitting, the permuted-k fragment
// order, buffer-resource loads and stores.  Not part of the ABI.
//
// Conventions.  A lane l of a wave64 has group g = l / 16 and row lr = l % 16.
// v_mfma_f32_16x16x32_bf16 takes from each lane 8 bf16 of the A operand (row
// m = lr, 8 values of the contraction index k), 8 bf16 of the B operand
// (column n = lr, the same 8 k values) and returns the 4 accumulator values
// D[4 g + r][lr], r = 0..3.  The kernels permute the contraction index of one
// 32-wide step kk: lane group g, element e carries
//     k = 32 kk + 4 g + (e % 4) + 16 (e / 4),
// which is the set of rows two stacked accumulator blocks give a lane, so an
// fp32 accumulator (the carried state) feeds the next product directly.  LDS
// operand rows store elements in that order: element k of a row sits at
//     fpos(k) = 32 (k / 32) + 8 ((k / 4) % 4) + 4 ((k / 16) % 2) + k % 4
// of its bf16 plane, and one fragment is one 16-byte read per plane.
#pragma once

#include <type_traits>

#include "race_internal.h"

namespace race {
namespace mfma {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// acc += A B with optional hi/lo operands: lo*hi and hi*lo first, then hi*hi.
template <bool kSplit>
__device__ __forceinline__ f32x4 mfma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                       const bf16x8& bl, f32x4 acc) {
    if constexpr (kSplit) {
        acc = mfma16(al, bh, acc);
        acc = mfma16(ah, bl, acc);
    }
    return mfma16(ah, bh, acc);
}

__device__ __forceinline__ constexpr int fpos(int k) {
    return (k & ~31) | (((k >> 2) & 3) << 3) | (((k >> 4) & 1) << 2) | (k & 3);
}

// Two floats to a packed pair of bf16 (round to nearest even).
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    const bf16x2 h = __builtin_convertvector(f32x2{a, b}, bf16x2);
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ float lo_half(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ uint32_t word(const uint2& u, int i) { return i ? u.y : u.x; }
__device__ __forceinline__ uint32_t half16(uint32_t w, int h) { return h ? (w >> 16) : (w & 0xffffu); }
__device__ __forceinline__ float hi_half(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// Four consecutive elements split into packed hi (and lo) pairs.
template <bool kSplit>
__device__ __forceinline__ void split4(float x0, float x1, float x2, float x3, uint2& hi, uint2& lo) {
    hi.x = pack2(x0, x1);
    hi.y = pack2(x2, x3);
    if constexpr (kSplit) {
        lo.x = pack2(x0 - lo_half(hi.x), x1 - hi_half(hi.x));
        lo.y = pack2(x2 - lo_half(hi.y), x3 - hi_half(hi.y));
    }
}

// ---------------------------------------------------------------------------
// Global -> register traffic.  Token rows of one stream are contiguous.

template <typename TIn>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int kPerVec = 4;  // elements per 16-byte vector
    __device__ static float get(const uint4& v, int i) {
        return __uint_as_float(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
    }
};
template <>
struct Elem<bf16_t> {
    static constexpr int kPerVec = 8;
    __device__ static float get(const uint4& v, int i) {
        const uint32_t w = (i >> 1) == 0 ? v.x : (i >> 1) == 1 ? v.y : (i >> 1) == 2 ? v.z : v.w;
        return (i & 1) ? hi_half(w) : lo_half(w);
    }
};

// Buffer resource over `bytes` bytes from `base`: loads past the end return
// zero and stores past the end are dropped, which is how a ragged last
// sub-chunk reads zero rows and writes nothing past the sequence.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(bytes),
                                             0x00020000);
}
// Cache policy bits of buffer loads and stores (the instruction's aux field):
// 0 = default, 2 = nontemporal (`nt`).  Streaming reads with `nt` run at about
// 7.1 TB/s on MI355X against 6.3 TB/s without it; each kernel picks its own.
constexpr int kPolicyDefault = 0;
constexpr int kPolicyStream = 2;
#ifndef RACE_SUMS_LOAD_POLICY
#define RACE_SUMS_LOAD_POLICY 2
#endif
#ifndef RACE_OUT_KV_POLICY
#define RACE_OUT_KV_POLICY 0
#endif
#ifndef RACE_OUT_Q_POLICY
#define RACE_OUT_Q_POLICY 0
#endif
#ifndef RACE_OUT_STORE_POLICY
#define RACE_OUT_STORE_POLICY 0
#endif
#ifndef RACE_OUT_WG_STORE_POLICY
#define RACE_OUT_WG_STORE_POLICY 2
#endif
#ifndef RACE_ALG1_STORE_POLICY
#define RACE_ALG1_STORE_POLICY 0
#endif
#ifndef RACE_SUMS_F32_LOAD_POLICY
#define RACE_SUMS_F32_LOAD_POLICY 0
#endif
#ifndef RACE_OUT_Q_F32_POLICY
#define RACE_OUT_Q_F32_POLICY 2
#endif
constexpr int kSumsLoadPolicy = RACE_SUMS_LOAD_POLICY;  // K1 reads of K and V
// fp32 tokens at S = d = 64: K1 (tile_sums_quad_kernel) walks each tile from
// its end to its start with cache-allocating loads, so the 256 MB memory-side
// cache holds the start of every tile when the output pass begins there; the
// output pass streams Q past the cache (`nt`) so it does not evict them.
// Measured at cfg2 (T = 65536, one box, 20 steps after the settling phase)
// with one-wave-per-tile K1 walking backward: 3527 -> 3748 M tokens/s with
// the same inputs every step, 3210 -> 3372 with two input sets alternating
// (no step finds its inputs left over from the step before).
constexpr int kSumsF32LoadPolicy = RACE_SUMS_F32_LOAD_POLICY;
constexpr int kOutQPolicyF32 = RACE_OUT_Q_F32_POLICY;
constexpr int kOutKVPolicy = RACE_OUT_KV_POLICY;        // K3 reads of K and V read once
constexpr int kOutQPolicy = RACE_OUT_Q_POLICY;          // K3 reads of Q
constexpr int kOutStorePolicy = RACE_OUT_STORE_POLICY;  // register-direct K3 writes of out
// Workgroup K3 writes of fp32 out: `nt` measured 120 -> 116 us at cfg2; bf16
// writes keep the default (the S = 256 kernel at cfg5 ran 997 -> 1015 us with
// `nt`, the register-direct kernel at cfg3 866 -> 881 us).
constexpr int kOutWgStorePolicyF32 = RACE_OUT_WG_STORE_POLICY;
constexpr int kAlg1StorePolicy = RACE_ALG1_STORE_POLICY;  // Algorithm-1 K3 writes of out

template <int P>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, P));
}
template <int P>
__device__ __forceinline__ uint2 buf_load8(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, P));
}

// Four consecutive Q values at byte offset `off` of a buffer, as floats.
template <typename TIn, int P>
__device__ __forceinline__ f32x4 load_q4(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (std::is_same<TIn, float>::value) {
        return __builtin_bit_cast(f32x4, buf_load16<P>(r, off));
    } else {
        const uint2 u = buf_load8<P>(r, off);
        return f32x4{lo_half(u.x), hi_half(u.x), lo_half(u.y), hi_half(u.y)};
    }
}

// Four consecutive output values at byte offset `off` of a buffer.
template <typename TIn, int P>
__device__ __forceinline__ void store4(__amdgpu_buffer_rsrc_t r, int off, const f32x4& x) {
    if constexpr (std::is_same<TIn, float>::value) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r, off, 0, P);
    } else {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2(x[0], x[1]), pack2(x[2], x[3])}, r, off, 0, P);
    }
}

// Plane tile geometry for rows of K elements.  A plane row is K / 8 chunks of
// 16 bytes (8 elements).  Chunk u of row r is stored at chunk u ^ sw(r),
//     sw(r) = ((r / 8) % 8 ^ (r / 4) % 2) & (K / 8 - 1),
// and rows are 32 bytes longer than the planes.  With that layout the 16-byte
// fragment reads (16 consecutive rows, one chunk) touch every bank once, and
// the transposed staging stores (rows 4 apart, one 8-byte half chunk) are
// spread over all banks instead of piling into two.
//
// kHalfSwap: odd rows also hold the two 8-byte halves of every chunk swapped.
// A transposed read (8 bytes per lane, served 32 lanes per pass) reads 8 rows
// x 4 chunks all in the same half of their chunk, so without the swap its 32
// pieces meet on the 16 half-chunk slots of one parity in a 256-byte span: a
// 2-way conflict on every such read.  With it, the odd rows' pieces take the
// other parity and (bf16 rows of 256 elements, the K tile at S = 256) every
// pass touches each bank once.  The 16-byte fragment reads keep their
// addresses and swap the halves back in registers for odd rows.
template <bool kSplit, int K, bool kHalfSwap = false>
struct Plane {
    static constexpr int kLoOff = 2 * K;                       // bytes to the lo plane
    static constexpr int kPitch = (kSplit ? 4 : 2) * K + 32;   // row pitch in bytes
    static constexpr int kMask = (K / 8 < 8 ? K / 8 : 8) - 1;
    __device__ __forceinline__ static int sw(int row) { return ((row >> 3) ^ ((row >> 2) & 1)) & kMask; }
    // Which 8-byte half of a chunk holds a chunk's first four elements.
    __device__ __forceinline__ static int hs(int row) { return kHalfSwap ? (row & 1) : 0; }
    // Store 4 consecutive elements k0..k0+3 (k0 % 4 == 0) of row `row`.
    __device__ __forceinline__ static void put4(unsigned char* t, int row, int k0, const uint2& hi,
                                                const uint2& lo) {
        unsigned char* p = t + off4(row, k0);
        *reinterpret_cast<uint2*>(p) = hi;
        if constexpr (kSplit) *reinterpret_cast<uint2*>(p + kLoOff) = lo;
    }
    // One element k of row `row` (hi and, with kSplit, lo bf16 bit patterns).
    __device__ __forceinline__ static void put1(unsigned char* t, int row, int k, uint16_t hi,
                                                uint16_t lo) {
        const int pos = fpos(k);
        unsigned char* p = t + row * kPitch + 16 * ((pos >> 3) ^ sw(row)) + 2 * ((pos & 7) ^ (hs(row) << 2));
        *reinterpret_cast<uint16_t*>(p) = hi;
        if constexpr (kSplit) *reinterpret_cast<uint16_t*>(p + kLoOff) = lo;
    }
    // Fragment of row `row` for contraction step kk.
    __device__ __forceinline__ static void frag(const unsigned char* t, int row, int kk, int g,
                                                bf16x8& hi, bf16x8& lo) {
        const unsigned char* p = t + row * kPitch + 16 * ((4 * kk + g) ^ sw(row));
        hi = *reinterpret_cast<const bf16x8*>(p);
        if constexpr (kSplit) lo = *reinterpret_cast<const bf16x8*>(p + kLoOff);
        if constexpr (kHalfSwap) {
            if (row & 1) {
                hi = __builtin_shufflevector(hi, hi, 4, 5, 6, 7, 0, 1, 2, 3);
                if constexpr (kSplit) lo = __builtin_shufflevector(lo, lo, 4, 5, 6, 7, 0, 1, 2, 3);
            }
        }
    }
    // Byte offset of the 8-byte group holding elements k0 .. k0 + 3 (k0 % 4 == 0)
    // of row `row` in the hi plane.
    __device__ __forceinline__ static int off4(int row, int k0) {
        const int pos = fpos(k0);
        return row * kPitch + 16 * ((pos >> 3) ^ sw(row)) + 8 * (((pos >> 2) & 1) ^ hs(row));
    }
    // Fragment of the transposed tile, whose contraction index runs over this
    // plane's rows: lane (g, lr) gets elements (row0 + 4 g + e % 4 + 16 (e / 4),
    // col0 + lr), e = 0..7 (row0 % 32 == 0, col0 % 16 == 0).  Two
    // ds_read_b64_tr_b16 per plane: within each 16-lane group, lane 4 r + q
    // addresses row r, columns 4 q .. 4 q + 3 of a 4 x 16 block, and lane i
    // receives column i.
    __device__ __forceinline__ static void frag_tr(const unsigned char* t, int row0, int col0, int g,
                                                   int lr, bf16x8& hi, bf16x8& lo) {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const int r = row0 + 4 * g + (lr >> 2), k0 = col0 + 4 * (lr & 3);
        const unsigned char* p0 = t + off4(r, k0);
        const unsigned char* p1 = t + off4(r + 16, k0);
        const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
        const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
        hi = __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
        if constexpr (kSplit) {
            const s16x4 c = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0 + kLoOff));
            const s16x4 d = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1 + kLoOff));
            lo = __builtin_bit_cast(bf16x8, __builtin_shufflevector(c, d, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    }
};

// Lower-triangular ones as a B operand for the running mass: element e of
// lane (g, lr) is (j' <= i') with j' = 4 g + e % 4 + 16 (e / 4) and
// i' = off + lr (off = 0 or 16).
__device__ __forceinline__ bf16x8 tril_frag(int off, int g, int lr) {
    bf16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (4 * g + (e & 3) + 16 * (e >> 2) <= off + lr) ? __bf16(1.0f) : __bf16(0.0f);
    return f;
}

// A token-row tile in LDS staged between global memory and the accumulator
// layout: [C][D] elements of TIn, row r a run of D * sizeof(TIn) / 16 chunks
// of 16 bytes with chunk u stored at u ^ swz(r).  swz runs over the 256-byte
// spans the 64 banks cover: rows shorter than a span (bf16 rows of 64 values,
// 128 bytes) share their span's value, swz(r) = (r / rows per span) mod the
// chunk count (at most 16).  Accumulator-layout accesses (16 rows, 4 values
// each, or 4 rows of 16 single values) and the row-contiguous transfers then
// touch each bank at most once per 16 lanes, and the global side moves whole
// rows: 16 bytes per thread, consecutive threads on consecutive bytes.
template <typename TIn, int D, int C>
struct OutTile {
    static constexpr int kRowBytes = D * int(sizeof(TIn));
    static constexpr int kChunks = kRowBytes / 16;
    static constexpr int kMask = (kChunks < 16 ? kChunks : 16) - 1;
    static constexpr int kRowsPerSpan = kRowBytes >= 256 ? 1 : 256 / kRowBytes;
    __device__ __forceinline__ static int swz(int row) { return (row / kRowsPerSpan) & kMask; }
    __device__ __forceinline__ static int at(int row, int byte) {
        return row * kRowBytes + 16 * ((byte >> 4) ^ swz(row)) + (byte & 15);
    }
    // Values [row][col .. col + 3] (col % 4 == 0) from the accumulator layout.
    __device__ __forceinline__ static void put(unsigned char* t, int row, int col, const f32x4& x) {
        unsigned char* p = t + at(row, col * int(sizeof(TIn)));
        if constexpr (std::is_same<TIn, float>::value) {
            *reinterpret_cast<f32x4*>(p) = x;
        } else {
            *reinterpret_cast<uint2*>(p) = make_uint2(pack2(x[0], x[1]), pack2(x[2], x[3]));
        }
    }
    // One value at [row][col].
    __device__ __forceinline__ static void put1(unsigned char* t, int row, int col, float x) {
        unsigned char* p = t + at(row, col * int(sizeof(TIn)));
        if constexpr (std::is_same<TIn, float>::value) {
            *reinterpret_cast<float*>(p) = x;
        } else {
            *reinterpret_cast<uint16_t*>(p) = uint16_t(pack2(x, 0.f) & 0xffffu);
        }
    }
    // Values [row][col .. col + 3] (col % 4 == 0) as floats.
    __device__ __forceinline__ static f32x4 get4(const unsigned char* t, int row, int col) {
        const unsigned char* p = t + at(row, col * int(sizeof(TIn)));
        if constexpr (std::is_same<TIn, float>::value) {
            return *reinterpret_cast<const f32x4*>(p);
        } else {
            const uint2 u = *reinterpret_cast<const uint2*>(p);
            return f32x4{lo_half(u.x), hi_half(u.x), lo_half(u.y), hi_half(u.y)};
        }
    }
    // 16-byte chunk q (row-major over the tile) to or from its swizzled place.
    __device__ __forceinline__ static int chunk_at(int q) {
        const int row = q / kChunks, u = q % kChunks;
        return row * kRowBytes + 16 * (u ^ swz(row));
    }
    // A thread's chunks of the tile (NT threads): chunk q = threadIdx.x + i NT.
    template <int NT>
    struct Chunks {
        static constexpr int kTotal = C * kChunks;
        static constexpr int kPer = (kTotal + NT - 1) / NT;
        uint4 x[kPer];
    };
    template <int NT>
    __device__ __forceinline__ static void read(const unsigned char* t, Chunks<NT>& c) {
#pragma unroll
        for (int i = 0; i < Chunks<NT>::kPer; ++i) {
            const int q = int(threadIdx.x) + i * NT;
            if (Chunks<NT>::kTotal % NT != 0 && q >= Chunks<NT>::kTotal) break;
            c.x[i] = *reinterpret_cast<const uint4*>(t + chunk_at(q));
        }
    }
    // Store chunks to rows r0 .. r0 + C - 1 of `o` (rows past the tile are
    // dropped by the buffer range), 16 bytes per thread and step.
    template <int P, int NT>
    __device__ __forceinline__ static void write(const Chunks<NT>& c, __amdgpu_buffer_rsrc_t o, int r0) {
#pragma unroll
        for (int i = 0; i < Chunks<NT>::kPer; ++i) {
            const int q = int(threadIdx.x) + i * NT;
            if (Chunks<NT>::kTotal % NT != 0 && q >= Chunks<NT>::kTotal) break;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, c.x[i]), o,
                                                   r0 * kRowBytes + 16 * q, 0, P);
        }
    }
    // The whole tile: every chunk is read before any is stored, so no store's
    // data registers are reused by a later read of the same flush.
    template <int P, int NT>
    __device__ __forceinline__ static void flush(const unsigned char* t, __amdgpu_buffer_rsrc_t o,
                                                 int r0) {
        Chunks<NT> c;
        read<NT>(t, c);
        write<P, NT>(c, o, r0);
    }
};

}  // namespace mfma
}  // namespace race
