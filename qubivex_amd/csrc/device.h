// Device-side helpers shared by the kernel translation units (kernels.hip, prefill.hip):
// kernel-side geometry, error flags, q8_0 byte permutations, the decode attention
// tile (load, MFMA scores, online softmax, P.V) and the generic per-head attention.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "fastdiv.h"
#include "internal.h"

namespace qvkv {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

// Stores that name the global address space.  A store through a pointer the compiler
// cannot place (one kept in an array, or chosen by a condition with nullptr) comes out as
// a flat store, which also counts on the LDS counter: every later LDS wait then waits
// for the store too.  st_g / st_g_nt (non-temporal) make it a global store.
template <class T>
__device__ __forceinline__ void st_g(T *p, T v) {
    *(__attribute__((address_space(1))) T *)p = v;
}
template <class T>
__device__ __forceinline__ void st_g_nt(T *p, T v) {
    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) T *)p);
}
typedef float f2v __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

enum : int { ERR_BLOCK = 1, ERR_TABLE = 2, ERR_POS = 4, ERR_OUT = 8, ERR_RANGE = 16 };

struct Geo {  // kernel-side copy of Geometry
    int dtype, G, D, B;
    uint32_t kv_out;
    uint64_t bb, k_off, ks_off, v_off, vs_off;
    uint32_t xcd_map;  // attention: XCD-aware workgroup order
    FastDiv fd_b;      // division by B
};

inline Geo to_geo(const Geometry &g) {
    return Geo{g.dtype, g.G, g.D, g.B, (uint32_t)g.kv_out, g.block_bytes,
               g.k_off, g.ks_off, g.v_off, g.vs_off, (uint32_t)tune(KNOB_ATTN_XCD),
               FastDiv((uint32_t)g.B)};
}

__device__ __forceinline__ void flag(int *err, int bit) { atomicOr(err, bit); }

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    h2 v = {(_Float16)a, (_Float16)b};  // v_cvt_f16_f32: IEEE round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

// Position of logical value d inside a stored q8_0 row.
__device__ __forceinline__ uint32_t kperm(uint32_t d, uint32_t D) {
    return ((d & 31u) >> 3) * (D >> 2) + (d >> 5) * 8u + (d & 7u);
}
__device__ __forceinline__ uint32_t vperm(uint32_t d, uint32_t D) {
    return ((d & 31u) >> 1) * (D >> 4) + 2u * (d >> 5) + (d & 1u);
}

// ---------------------------------------------------------------------------------
// The 16-position attention tile (v_mfma_f32_16x16x16_f16) of decode attention and of
// the q8_0 / d=256 prefill: loading from the pool, scores, online softmax, P.V.
// Lane l: c = l % 16 (MFMA column / K row), q = l / 16.
// ---------------------------------------------------------------------------------
constexpr float LOG2E_F = 1.4426950408889634f;

__device__ __forceinline__ h4 h4_of(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(h4, make_uint2(a, b));
}

// Four signed bytes -> four f16 (exact), one v_cvt_f16_i16 per value: SDWA selects and
// sign-extends the byte on the way in and writes one half of the result.  Each block
// defines one MFMA operand (two registers) and ends in s_nop 1: an MFMA reading a VGPR
// that a VALU instruction wrote needs 2 wait states in between, which the compiler's
// hazard recognizer does not provide after inline asm.
//   i8x4_to_h4(w): bytes 0..3 of w;  bytes_to_h4<BY>(w0..w3): byte BY of w0, w1, w2, w3.
#define QV_CVT(DST, SRC, WORD, UNUSED, BYTE)                                                    \
    "v_cvt_f16_i16_sdwa " DST ", sext(" SRC ") dst_sel:" WORD " dst_unused:" UNUSED             \
    " src0_sel:" BYTE "\n"
#define QV_CVT4(B0, B1, B2, B3)                                                                 \
    QV_CVT("%0", "%2", "WORD_0", "UNUSED_PAD", B0)                                              \
    QV_CVT("%0", "%3", "WORD_1", "UNUSED_PRESERVE", B1)                                         \
    QV_CVT("%1", "%4", "WORD_0", "UNUSED_PAD", B2)                                              \
    QV_CVT("%1", "%5", "WORD_1", "UNUSED_PRESERVE", B3) "s_nop 1"

__device__ __forceinline__ h4 i8x4_to_h4(uint32_t w) {
    uint32_t a, b;
    asm(QV_CVT4("BYTE_0", "BYTE_1", "BYTE_2", "BYTE_3")
        : "=&v"(a), "=&v"(b) : "v"(w), "v"(w), "v"(w), "v"(w));
    return h4_of(a, b);
}

// The same four conversions for a consumer that is not an MFMA (no padding).
__device__ __forceinline__ h4 i8x4_to_h4_vals(uint32_t w) {
    uint32_t a, b;
    asm(QV_CVT("%0", "%2", "WORD_0", "UNUSED_PAD", "BYTE_0")
        QV_CVT("%0", "%2", "WORD_1", "UNUSED_PRESERVE", "BYTE_1")
        QV_CVT("%1", "%2", "WORD_0", "UNUSED_PAD", "BYTE_2")
        QV_CVT("%1", "%2", "WORD_1", "UNUSED_PRESERVE", "BYTE_3")
        : "=&v"(a), "=&v"(b) : "v"(w));
    return h4_of(a, b);
}

// Two MFMA operands in one block (one s_nop for both): i8x8_to_h4x2: bytes 0..3 of w0
// and of w1; bytes_to_h4x2<BY>: byte BY, then byte BY + 1, of w0, w1, w2, w3.
__device__ __forceinline__ void i8x8_to_h4x2(uint32_t w0, uint32_t w1, h4 &x, h4 &y) {
    uint32_t a, b, c, d;
    asm(QV_CVT("%0", "%4", "WORD_0", "UNUSED_PAD", "BYTE_0")
        QV_CVT("%0", "%4", "WORD_1", "UNUSED_PRESERVE", "BYTE_1")
        QV_CVT("%1", "%4", "WORD_0", "UNUSED_PAD", "BYTE_2")
        QV_CVT("%1", "%4", "WORD_1", "UNUSED_PRESERVE", "BYTE_3")
        QV_CVT("%2", "%5", "WORD_0", "UNUSED_PAD", "BYTE_0")
        QV_CVT("%2", "%5", "WORD_1", "UNUSED_PRESERVE", "BYTE_1")
        QV_CVT("%3", "%5", "WORD_0", "UNUSED_PAD", "BYTE_2")
        QV_CVT("%3", "%5", "WORD_1", "UNUSED_PRESERVE", "BYTE_3") "s_nop 1"
        : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d) : "v"(w0), "v"(w1));
    x = h4_of(a, b);
    y = h4_of(c, d);
}
#define QV_CVT8(B0, B1)                                                                         \
    QV_CVT("%0", "%4", "WORD_0", "UNUSED_PAD", B0) QV_CVT("%0", "%5", "WORD_1", "UNUSED_PRESERVE", B0) \
    QV_CVT("%1", "%6", "WORD_0", "UNUSED_PAD", B0) QV_CVT("%1", "%7", "WORD_1", "UNUSED_PRESERVE", B0) \
    QV_CVT("%2", "%4", "WORD_0", "UNUSED_PAD", B1) QV_CVT("%2", "%5", "WORD_1", "UNUSED_PRESERVE", B1) \
    QV_CVT("%3", "%6", "WORD_0", "UNUSED_PAD", B1) QV_CVT("%3", "%7", "WORD_1", "UNUSED_PRESERVE", B1) \
    "s_nop 1"
template <int BY>
__device__ __forceinline__ void bytes_to_h4x2(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                              h4 &x, h4 &y) {
    uint32_t a, b, c, d;
    if constexpr (BY == 0)
        asm(QV_CVT8("BYTE_0", "BYTE_1")
            : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d) : "v"(w0), "v"(w1), "v"(w2), "v"(w3));
    else
        asm(QV_CVT8("BYTE_2", "BYTE_3")
            : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d) : "v"(w0), "v"(w1), "v"(w2), "v"(w3));
    x = h4_of(a, b);
    y = h4_of(c, d);
}
#undef QV_CVT8

// Bytes BY and BY + 1 of w -> two f16 (low, high half); for a non-MFMA consumer.
template <int BY>
__device__ __forceinline__ uint32_t i8x2_to_h2(uint32_t w) {
    uint32_t a;
    if constexpr (BY == 0)
        asm(QV_CVT("%0", "%1", "WORD_0", "UNUSED_PAD", "BYTE_0")
            QV_CVT("%0", "%1", "WORD_1", "UNUSED_PRESERVE", "BYTE_1") : "=&v"(a) : "v"(w));
    else
        asm(QV_CVT("%0", "%1", "WORD_0", "UNUSED_PAD", "BYTE_2")
            QV_CVT("%0", "%1", "WORD_1", "UNUSED_PRESERVE", "BYTE_3") : "=&v"(a) : "v"(w));
    return a;
}

template <int BY>
__device__ __forceinline__ h4 bytes_to_h4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    uint32_t a, b;
    if constexpr (BY == 0)
        asm(QV_CVT4("BYTE_0", "BYTE_0", "BYTE_0", "BYTE_0")
            : "=&v"(a), "=&v"(b) : "v"(w0), "v"(w1), "v"(w2), "v"(w3));
    else if constexpr (BY == 1)
        asm(QV_CVT4("BYTE_1", "BYTE_1", "BYTE_1", "BYTE_1")
            : "=&v"(a), "=&v"(b) : "v"(w0), "v"(w1), "v"(w2), "v"(w3));
    else if constexpr (BY == 2)
        asm(QV_CVT4("BYTE_2", "BYTE_2", "BYTE_2", "BYTE_2")
            : "=&v"(a), "=&v"(b) : "v"(w0), "v"(w1), "v"(w2), "v"(w3));
    else
        asm(QV_CVT4("BYTE_3", "BYTE_3", "BYTE_3", "BYTE_3")
            : "=&v"(a), "=&v"(b) : "v"(w0), "v"(w1), "v"(w2), "v"(w3));
    return h4_of(a, b);
}
#undef QV_CVT4
#undef QV_CVT

// x + x of lane l ^ 8: within each row of 16 lanes, a DPP rotate by 8.
__device__ __forceinline__ float add_xor8(float x) {
    return x + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x),
                                                                  0x128 /* row_ror:8 */, 0xf,
                                                                  0xf, false));
}

// The sum of a high part and its residual held in lanes l and l ^ 8 (lanes with hi_col
// hold the high part): hi + lo, or hi alone when hi is infinite (the residual of an
// infinite product is inf * 0 = NaN or an infinity of the other sign, where the f32
// product the split stands for is just the infinity).  Both lanes get the same value.
__device__ __forceinline__ float split_sum(float x, bool hi_col) {
    const float o = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x),
                                                                       0x128 /* row_ror:8 */, 0xf,
                                                                       0xf, false));
    const float hi = hi_col ? x : o, lo = hi_col ? o : x;
    return __builtin_isinf(hi) ? hi : hi + lo;
}
// The same for a high part in lane l and its residual in lane l ^ 32.
__device__ __forceinline__ float split_sum32(float hi, float lo) {
    return __builtin_isinf(hi) ? hi : hi + lo;
}

// max of x over lanes l, l ^ 16, l ^ 32, l ^ 48.  v_permlane16_swap (vdst, vsrc both x)
// leaves x of rows (0, 0, 2, 2) in one result and (1, 1, 3, 3) in the other; the max of
// the two is the max over l and l ^ 16.  v_permlane32_swap does the same for halves.
// Each result element is copied to a scalar before its bit_cast: hipcc's
// __builtin_bit_cast of a vector element (a[1]) reads element 0, which had turned this
// into the max of row group 0 alone.
__device__ __forceinline__ float max_xor16_32(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t a0 = a[0], a1 = a[1];
    x = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
    const uint32_t v = __builtin_bit_cast(uint32_t, x);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    const uint32_t b0 = b[0], b1 = b[1];
    return fmaxf(__builtin_bit_cast(float, b0), __builtin_bit_cast(float, b1));
}

// f32 -> (high f16, residual f16); lane columns < 8 take the high part.
// f32 product rounded once to f32, never fused into a later f16 conversion: the high
// part and the residual of a split must both come from this one rounded value.  hipcc
// contracts by default and may fuse the product into a v_fma_mix_f16 for one use (one
// rounding) but not the other, and then high + residual misses the product by one f16
// ulp of the high part wherever the two roundings disagree.
__device__ __forceinline__ float mul_rn(float a, float b) {
    float y = a * b;
    asm volatile("" : "+v"(y));  // the rounded f32 value, opaque to later fusion
    return y;
}

// a * b rounded once, with 0 * x = 0 for every x (NaN and inf included): v_mul_legacy_f32.
// Opaque to the compiler, so never contracted into a later operation either.
// The s_nop 0 is required: `a` is often a v_exp_f32 result, and on gfx950 a VALU
// instruction that reads the result of a transcendental instruction (v_exp, v_log, v_rcp,
// ...) issued just before it needs one wait state.  The compiler inserts that wait for its
// own instructions but not for inline asm, and without it the multiply read the register's
// old contents -- for v_exp_f32 vN, vN that is the exponent itself, so a masked row read
// -inf instead of 0 and -inf * scale put NaN into P.V.  The 3-wave q8_0 builds had placed
// the multiply right after the v_exp (the 4-wave builds had not).
__device__ __forceinline__ float mul_legacy(float a, float b) {
    float y;
    asm("s_nop 0\n\tv_mul_legacy_f32 %0, %1, %2" : "=v"(y) : "v"(a), "v"(b));
    return y;
}
// Four of them in one block behind one wait state.
__device__ __forceinline__ void mul_legacy4(const float a[4], const float b[4], float y[4]) {
    asm("s_nop 0\n\t"
        "v_mul_legacy_f32 %0, %4, %8\n\t"
        "v_mul_legacy_f32 %1, %5, %9\n\t"
        "v_mul_legacy_f32 %2, %6, %10\n\t"
        "v_mul_legacy_f32 %3, %7, %11"
        : "=&v"(y[0]), "=&v"(y[1]), "=&v"(y[2]), "=&v"(y[3])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]));
}

__device__ __forceinline__ _Float16 split_part(float x, bool hi_part) {
    const _Float16 hi = (_Float16)x;
    const _Float16 lo = (_Float16)(x - (float)hi);
    return hi_part ? hi : lo;
}

typedef uint32_t u2v __attribute__((ext_vector_type(2)));

// NB bytes (4, 8 or a multiple of 16) into words; NT: non-temporal (streamed once).
template <int NB, bool NT>
__device__ __forceinline__ void load_bytes(const uint8_t *p, uint32_t *w) {
    if constexpr (NB == 4) {
        w[0] = NT ? __builtin_nontemporal_load((const uint32_t *)p) : *(const uint32_t *)p;
    } else if constexpr (NB == 8) {
        const u2v x = NT ? __builtin_nontemporal_load((const u2v *)p) : *(const u2v *)p;
        w[0] = x.x; w[1] = x.y;
    } else {
#pragma unroll
        for (int i = 0; i < NB / 16; i++) {
            const u4v x = NT ? __builtin_nontemporal_load((const u4v *)(p + 16 * i))
                             : *(const u4v *)(p + 16 * i);
            w[4 * i] = x.x; w[4 * i + 1] = x.y; w[4 * i + 2] = x.z; w[4 * i + 3] = x.w;
        }
    }
}

template <int NB>
__device__ __forceinline__ void load_bytes(const uint8_t *p, uint32_t *w) {
    load_bytes<NB, false>(p, w);
}

// f16 number idx of a packed word array, as f32 (idx is a compile-time constant).
__device__ __forceinline__ float half_at(const uint32_t *w, int idx) {
    const uint32_t x = w[idx >> 1];
    return (float)__builtin_bit_cast(_Float16, (uint16_t)((idx & 1) ? (x >> 16) : (x & 0xffffu)));
}

// One 16-position tile's operands for one lane, as loaded from the pool.
template <int D, bool Q8>
struct Tile {
    static constexpr int KW = Q8 ? D / 16 : D / 8;                    // key words
    static constexpr int VW = Q8 ? (D / 64 > 0 ? D / 64 : 1) : D / 32;  // value words per row
    static constexpr int SW = Q8 ? 2 * (D / 32) : 1;                  // scale words (4 rows)
    uint32_t k[KW];
    uint32_t v[4][VW];
    uint32_t ks[SW], vs[SW];
    uint32_t p0;
    bool ok;
};

// Fused append + attention, f16 pools: the tile that holds the appended position (rel =
// its index in the tile) takes that position's key and value from the new rows kn / vn
// (this KV head's d values, f32) instead of what the pool held there, rounded to f16 as the
// append stores them (RNE); with `store`, the lanes also write them to the pool rows krow /
// vrow, which is the append itself.  Lane (c, qg) holds key d = 32 i + 8 qg .. +7 of
// position c and value d = c D/16 .. +D/16-1 of positions 4 qg .. 4 qg + 3.
template <int D>
__device__ __forceinline__ void patch_new_row(Tile<D, false> &t, uint32_t rel,
                                              const float *__restrict__ kn,
                                              const float *__restrict__ vn, uint8_t *krow,
                                              uint8_t *vrow, uint32_t c, uint32_t qg,
                                              bool store) {
    if (c == rel) {
#pragma unroll
        for (int i = 0; i < D / 32; i++) {
            const float4 a = *(const float4 *)(kn + 32 * i + 8 * qg);
            const float4 b = *(const float4 *)(kn + 32 * i + 8 * qg + 4);
            const u4v w = {pack_h2(a.x, a.y), pack_h2(a.z, a.w), pack_h2(b.x, b.y),
                           pack_h2(b.z, b.w)};
            t.k[4 * i] = w.x;
            t.k[4 * i + 1] = w.y;
            t.k[4 * i + 2] = w.z;
            t.k[4 * i + 3] = w.w;
            if (store) *(u4v *)(krow + (32 * i + 8 * qg) * 2) = w;
        }
    }
    const uint32_t vi = rel - 4 * qg;  // the value row of this lane that holds it, if any
    if (vi < 4) {
        constexpr int VW = D / 32;     // words of this lane's D/16 values
        uint32_t w[VW];
#pragma unroll
        for (int e = 0; e < VW; e++) w[e] = pack_h2(vn[c * (D / 16) + 2 * e], vn[c * (D / 16) + 2 * e + 1]);
#pragma unroll
        for (int r = 0; r < 4; r++)  // selects: a register array is not indexed by vi
#pragma unroll
            for (int e = 0; e < VW; e++) t.v[r][e] = (uint32_t)r == vi ? w[e] : t.v[r][e];
        if (store) {
#pragma unroll
            for (int e = 0; e < VW; e++) *(uint32_t *)(vrow + c * (D / 16) * 2 + 4 * e) = w[e];
        }
    }
}

// Tile tt (positions 16tt..16tt+15) of block blk (the table entry of position 16tt).
template <int D, bool Q8, bool NT>
__device__ __forceinline__ void load_tile_of(Tile<D, Q8> &t, uint32_t tt, uint32_t blk,
                                             const uint8_t *pool, uint64_t pool_blocks,
                                             uint32_t g, uint32_t c, uint32_t qg,
                                             const Geo &geo, int *err) {
    const uint32_t B = (uint32_t)geo.B;
    t.p0 = tt * 16u;
    t.ok = blk < pool_blocks;
    if (!t.ok) {
        if ((threadIdx.x & 63u) == 0) flag(err, ERR_BLOCK);
        return;
    }
    const uint8_t *base = pool + (uint64_t)blk * geo.bb;
    const uint64_t rows = (uint64_t)g * B + t.p0 % B;  // first (head, position) row of the tile
    if constexpr (!Q8) {
        // K row c: 16-byte pieces at d = 32i + 8qg; V rows 4qg..4qg+3 at d = c*D/16
        const uint8_t *kr = base + geo.k_off + ((rows + c) * D + 8 * qg) * 2u;
#pragma unroll
        for (int i = 0; i < D / 32; i++) load_bytes<16, NT>(kr + 64u * i, t.k + 4 * i);
        const uint8_t *vr = base + geo.v_off + ((rows + 4 * qg) * D + c * (D / 16)) * 2u;
#pragma unroll
        for (int i = 0; i < 4; i++) load_bytes<D / 8, NT>(vr + (uint64_t)i * D * 2u, t.v[i]);
    } else {
        load_bytes<D / 4, NT>(base + geo.k_off + (rows + c) * D + qg * (D / 4), t.k);
        load_bytes<8 * (D / 32), NT>(base + geo.ks_off + (rows + 4 * qg) * (D / 32) * 2u, t.ks);
        load_bytes<8 * (D / 32), NT>(base + geo.vs_off + (rows + 4 * qg) * (D / 32) * 2u, t.vs);
        const uint8_t *vr = base + geo.v_off + (rows + 4 * qg) * D + c * (D / 16);
#pragma unroll
        for (int i = 0; i < 4; i++) load_bytes<D / 16, NT>(vr + (uint64_t)i * D, t.v[i]);
    }
}

template <int D, bool Q8, bool NT>
__device__ __forceinline__ void load_tile(Tile<D, Q8> &t, uint32_t tt, const uint8_t *pool,
                                          uint64_t pool_blocks, const uint32_t *blocks,
                                          uint32_t tab, uint32_t g, uint32_t c, uint32_t qg,
                                          const Geo &geo, int *err) {
    load_tile_of<D, Q8, NT>(t, tt, blocks[tab + tt * 16u / (uint32_t)geo.B], pool, pool_blocks,
                            g, c, qg, geo, err);
}

// Online-softmax state of one lane: running max and partial sum (head c % 8), and the
// output accumulator (rows 4qg..4qg+3 of the MFMA tile, columns by d mapping).
template <int D>
struct SoftmaxState {
    float m, l;
    f4 acc[D / 16];
};

// (x0, x1) as an f16 pair: each x rounded to f16 (c = 0) or the residual x - f16(x) rounded
// once (c = -1), as (_Float16)fmaf(c, (float)(_Float16)x, x).  v_fma_mixlo/mixhi_f16 take the
// rounded values straight from the packed pair (op_sel_hi: source 0 is f16, op_sel picks
// the half): 4 instructions per pair instead of 8.  The pair feeds an MFMA, and a VALU
// write read by an MFMA needs 2 wait states that the compiler's hazard checks do not insert
// after inline asm: hence the s_nop.
__device__ __forceinline__ uint32_t split_sel2(float x0, float x1, float c) {
    const uint32_t u = __builtin_bit_cast(uint32_t, h2{(_Float16)x0, (_Float16)x1});
    uint32_t r;
    asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, %4 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "=&v"(r)
        : "v"(u), "v"(c), "v"(x0), "v"(x1));
    return r;
}

// PK ("packed", q8_0 with at most 4 query heads per KV head): MFMA columns c and c^4
// carry the same head (c & 3), and in the P.V step lane c's row holds the scaled
// probabilities of group 2m + sigma (sigma = (c >> 2) & 1), so one A operand serves two
// 32-value groups and each lane scales for one group instead of two.
// n_col: positions this lane's query column sees (causal limit); n_max: the largest n_col
// of the wave -- rows at or past it may never have been written and are zeroed.
template <int D, bool Q8, bool PK>
__device__ __forceinline__ void compute_tile(Tile<D, Q8> &t, SoftmaxState<D> &st,
                                             const h4 *qf, uint32_t n_col, uint32_t n_max,
                                             uint32_t qg, bool hi_col, uint32_t sigma) {
    constexpr int NJ = D / 16;
    constexpr int NG = D / 32;
    if (!t.ok) return;
    const uint32_t p0 = t.p0;
    // ---- scores S^T[position][column] = K . Q^T
    f4 s = f4{0.f, 0.f, 0.f, 0.f};
    uint32_t vw[4][Tile<D, Q8>::VW];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int x = 0; x < Tile<D, Q8>::VW; x++) vw[i][x] = t.v[i][x];
    if constexpr (!Q8) {
#pragma unroll
        for (int i = 0; i < NG; i++) {
            s = __builtin_amdgcn_mfma_f32_16x16x16f16(h4_of(t.k[4 * i], t.k[4 * i + 1]), qf[2 * i], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x16f16(h4_of(t.k[4 * i + 2], t.k[4 * i + 3]), qf[2 * i + 1], s, 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            f4 sg = f4{0.f, 0.f, 0.f, 0.f};
            h4 ka, kb;
            i8x8_to_h4x2(t.k[2 * gi], t.k[2 * gi + 1], ka, kb);
            sg = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, qf[2 * gi], sg, 0, 0, 0);
            sg = __builtin_amdgcn_mfma_f32_16x16x16f16(kb, qf[2 * gi + 1], sg, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] = fmaf(sg[i], half_at(t.ks, i * NG + gi), s[i]);
        }
    }

    // ---- high + residual columns, mask, online softmax (log2 domain)
    float sc[4];
    const bool partial = p0 + 16u > n_max;  // wave-uniform
#pragma unroll
    for (int i = 0; i < 4; i++) sc[i] = add_xor8(s[i]);
    if constexpr (!Q8) {
        // An infinite key makes the high column's q_hi k infinite and the residual's
        // inf * q_lo NaN (q_lo = 0) or an opposite infinity, where the reference's q . k is
        // just the infinity: when a sum came out NaN, redo the tile's sums with an infinite
        // high part standing alone (rare, so the common path keeps the single add).
        const bool nan_sum = (sc[0] != sc[0]) | (sc[1] != sc[1]) | (sc[2] != sc[2]) | (sc[3] != sc[3]);
        if (__builtin_expect(__any(nan_sum), 0)) {
#pragma unroll
            for (int i = 0; i < 4; i++) sc[i] = split_sum(s[i], hi_col);
        }
    }
    if (__any(p0 + 16u > n_col)) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (p0 + 4 * qg + i >= n_col) sc[i] = -INFINITY;
    }
    const float tmax = max_xor16_32(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float mnew = fmaxf(st.m, tmax);
    const float msafe = mnew == -INFINITY ? 0.0f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(st.m - msafe);
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pr[i] = __builtin_amdgcn_exp2f(sc[i] - msafe);
    st.l = st.l * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    if (__any(mnew > st.m)) {
        float ar[4];
#pragma unroll
        for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * qg + i);
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) st.acc[j][i] *= ar[i];
    }
    st.m = mnew;

    // ---- O += P . V
    if constexpr (!Q8) {
        if (partial) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (p0 + 4 * qg + i >= n_max)
#pragma unroll
                    for (int x = 0; x < D / 32; x++) vw[i][x] = 0u;
        }
        const h4 pa = h4{split_part(pr[0], hi_col), split_part(pr[1], hi_col),
                         split_part(pr[2], hi_col), split_part(pr[3], hi_col)};
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t w0 = __builtin_amdgcn_perm(vw[1][j >> 1], vw[0][j >> 1], sel);
            const uint32_t w1 = __builtin_amdgcn_perm(vw[3][j >> 1], vw[2][j >> 1], sel);
            st.acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, h4_of(w0, w1), st.acc[j], 0, 0, 0);
        }
    } else {
        // V operand of MFMA j (group j/2): rows 4qg..4qg+3 at byte j of each row's run,
        // int8 exactly as f16.  The rows' scales of group j/2 fold into the probabilities
        // (P' = p * scale in f32, then f16 high part + residual: exact to ~2^-22), so the
        // products the MFMA forms are exact.
        // Rows at or past n_max (a partial tile only) may never have been written: their
        // scales may be any f16 bits (NaN, inf).  Their p is 0 exactly (score -inf), and
        // v_mul_legacy_f32's 0 * x is 0 for every x, but the tile does not rest on that: in
        // a partial tile (wave-uniform, at most one per unit) those rows' scales and int8
        // values are zeroed before use, as the f16 branch zeroes its value rows.
        uint32_t *vs = t.vs;  // masked in place (the caller's tile is not used again)
        if (partial) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (p0 + 4 * qg + i >= n_max) {
#pragma unroll
                    for (int x = 0; x < NG / 2; x++) vs[i * (NG / 2) + x] = 0u;
#pragma unroll
                    for (int x = 0; x < Tile<D, Q8>::VW; x++) vw[i][x] = 0u;
                }
        }
        const float neg_lo = hi_col ? 0.0f : -1.0f;
        // The A operand of scaled probabilities for group g (this lane's scale pick): the f16
        // high part u of x = p * scale, or the residual x - u.
        auto scaled = [&](float sc_of_row[4]) {
            float x[4];
            mul_legacy4(pr, sc_of_row, x);
            const uint32_t a = split_sel2(x[0], x[1], neg_lo), b = split_sel2(x[2], x[3], neg_lo);
            return __builtin_bit_cast(h4, u2v{a, b});
        };
        // P'.V for the two MFMAs of group gi (bytes 2gi, 2gi+1 of each row's run): the B
        // operand of MFMA j is byte j % 4 of word j / 4 of rows 0..3, converted by SDWA.
        auto pv_group = [&](const h4 &pa, int gi) {
            const int wd = gi >> 1;  // MFMAs j = 2 gi, 2 gi + 1: bytes 2 (gi % 2), +1
            h4 b0, b1;
            if (gi & 1) bytes_to_h4x2<2>(vw[0][wd], vw[1][wd], vw[2][wd], vw[3][wd], b0, b1);
            else bytes_to_h4x2<0>(vw[0][wd], vw[1][wd], vw[2][wd], vw[3][wd], b0, b1);
            st.acc[2 * gi] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, b0, st.acc[2 * gi], 0, 0, 0);
            st.acc[2 * gi + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, b1, st.acc[2 * gi + 1], 0, 0, 0);
        };
        if constexpr (PK) {
            // Groups 2m and 2m+1 share one A operand: the scales of row i are the low and
            // high f16 of word i*NG/2 + m (row-major [row][group] f16 scales).
#pragma unroll
            for (int m = 0; m < NG / 2; m++) {
                float sc[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t w = vs[(i * NG) / 2 + m] >> (16u * sigma);
                    sc[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
                }
                const h4 pa = scaled(sc);
                pv_group(pa, 2 * m);
                pv_group(pa, 2 * m + 1);
            }
        } else {
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                float sc[4];
#pragma unroll
                for (int i = 0; i < 4; i++) sc[i] = half_at(vs, i * NG + gi);
                pv_group(scaled(sc), gi);
            }
        }
    }
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// Probabilities x0, x1 as f16 high parts (round to nearest even, packed) and the f16
// residuals x - hi: x - hi is exact in f32, so one rounding to f16 makes the residual,
// as (_Float16)(x - (float)hi) does.  v_fma_mixlo/mixhi_f16 read hi straight from the
// packed word (op_sel_hi: source 0 is f16; op_sel picks its half) instead of converting it
// back to f32 first: 6 instructions per pair instead of 14.  The residual feeds an MFMA,
// and a VALU write read by an MFMA needs 2 wait states, which the compiler's hazard
// checks do not insert for inline asm: hence the s_nop.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t &hi, uint32_t &lo) {
    hi = __builtin_bit_cast(uint32_t, h2{(_Float16)x0, (_Float16)x1});
    uint32_t r;
    asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "=&v"(r)
        : "v"(hi), "v"(x0), "v"(x1));
    lo = r;
}

// ---------------------------------------------------------------------------------
// Decode attention, generic form (any d that is a multiple of 8 up to 512, any group):
// one wave per (item, query head); lanes take 64 positions at a time for the scores,
// then d-columns for P.V.  Used where the MFMA form has no instance.
// ---------------------------------------------------------------------------------
template <bool Q8>
__device__ __forceinline__ float kv_elem(const uint8_t *base, const Geo &geo, bool isv,
                                         uint64_t row, uint32_t d) {
    const uint32_t D = (uint32_t)geo.D;
    if constexpr (!Q8) {
        return (float)((const _Float16 *)(base + (isv ? geo.v_off : geo.k_off)))[row * D + d];
    } else {
        const int8_t qv = (int8_t)base[(isv ? geo.v_off : geo.k_off) + row * D +
                                       (isv ? vperm(d, D) : kperm(d, D))];
        const float sc = (float)((const _Float16 *)(base + (isv ? geo.vs_off : geo.ks_off)))
            [row * (D >> 5) + (d >> 5)];
        return (float)qv * sc;
    }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// One wave: query row qrow of KV head g over positions 0..n-1 of table tab -> orow.
template <bool Q8>
__device__ __forceinline__ void generic_body(const uint8_t *__restrict__ pool,
                                             uint64_t pool_blocks,
                                             const uint32_t *__restrict__ blocks, uint32_t tab,
                                             uint32_t n, uint32_t g, const float *qrow,
                                             float *orow, const Geo &geo, int *err) {
    __shared__ float qs[512];
    __shared__ float ps[64];
    const uint32_t D = (uint32_t)geo.D, B = (uint32_t)geo.B;
    const uint32_t lane = threadIdx.x;
    const float scale = (1.0f / sqrtf((float)D)) * LOG2E_F;
    for (uint32_t i = lane; i < D; i += 64) qs[i] = qrow[i] * scale;
    __syncthreads();
    float m = -INFINITY, l = 0.0f, acc[8];
#pragma unroll
    for (int x = 0; x < 8; x++) acc[x] = 0.0f;
    for (uint32_t b0 = 0; b0 < n; b0 += 64) {
        const uint32_t p = b0 + lane;
        float s = -INFINITY;
        if (p < n) {
            const uint32_t blk = blocks[tab + p / B];
            if (blk < pool_blocks) {
                const uint8_t *base = pool + (uint64_t)blk * geo.bb;
                const uint64_t row = (uint64_t)g * B + p % B;
                float t = 0.0f;
                for (uint32_t d = 0; d < D; d++) t = fmaf(qs[d], kv_elem<Q8>(base, geo, false, row, d), t);
                s = t;
            } else {
                flag(err, ERR_BLOCK);
            }
        }
        const float mnew = fmaxf(m, wave_max(s));
        const float msafe = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = __builtin_amdgcn_exp2f(m - msafe);
        const float e = p < n ? __builtin_amdgcn_exp2f(s - msafe) : 0.0f;
        l = l * alpha + wave_sum(e);
#pragma unroll
        for (int x = 0; x < 8; x++) acc[x] *= alpha;
        m = mnew;
        ps[lane] = e;
        __syncthreads();
        const uint32_t cnt = min(64u, n - b0);
        for (uint32_t pp = 0; pp < cnt; pp++) {
            const uint32_t p2 = b0 + pp;
            const uint32_t blk = blocks[tab + p2 / B];
            if (blk >= pool_blocks) continue;
            const uint8_t *base = pool + (uint64_t)blk * geo.bb;
            const uint64_t row = (uint64_t)g * B + p2 % B;
            const float wgt = ps[pp];
#pragma unroll
            for (int x = 0; x < 8; x++) {
                const uint32_t d = lane + 64u * x;
                if (d < D) acc[x] = fmaf(wgt, kv_elem<Q8>(base, geo, true, row, d), acc[x]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int x = 0; x < 8; x++) {
        const uint32_t d = lane + 64u * x;
        if (d < D) orow[d] = acc[x] / l;
    }
}

}  // namespace qvkv
