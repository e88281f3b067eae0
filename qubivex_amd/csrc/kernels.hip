// HIP kernels of the paged KV-cache hot path, written for gfx950 (CDNA4, wave64).
//
// Pool layout in HBM (one block = `B` positions of one layer, all KV heads):
//   f16 : K [G][B][d] f16 | V [G][B][d] f16
//   q8_0: K int8 [G][B][d] | K scales [G][B][d/32] f16 | V int8 [G][B][d] | V scales
// Each (head, position) row of d values is contiguous, so appending one position
// writes G short contiguous runs, and a 16-position tile of one head is one
// contiguous 16*d-element run (the gather's unit and the attention's MFMA tile).
//
// q8_0 rows are stored with their bytes permuted so that each MFMA lane reads its
// operand with one contiguous load (the 32-value quantization groups are the logical
// ones, along d, as in the reference's q8_0 format):
//   K: logical d = 32*i + 8*q + t  is stored at byte  q*(d/4) + 8*i + t
//   V: logical d = 32*g + 2*c + u  is stored at byte  c*(d/16) + 2*g + u
//
// Decode attention uses v_mfma_f32_16x16x16_f16 for the GQA group contraction: a
// 16-position K tile against the group's query heads (8 columns for the heads' f16
// high parts, 8 for their f16 residuals, so q keeps ~22 significant bits), and the
// probabilities (again high part + residual) against the V tile.  Accumulation is f32.
// The score tile produced by the first MFMA is, lane for lane, the A operand of the
// second, so probabilities never leave registers.
#include <atomic>
#include <string.h>

#include "device.h"

namespace qvkv {

// ---------------------------------------------------------------------------------
// Append.  Thread = 8 consecutive values of one row of K or V (two 16-byte loads).
// f16: one 16-byte store.  q8_0: the 4 threads of a 32-value group share the group's
// absolute maximum through two lane swaps, then quantize exactly as the reference
// quantizer: d = amax/127 (f32), scale = f16(d) RNE, inv = d > 0 ? 1/d : 0 from the
// f32 d, q = clamp(round_half_away(x*inv), -127, 127), NaN -> 0.
// ---------------------------------------------------------------------------------

template <bool NT>
__device__ __forceinline__ float4 load_f4(const float *p) {
    if constexpr (NT) {
        const f4v x = __builtin_nontemporal_load((const f4v *)p);
        return make_float4(x.x, x.y, x.z, x.w);
    } else {
        return *(const float4 *)p;
    }
}

// One 8-value chunk: where it comes from and where it goes.  Work item w of a launch is
// chunk w % (2 cpr) of row w / (2 cpr): K chunks first, then V.  The divisions by 2 cpr and
// by B are invariant multiplications; DD is the head dim when known at compile time.
struct AppendItem {
    const float *src;
    uint8_t *base;     // its block
    uint32_t rowidx;   // (head, position) row inside the K or V region
    uint32_t i;        // first value's index along d
    uint32_t row, g;   // source row and KV head
    bool isv, ok;
};

// Tile order (d known at compile time): work items run over tiles of 16 consecutive rows;
// inside a tile, K heads then V heads, and for each head its 16 rows of D/8 lanes.  A
// workgroup thus covers 16 rows of one head (d = 128), and when the rows are consecutive
// positions of a block (a prefill chunk) its stores fill one contiguous block tile instead
// of short pieces of many.  fd_row divides by 16 * 2 * cpr; items past row n are padding.
struct RowChunk {
    uint32_t row, g, m;  // row, head, 8-value chunk within the head's row
    bool isv;
};
template <int DD>
__device__ __forceinline__ RowChunk row_tile_order(uint32_t w, uint32_t cpr, FastDiv fd_tile) {
    constexpr uint32_t LPR = DD / 8, PER_HEAD = 16u * LPR;
    RowChunk rc;
    const uint32_t tile = fd_tile.div(w);
    const uint32_t rem = w - tile * 32u * cpr;
    const uint32_t hv = rem / PER_HEAD;     // K heads 0..G-1, then V heads
    const uint32_t G = cpr / LPR;
    rc.isv = hv >= G;
    rc.g = rc.isv ? hv - G : hv;
    const uint32_t inh = rem % PER_HEAD;
    rc.row = tile * 16u + inh / LPR;
    rc.m = inh % LPR;
    return rc;
}

template <int DD>
__device__ __forceinline__ AppendItem append_item(uint32_t w, uint32_t total, uint32_t n,
                                                  uint32_t cpr,
                                                  FastDiv fd_row, uint8_t *pool,
                                                  uint64_t pool_blocks, const float *k,
                                                  const float *v, const uint32_t *slots,
                                                  const Geo &geo, int *err) {
    AppendItem it{};
    it.ok = false;
    if (w >= total) return it;
    const uint32_t D = DD ? (uint32_t)DD : (uint32_t)geo.D;
    uint32_t row, g;
    if constexpr (DD != 0) {
        const RowChunk rc = row_tile_order<DD>(w, cpr, fd_row);
        if (rc.row >= n) return it;
        row = rc.row;
        it.isv = rc.isv;
        g = rc.g;
        it.i = rc.m * 8u;
    } else {
        row = fd_row.div(w);
        const uint32_t rem = w - row * 2u * cpr;
        it.isv = rem >= cpr;
        const uint32_t e = (it.isv ? rem - cpr : rem) * 8u;
        g = e / D;
        it.i = e - g * D;
    }
    it.src = (it.isv ? v : k) + (uint64_t)row * geo.kv_out + g * D + it.i;
    it.row = row;
    it.g = g;
    it.ok = true;
    return it;
}

// The destination of an item whose source loads are in flight: the slot is loaded after
// them (its latency overlaps theirs: the source address does not depend on it).  A block
// id past the pool clears ok (whole rows: every lane of a q8_0 group agrees).
__device__ __forceinline__ void append_dest(AppendItem &it, uint8_t *pool, uint64_t pool_blocks,
                                            const uint32_t *slots, const Geo &geo, int *err) {
    const uint32_t slot = slots[it.row];
    const uint32_t blk = geo.fd_b.div(slot);
    if (blk >= pool_blocks) {
        flag(err, ERR_BLOCK);
        it.ok = false;
        return;
    }
    it.base = pool + (uint64_t)blk * geo.bb;
    it.rowidx = it.g * (uint32_t)geo.B + (slot - blk * (uint32_t)geo.B);
}

// U chunks per thread per round, all loads issued before any store.  (64-thread workgroups,
// which help the block copy, measured slower here: 5.09-5.24 against 5.43-5.47 TB/s.)
template <int DT, int U, bool NT, int DD, int T = 256>
__global__ __launch_bounds__(T) void k_append(uint8_t *__restrict__ pool, uint64_t pool_blocks,
                                                const float *__restrict__ k,
                                                const float *__restrict__ v,
                                                const uint32_t *__restrict__ slots, uint32_t n,
                                                FastDiv fd_row, Geo geo, int *err) {
    const uint32_t cpr = geo.kv_out >> 3;  // 8-value chunks per K (or V) row
    const uint32_t total = (DD ? (n + 15u) / 16u * 16u : n) * 2u * cpr;
    const uint32_t D = DD ? (uint32_t)DD : (uint32_t)geo.D;
    for (uint32_t b0 = blockIdx.x * (uint32_t)T * U; b0 < total; b0 += gridDim.x * (uint32_t)T * U) {
        AppendItem its[U];
        float4 xa[U], xb[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            its[u] = append_item<DD>(b0 + u * (uint32_t)T + threadIdx.x, total, n, cpr, fd_row, pool,
                                     pool_blocks, k, v, slots, geo, err);
            if (its[u].ok) {
                xa[u] = load_f4<NT>(its[u].src);
                xb[u] = load_f4<NT>(its[u].src + 4);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (its[u].ok) append_dest(its[u], pool, pool_blocks, slots, geo, err);
#pragma unroll
        for (int u = 0; u < U; u++) {
        if (!its[u].ok) continue;
        const float4 x0 = xa[u], x1 = xb[u];
        uint8_t *base = its[u].base;
        const uint64_t rowidx = its[u].rowidx;  // < 2^32: G * B rows per block
        const uint32_t i = its[u].i;
        const bool isv = its[u].isv;
        if (DT == QVKV_F16) {
            uint4 o;
            o.x = pack_h2(x0.x, x0.y);
            o.y = pack_h2(x0.z, x0.w);
            o.z = pack_h2(x1.x, x1.y);
            o.w = pack_h2(x1.z, x1.w);
            u4v* dst = (u4v *)(base + (isv ? geo.v_off : geo.k_off) + (rowidx * D + i) * 2u);
            const u4v ov = {o.x, o.y, o.z, o.w};
            if constexpr (NT) __builtin_nontemporal_store(ov, dst);
            else *dst = ov;
        } else {
            float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            float amax = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; t++) amax = fmaxf(amax, fabsf(xs[t]));
            amax = fmaxf(amax, __shfl_xor(amax, 1));
            amax = fmaxf(amax, __shfl_xor(amax, 2));
            const float d = amax / 127.0f;
            const float inv = d > 0.0f ? 1.0f / d : 0.0f;
            // roundf (half away from zero), NaN -> 0, clamp to +-127, as three instructions
            // per value: for |y| < 2^23, trunc(y + copysign(0.49999997, y)) equals roundf(y)
            // for every f32 (checked exhaustively); v_cvt_i32_f32 truncates, maps NaN to 0
            // and saturates +-inf; the clamp is then integer.  y is one rounded product.
            int qi[8];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float y = mul_rn(xs[t], inv);
                const float yr = y + __builtin_copysignf(0.49999997f, y);
                int ri;
                asm("v_cvt_i32_f32 %0, %1" : "=v"(ri) : "v"(yr));
                qi[t] = min(max(ri, -127), 127);
            }
            uint32_t qb[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t lo = __builtin_amdgcn_perm((uint32_t)qi[4 * h + 1], (uint32_t)qi[4 * h], 0x0c0c0400u);
                const uint32_t hi = __builtin_amdgcn_perm((uint32_t)qi[4 * h + 3], (uint32_t)qi[4 * h + 2], 0x0c0c0400u);
                qb[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
            }
            const uint32_t grp = i >> 5;
            if (!isv) {
                uint8_t *dst = base + geo.k_off + rowidx * D + kperm(i, D);
                *(uint2 *)dst = make_uint2(qb[0], qb[1]);
                if ((i & 31u) == 0) {
                    _Float16 sh = (_Float16)d;
                    *(_Float16 *)(base + geo.ks_off + (rowidx * (D >> 5) + grp) * 2u) = sh;
                }
            } else {
                uint8_t *dst = base + geo.v_off + rowidx * D;
                if (D == 128u) {
                    // V bytes sit at vperm(d) = 8 (d % 32 / 2) + 2 (d / 32) + d % 2: the 8-byte
                    // chunk m holds value pair m of all four 32-groups.  The lanes 4g + o
                    // (g = group, o = i % 32 / 8) of a head row hold pairs 4o..4o+3 of group g;
                    // a 4 x 4 exchange over lanes ^ 4, ^ 8, ^ 12 hands lane 4g + o chunk
                    // 4o + g whole, and the row's 16 lanes write its 128 bytes contiguously.
                    const uint32_t gl = (threadIdx.x >> 2) & 3u;  // this lane's group g
                    auto pair_of = [&](uint32_t m) { return (qb[m >> 1] >> (16u * (m & 1u))) & 0xffffu; };
                    uint32_t part[4];
                    part[gl] = pair_of(gl);
#pragma unroll
                    for (uint32_t r = 1; r < 4; r++) {
                        // lane g sends its pair g ^ r to lane g ^ r, which wants pair g ^ r
                        const uint32_t got = (uint32_t)__shfl_xor((int)pair_of(gl ^ r), (int)(4u * r));
                        part[gl ^ r] = got;
                    }
                    const uint32_t m = (i & 31u) / 2u + gl;  // this lane's chunk
                    *(uint2 *)(dst + 8u * m) = make_uint2(part[0] | (part[1] << 16), part[2] | (part[3] << 16));
                } else {
#pragma unroll
                    for (int t = 0; t < 8; t += 2) {
                        const uint32_t pair = (qb[t >> 2] >> (8 * (t & 3))) & 0xffffu;
                        *(uint16_t *)(dst + vperm(i + t, D)) = (uint16_t)pair;
                    }
                }
                if ((i & 31u) == 0) {
                    _Float16 sh = (_Float16)d;
                    *(_Float16 *)(base + geo.vs_off + (rowidx * (D >> 5) + grp) * 2u) = sh;
                }
            }
        }
        }
    }
}

// ---------------------------------------------------------------------------------
// q8_0 append for d = 64, 128, 256.  A (head, position) row of K or V is D/8 lanes; lane
// m of a row produces the 8 stored bytes at 8m of its K or V row, so every lane stores
// one aligned 8-byte piece and no bytes change lanes:
//   K: the piece at q*(D/4) + 8i holds logical d = 32i + 8q .. +7, so lane m loads
//      values 8m .. 8m+7 (i = m/4, q = m%4): its group is its quad;
//   V: byte c*(D/16) + 2g + u holds d = 32g + 2c + u, so lane m loads the 4 value pairs
//      of bytes 8m + 2j, j = 0..3; a group's pairs lie in lanes of one row.
// Group maxima are all-reduced over the lanes that hold the group with DPP row moves.
// Each lane divides for one group (amax / 127, then 1 / d, correctly rounded like the
// reference's f32 arithmetic) and a quad-broadcast hands the others their inverse.
// ---------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    // every lane read is in the executing set (rows are whole); bound_ctrl lets the move
    // fold into the consuming instruction as a DPP operand
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL,
                                                              0xF, 0xF, true));
}
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128,
             DPP_HALF_MIRROR = 0x141 };
template <int S>  // quad_perm [S, S, S, S]: every lane of a quad reads quad lane S
__device__ __forceinline__ float quad_bcast(float x) { return dpp_f<S * 0x55>(x); }

// roundf (half away from zero), NaN -> 0, clamp to +-127, as four instructions per value:
// for |y| < 2^23, trunc(y + copysign(0.49999997, y)) equals roundf(y) for every f32;
// v_cvt_i32_f32 truncates, maps NaN to 0 and saturates +-inf; the clamp is integer.
// y is one rounded product (as the reference's x * inv).
__device__ __forceinline__ int quant_q8(float x, float inv) {
    const float y = mul_rn(x, inv);
    const float yr = y + __builtin_copysignf(0.49999997f, y);
    int ri;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(ri) : "v"(yr));
    return min(max(ri, -127), 127);
}
__device__ __forceinline__ uint32_t pack_q4(int a, int b, int c, int d) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
template <bool NTS>
__device__ __forceinline__ void st_u2(uint8_t *p, uint32_t a, uint32_t b) {
    if constexpr (NTS) st_g_nt((u2v *)p, u2v{a, b});
    else st_g((u2v *)p, u2v{a, b});
}
__device__ __forceinline__ void q8_scale(float amax, float &d, float &inv) {
    d = amax / 127.0f;
    inv = d > 0.0f ? 1.0f / d : 0.0f;
}

// Fused append + attention, q8_0 pools: the tile that holds the appended position (rel =
// its index in the tile) takes that position's key and value rows quantised from the new
// rows kn / vn (this KV head's d values, f32, here staged in LDS) exactly as k_append_q8
// stores them (group maxima, q8_scale, quant_q8), instead of what the pool held there; with
// krow set (the first head chunk), the lanes also store the row's bytes and scales (krow/ks:
// K bytes and scales, vrow/vs: V bytes and scales), which is the append itself.  Lane
// (c, qg) holds the K bytes of position c for logical d = 32 i + 8 qg + e (its stored run:
// byte 8 i + e), the V bytes of positions 4 qg .. 4 qg + 3 for d = 32 g + 2 c + u (byte
// 2 g + u), and the scales of positions 4 qg .. 4 qg + 3.  Every lane quantises the slices
// it would hold (the groups' maxima over the lanes sharing a group: 4 for K, 16 for V); the
// lanes holding position rel take them.  Runs once per unit, on its last tile.  The lane
// swaps are DPP and permlane moves: with __shfl_xor (ds_bpermute) here, inside the tile
// loop, the 4-waves-per-SIMD build returned wrong outputs (its 3-wave build did not).
template <int D>
__device__ __forceinline__ void q8_patch_new_row(Tile<D, true> &t, uint32_t rel,
                                                 const float *kn, const float *vn,
                                                 uint8_t *krow, uint8_t *ks, uint8_t *vrow,
                                                 uint8_t *vs, uint32_t c, uint32_t qg) {
    constexpr int NG = D / 32;
    constexpr int VW = Tile<D, true>::VW;
    const uint32_t ri = rel - 4 * qg;  // the tile row of this lane's V rows and scales
    // K, group by group; every lane knows each group's scale after the lane swaps
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const float4 a = *(const float4 *)(kn + 32 * i + 8 * qg);
        const float4 b = *(const float4 *)(kn + 32 * i + 8 * qg + 4);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(x[e]));
        amax = max_xor16_32(amax);  // the 4 lane groups
        float d, inv;
        q8_scale(amax, d, inv);
        const uint32_t w0 = pack_q4(quant_q8(x[0], inv), quant_q8(x[1], inv),
                                    quant_q8(x[2], inv), quant_q8(x[3], inv));
        const uint32_t w1 = pack_q4(quant_q8(x[4], inv), quant_q8(x[5], inv),
                                    quant_q8(x[6], inv), quant_q8(x[7], inv));
        if (c == rel) {
            t.k[2 * i] = w0;
            t.k[2 * i + 1] = w1;
            if (krow) *(u2v *)(krow + qg * (D / 4) + 8 * i) = u2v{w0, w1};
        }
        const uint32_t sb = __builtin_bit_cast(uint16_t, (_Float16)d);
#pragma unroll
        for (int r = 0; r < 4; r++) {  // selects: a register array indexed by ri would be
            const int h = r * NG + i, wd = h >> 1, sh = 16 * (h & 1);  // moved to scratch
            t.ks[wd] = (uint32_t)r == ri ? (t.ks[wd] & ~(0xffffu << sh)) | (sb << sh) : t.ks[wd];
        }
        if (krow && c == 0 && qg == 0) *(_Float16 *)(ks + 2 * i) = (_Float16)d;
    }
    // V: this lane's two values of each group
    uint32_t vw[VW];
#pragma unroll
    for (int i = 0; i < VW; i++) vw[i] = 0u;
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const float x0 = vn[32 * g + 2 * c], x1 = vn[32 * g + 2 * c + 1];
        float amax = fmaxf(fabsf(x0), fabsf(x1));
        amax = fmaxf(amax, dpp_f<DPP_XOR1>(amax));  // the 16 lanes of the row
        amax = fmaxf(amax, dpp_f<DPP_XOR2>(amax));
        amax = fmaxf(amax, dpp_f<DPP_ROR4>(amax));
        amax = fmaxf(amax, dpp_f<DPP_ROR8>(amax));
        float d, inv;
        q8_scale(amax, d, inv);
        const uint32_t pair = ((uint32_t)quant_q8(x0, inv) & 0xffu) |
                              (((uint32_t)quant_q8(x1, inv) & 0xffu) << 8);
        vw[g >> 1] |= pair << (16 * (g & 1));  // stored bytes 2 g, 2 g + 1
        const uint32_t sb = __builtin_bit_cast(uint16_t, (_Float16)d);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int h = r * NG + g, wd = h >> 1, sh = 16 * (h & 1);
            t.vs[wd] = (uint32_t)r == ri ? (t.vs[wd] & ~(0xffffu << sh)) | (sb << sh) : t.vs[wd];
        }
        if (vrow && c == 0 && qg == 0) *(_Float16 *)(vs + 2 * g) = (_Float16)d;
    }
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < VW; i++) t.v[r][i] = (uint32_t)r == ri ? vw[i] : t.v[r][i];
    if (vrow && qg == 0) {
#pragma unroll
        for (int i = 0; i < VW; i++) *(uint32_t *)(vrow + c * (D / 16) + 4 * i) = vw[i];
    }
}

template <int U, int MODE, int D>
__global__ __launch_bounds__(256) void k_append_q8(uint8_t *__restrict__ pool,
                                                   uint64_t pool_blocks,
                                                   const float *__restrict__ k,
                                                   const float *__restrict__ v,
                                                   const uint32_t *__restrict__ slots,
                                                   uint32_t n, FastDiv fd_row, Geo geo,
                                                   int *err) {
    static_assert(D == 64 || D == 128 || D == 256, "d");
    constexpr bool NT = MODE & 1, NTS = MODE & 2;  // non-temporal loads / stores
    constexpr uint32_t P16 = D / 16;   // V: bytes per c
    const uint32_t cpr = geo.kv_out >> 3;
    const uint32_t total = (n + 15u) / 16u * 16u * 2u * cpr;
    const uint32_t B = (uint32_t)geo.B;
    for (uint32_t b0 = blockIdx.x * 256u * U; b0 < total; b0 += gridDim.x * 256u * U) {
        float x[U][8];
        uint8_t *rowk[U];   // the row's first byte in the K or V region
        uint8_t *rows[U];   // the row's first scale
        bool isv[U];
        uint32_t mm[U], rowi[U], gi[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            rowk[u] = nullptr;
            const uint32_t w = b0 + u * 256u + threadIdx.x;
            if (w >= total) continue;
            const RowChunk rc = row_tile_order<D>(w, cpr, fd_row);
            if (rc.row >= n) continue;
            const uint32_t row = rc.row, g = rc.g, m = rc.m;
            isv[u] = rc.isv;
            mm[u] = m;
            rowk[u] = (uint8_t *)1;  // (placed below, once the source loads are issued)
            rowi[u] = row;
            gi[u] = g;
            const float *src = (isv[u] ? v : k) + (uint64_t)row * geo.kv_out + g * D;
            if (!isv[u]) {
                const float4 a = load_f4<NT>(src + 8u * m), b = load_f4<NT>(src + 8u * m + 4);
                x[u][0] = a.x; x[u][1] = a.y; x[u][2] = a.z; x[u][3] = a.w;
                x[u][4] = b.x; x[u][5] = b.y; x[u][6] = b.z; x[u][7] = b.w;
            } else {
#pragma unroll
                for (uint32_t j = 0; j < 4; j++) {
                    const uint32_t by = 8u * m + 2u * j;
                    const uint32_t dd = 32u * ((by % P16) / 2u) + 2u * (by / P16);
                    const float2 p = *(const float2 *)(src + dd);
                    x[u][2 * j] = p.x;
                    x[u][2 * j + 1] = p.y;
                }
            }
        }
        // destinations: the slots load after the sources (the source address does not
        // depend on them, so the two latencies overlap)
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (!rowk[u]) continue;
            const uint32_t slot = slots[rowi[u]];
            const uint32_t blk = geo.fd_b.div(slot);
            if (blk >= pool_blocks) {  // whole rows: every lane of a group agrees
                flag(err, ERR_BLOCK);
                rowk[u] = nullptr;
                continue;
            }
            const uint32_t rowidx = gi[u] * B + (slot - blk * B);
            uint8_t *base = pool + (uint64_t)blk * geo.bb;
            rowk[u] = base + (isv[u] ? geo.v_off : geo.k_off) + (uint64_t)rowidx * D;
            rows[u] = base + (isv[u] ? geo.vs_off : geo.ks_off) + (uint64_t)rowidx * (D / 16);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (!rowk[u]) continue;
            const uint32_t m = mm[u];
            int qi[8];
            if (!isv[u]) {
                float amax = 0.0f;
#pragma unroll
                for (int t = 0; t < 8; t++) amax = fmaxf(amax, fabsf(x[u][t]));
                amax = fmaxf(amax, dpp_f<DPP_XOR1>(amax));
                amax = fmaxf(amax, dpp_f<DPP_XOR2>(amax));
                float d, inv;
                q8_scale(amax, d, inv);
#pragma unroll
                for (int t = 0; t < 8; t++) qi[t] = quant_q8(x[u][t], inv);
                st_u2<NTS>(rowk[u] + (m & 3u) * (D / 4) + (m >> 2) * 8u,
                           pack_q4(qi[0], qi[1], qi[2], qi[3]), pack_q4(qi[4], qi[5], qi[6], qi[7]));
                if ((m & 3u) == 0) st_g((_Float16 *)(rows[u] + (m >> 2) * 2u), (_Float16)d);
            } else {
                float pm[4];
#pragma unroll
                for (int j = 0; j < 4; j++) pm[j] = fmaxf(fabsf(x[u][2 * j]), fabsf(x[u][2 * j + 1]));
                float inv[4], dsc;
                if constexpr (D == 128) {
                    // pair j is group j; the group spans the row's 16 lanes
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_XOR1>(pm[j]));
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_XOR2>(pm[j]));
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_ROR4>(pm[j]));
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_ROR8>(pm[j]));
                    }
                    const uint32_t sel = m & 3u;
                    const float a = sel == 0 ? pm[0] : sel == 1 ? pm[1] : sel == 2 ? pm[2] : pm[3];
                    float is;
                    q8_scale(a, dsc, is);
                    inv[0] = quad_bcast<0>(is);
                    inv[1] = quad_bcast<1>(is);
                    inv[2] = quad_bcast<2>(is);
                    inv[3] = quad_bcast<3>(is);
                } else if constexpr (D == 64) {
                    // pairs 0, 2 are group 0 and 1, 3 group 1; a group spans the row's 8 lanes
                    float g0 = fmaxf(pm[0], pm[2]), g1 = fmaxf(pm[1], pm[3]);
                    g0 = fmaxf(g0, dpp_f<DPP_XOR1>(g0));
                    g0 = fmaxf(g0, dpp_f<DPP_XOR2>(g0));
                    g0 = fmaxf(g0, dpp_f<DPP_HALF_MIRROR>(g0));
                    g1 = fmaxf(g1, dpp_f<DPP_XOR1>(g1));
                    g1 = fmaxf(g1, dpp_f<DPP_XOR2>(g1));
                    g1 = fmaxf(g1, dpp_f<DPP_HALF_MIRROR>(g1));
                    float is;
                    q8_scale((m & 1u) ? g1 : g0, dsc, is);
                    const float i0 = quad_bcast<0>(is), i1 = quad_bcast<1>(is);
                    inv[0] = i0; inv[1] = i1; inv[2] = i0; inv[3] = i1;
                } else {
                    // pair j is group 4 (m % 2) + j; the group spans the row's 16 lanes of
                    // m's parity (lanes ^ 2, ^ 4, ^ 8, ^ 16)
                    float ds[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_XOR2>(pm[j]));
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_ROR4>(pm[j]));
                        pm[j] = fmaxf(pm[j], dpp_f<DPP_ROR8>(pm[j]));
                        pm[j] = fmaxf(pm[j], __shfl_xor(pm[j], 16));
                        q8_scale(pm[j], ds[j], inv[j]);
                    }
                    const uint32_t sel = (m >> 1) & 3u;
                    dsc = sel == 0 ? ds[0] : sel == 1 ? ds[1] : sel == 2 ? ds[2] : ds[3];
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    qi[2 * j] = quant_q8(x[u][2 * j], inv[j]);
                    qi[2 * j + 1] = quant_q8(x[u][2 * j + 1], inv[j]);
                }
                st_u2<NTS>(rowk[u] + 8u * m, pack_q4(qi[0], qi[1], qi[2], qi[3]),
                           pack_q4(qi[4], qi[5], qi[6], qi[7]));
                // scale writers: D = 64, 128: lane m < D/32 holds group m's d;
                // D = 256: lane m < 8 holds group 4 (m % 2) + m / 2
                if (m < D / 32) {
                    const uint32_t grp = D == 256 ? 4u * (m & 1u) + (m >> 1) : m;
                    st_g((_Float16 *)(rows[u] + grp * 2u), (_Float16)dsc);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------
// Gather.  Workgroup = one 16-position tile of one item, every head, K and V.
// ---------------------------------------------------------------------------------
// Output rows are written with non-temporal stores (a pure stream the kernel never reads
// back): 5.9-6.2 vs 5.6-5.7 TB/s with plain stores at cfg5.
__device__ __forceinline__ void store_f8(float *dst, const float *y) {
    st_g_nt((f4v *)dst, f4v{y[0], y[1], y[2], y[3]});
    st_g_nt((f4v *)(dst + 4), f4v{y[4], y[5], y[6], y[7]});
}

// T threads per workgroup; UF: loads in flight per thread in the f16 -> f16 copy.
template <int DT, int OUT, int T = 256, int UF = 8>
__global__ __launch_bounds__(T) void k_gather(const uint8_t *__restrict__ pool,
                                                uint64_t pool_blocks,
                                                const uint32_t *__restrict__ blocks,
                                                uint64_t n_table,
                                                const uint32_t *__restrict__ table_at,
                                                const uint32_t *__restrict__ lens,
                                                const uint64_t *__restrict__ out_at,
                                                uint32_t n_items, uint32_t tiles_max,
                                                uint64_t out_positions, void *out_k,
                                                void *out_v, uint32_t parts, Geo geo, int *err) {
    // parts workgroups share one tile (each one batch of loads and stores of it)
    const uint32_t part = blockIdx.x % parts, bt = blockIdx.x / parts;
    const uint32_t item = bt / tiles_max;
    const uint32_t tile = bt - item * tiles_max;
    if (item >= n_items) return;
    const uint32_t len = lens[item];
    const uint32_t p0 = tile * 16u;
    if (p0 >= len) return;
    const uint32_t D = (uint32_t)geo.D, B = (uint32_t)geo.B, G = (uint32_t)geo.G;
    const uint32_t tab = table_at[item];
    const uint32_t nblk = (len + B - 1) / B;
    if ((uint64_t)tab + nblk > n_table) {
        if (threadIdx.x == 0) flag(err, ERR_TABLE);
        return;
    }
    const uint64_t oat = out_at[item];
    if (oat + len > out_positions) {
        if (threadIdx.x == 0) flag(err, ERR_OUT);
        return;
    }
    const uint32_t blk = blocks[tab + p0 / B];
    if (blk >= pool_blocks) {
        if (threadIdx.x == 0) flag(err, ERR_BLOCK);
        return;
    }
    const uint32_t r0 = p0 % B;
    const uint8_t *base = pool + (uint64_t)blk * geo.bb;
    const uint32_t c8 = D >> 3;                 // 8-value chunks per row
    const uint32_t per_kv = G * 16u * c8;       // chunks per tile for K (or V)
    if (DT == QVKV_F16 && OUT == QVKV_F16) {
        // A byte copy of the tile's rows: UF loads in flight per thread, then UF stores.
        constexpr int U = UF;
        for (uint32_t b0 = part * (uint32_t)T * U; b0 < 2u * per_kv; b0 += parts * (uint32_t)T * U) {
            u4v x[U];
            uint16_t *dst[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                dst[u] = nullptr;
                const uint32_t idx = b0 + u * (uint32_t)T + threadIdx.x;
                if (idx >= 2u * per_kv) continue;
                const bool isv = idx >= per_kv;
                uint32_t r = isv ? idx - per_kv : idx;
                const uint32_t e = (r % c8) * 8u;
                r /= c8;
                const uint32_t row = r & 15u, g = r >> 4, p = p0 + row;
                if (p >= len) continue;
                x[u] = __builtin_nontemporal_load(
                    (const u4v *)(base + (isv ? geo.v_off : geo.k_off) +
                                  (((uint64_t)g * B + r0 + row) * D + e) * 2u));
                dst[u] = (uint16_t *)(isv ? out_v : out_k) + oat * (uint64_t)G * D +
                         ((uint64_t)g * len + p) * D + e;
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (dst[u]) st_g_nt((u4v *)dst[u], x[u]);
        }
        return;
    }
    if (DT == QVKV_F16 && OUT == QVKV_F32) {
        // f16 -> f32: 4 values per thread (an 8-byte load, a 16-byte store), so
        // consecutive lanes store consecutive 16-byte pieces and every store instruction
        // covers whole output lines; 8 loads in flight per thread.
        const uint32_t c4 = D >> 2;
        const uint32_t per4 = G * 16u * c4;
        constexpr int U = 8;
        for (uint32_t b0 = part * 256u * U; b0 < 2u * per4; b0 += parts * 256u * U) {
            u2v x[U];
            float *dst[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                dst[u] = nullptr;
                const uint32_t idx = b0 + u * 256u + threadIdx.x;
                if (idx >= 2u * per4) continue;
                const bool isv = idx >= per4;
                uint32_t r = isv ? idx - per4 : idx;
                const uint32_t e = (r % c4) * 4u;
                r /= c4;
                const uint32_t row = r & 15u, g = r >> 4, p = p0 + row;
                if (p >= len) continue;
                x[u] = __builtin_nontemporal_load(
                    (const u2v *)(base + (isv ? geo.v_off : geo.k_off) +
                                  (((uint64_t)g * B + r0 + row) * D + e) * 2u));
                dst[u] = (float *)(isv ? out_v : out_k) + oat * (uint64_t)G * D +
                         ((uint64_t)g * len + p) * D + e;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (!dst[u]) continue;
                const uint32_t w0 = x[u].x, w1 = x[u].y;
                const h2 a = __builtin_bit_cast(h2, w0), b = __builtin_bit_cast(h2, w1);
                st_g_nt((f4v *)dst[u], f4v{(float)a.x, (float)a.y, (float)b.x, (float)b.y});
            }
        }
        return;
    }
    for (uint32_t idx = part * 256u + threadIdx.x; idx < 2u * per_kv; idx += parts * 256u) {
        const bool isv = idx >= per_kv;
        uint32_t r = isv ? idx - per_kv : idx;
        const uint32_t e = (r % c8) * 8u;
        r /= c8;
        const uint32_t row = r & 15u;
        const uint32_t g = r >> 4;
        const uint32_t p = p0 + row;
        if (p >= len) continue;
        const uint64_t rowidx = (uint64_t)g * B + r0 + row;
        // out element offset: out_at*G*d + (g*len + p)*d + e
        const uint64_t o = oat * (uint64_t)G * D + ((uint64_t)g * len + p) * D + e;
        if (DT == QVKV_F16) {
            const uint4 x = *(const uint4 *)(base + (isv ? geo.v_off : geo.k_off) +
                                              (rowidx * D + e) * 2u);
            if (OUT == QVKV_F16) {
                st_g_nt((u4v *)((uint16_t *)(isv ? out_v : out_k) + o), u4v{x.x, x.y, x.z, x.w});
            } else {
                h2 a = __builtin_bit_cast(h2, x.x), b = __builtin_bit_cast(h2, x.y);
                h2 c = __builtin_bit_cast(h2, x.z), d2 = __builtin_bit_cast(h2, x.w);
                const float y[8] = {(float)a.x, (float)a.y, (float)b.x, (float)b.y,
                                    (float)c.x, (float)c.y, (float)d2.x, (float)d2.y};
                store_f8((float *)(isv ? out_v : out_k) + o, y);
            }
        } else {  // q8_0 -> f32: y = f32(q) * f32(scale), one multiply (the reference dequant)
            const uint8_t *rowp = base + (isv ? geo.v_off : geo.k_off) + rowidx * D;
            const _Float16 sh = *(const _Float16 *)(base + (isv ? geo.vs_off : geo.ks_off) +
                                                    (rowidx * (D >> 5) + (e >> 5)) * 2u);
            const float sc = (float)sh;
            float y[8];
            if (!isv) {
                const uint2 qb = *(const uint2 *)(rowp + kperm(e, D));
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint32_t w = t < 4 ? qb.x : qb.y;
                    y[t] = (float)(int8_t)(w >> (8 * (t & 3))) * sc;
                }
            } else {
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    const uint16_t pr = *(const uint16_t *)(rowp + vperm(e + t, D));
                    y[t] = (float)(int8_t)(pr & 0xff) * sc;
                    y[t + 1] = (float)(int8_t)(pr >> 8) * sc;
                }
            }
            store_f8((float *)(isv ? out_v : out_k) + o, y);
        }
    }
}

// q8_0 -> f32 gather for d = 64, 128, 256.  Thread = one 16-byte piece of a stored row
// (one load), dequantized and written as the contiguous logical runs it holds:
//   K (byte q*(D/4) + 8i + t holds d = 32i + 8q + t): a piece holds two 8-value runs,
//     d = 32i + 8q .. +7 and 32(i+1) + 8q .. +7;
//   V (byte c*(D/16) + 2g + u holds d = 32g + 2c + u): a piece holds NC = 256/D (>= 1)
//     consecutive c of NG = 8/NC groups, i.e. 2*NC consecutive values of each group.
// The row's D/32 f16 scales come in with one load.  8 pieces in flight per thread.
template <int D>
__device__ __forceinline__ void store_run(float *dst, const float *y, int n) {
    if (n == 8) store_f8(dst, y);
    else if (n == 4) st_g_nt((f4v *)dst, f4v{y[0], y[1], y[2], y[3]});
    else st_g_nt((f2v *)dst, f2v{y[0], y[1]});
}

// A wave's LDS writes before its reads of other lanes' data, and those reads before the
// next writes: a wave's LDS operations execute in issue order, so this waits for its LDS
// counter and keeps the compiler from moving LDS accesses across (no wave fence: on gfx9
// a fence also waits for every outstanding global load and store).
__device__ __forceinline__ void lds_order() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

template <int D>
__global__ __launch_bounds__(256) void k_gather_q8(const uint8_t *__restrict__ pool,
                                                   uint64_t pool_blocks,
                                                   const uint32_t *__restrict__ blocks,
                                                   uint64_t n_table,
                                                   const uint32_t *__restrict__ table_at,
                                                   const uint32_t *__restrict__ lens,
                                                   const uint64_t *__restrict__ out_at,
                                                   uint32_t n_items, uint32_t tiles_max,
                                                   uint64_t out_positions, float *out_k,
                                                   float *out_v, Geo geo, int *err) {
    const uint32_t item = blockIdx.x / tiles_max;
    const uint32_t tile = blockIdx.x - item * tiles_max;
    if (item >= n_items) return;
    const uint32_t len = lens[item];
    const uint32_t p0 = tile * 16u;
    if (p0 >= len) return;
    const uint32_t B = (uint32_t)geo.B, G = (uint32_t)geo.G;
    const uint32_t tab = table_at[item];
    const uint32_t nblk = (len + B - 1) / B;
    if ((uint64_t)tab + nblk > n_table) {
        if (threadIdx.x == 0) flag(err, ERR_TABLE);
        return;
    }
    const uint64_t oat = out_at[item];
    if (oat + len > out_positions) {
        if (threadIdx.x == 0) flag(err, ERR_OUT);
        return;
    }
    const uint32_t blk = blocks[tab + p0 / B];
    if (blk >= pool_blocks) {
        if (threadIdx.x == 0) flag(err, ERR_BLOCK);
        return;
    }
    const uint32_t r0 = p0 % B;
    const uint8_t *base = pool + (uint64_t)blk * geo.bb;
    // d = 128 keys: a per-wave LDS copy of the wave's 8 rows (row stride 132 floats)
    __shared__ __attribute__((aligned(16))) float kx[4][D == 128 ? 8 * 132 : 4];
    constexpr uint32_t PR = D / 16;           // pieces per row
    constexpr uint32_t NS = D / 32;           // scales per row
    constexpr uint32_t NC = D >= 256 ? 1 : 256 / D, NG = 8 / NC;
    const uint32_t per_kv = G * 16u * PR;
    constexpr int U = 8;
    for (uint32_t b0 = 0; b0 < 2u * per_kv; b0 += 256u * U) {
        u4v x[U];
        u4v sc[U];
        float *dst[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            dst[u] = nullptr;
            const uint32_t idx = b0 + u * 256u + threadIdx.x;
            if (idx >= 2u * per_kv) continue;
            const bool isv = idx >= per_kv;
            const uint32_t r = isv ? idx - per_kv : idx;
            const uint32_t j = r % PR, row = (r / PR) & 15u, g = r / (PR * 16u);
            const uint32_t p = p0 + row;
            if (p >= len) continue;
            const uint64_t rowidx = (uint64_t)g * B + r0 + row;
            x[u] = __builtin_nontemporal_load(
                (const u4v *)(base + (isv ? geo.v_off : geo.k_off) + rowidx * D + 16u * j));
            const uint8_t *sp = base + (isv ? geo.vs_off : geo.ks_off) + rowidx * NS * 2u;
            if constexpr (NS == 2) sc[u] = u4v{*(const uint32_t *)sp, 0u, 0u, 0u};
            else if constexpr (NS == 4) { const u2v t = *(const u2v *)sp; sc[u] = u4v{t.x, t.y, 0u, 0u}; }
            else sc[u] = *(const u4v *)sp;
            dst[u] = (isv ? out_v : out_k) + oat * (uint64_t)G * D + ((uint64_t)g * len + p) * D;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (!dst[u]) continue;
            const uint32_t idx = b0 + u * 256u + threadIdx.x;
            const bool isv = idx >= per_kv;
            const uint32_t j = (isv ? idx - per_kv : idx) % PR;
            const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
            auto qv = [&](uint32_t b) { return (float)(int8_t)(w[b >> 2] >> (8u * (b & 3u))); };
            auto scale = [&](uint32_t grp) {
                const uint32_t word = sc[u][grp >> 1];
                return (float)__builtin_bit_cast(_Float16, (uint16_t)(word >> (16u * (grp & 1u))));
            };
            if (!isv) {
                const uint32_t qq = (16u * j) / (D / 4), i0 = ((16u * j) % (D / 4)) / 8u;
                if constexpr (D == 128) {
                    // The piece's two 8-value runs go through the row's LDS copy in
                    // logical order, and lane j writes d = 32 k + 4 j .. +3 for k = 0..3:
                    // each store instruction then covers whole 128-byte output lines.
                    float *rowbuf = kx[threadIdx.x >> 6] + ((threadIdx.x & 63u) >> 3) * 132u;
#pragma unroll
                    for (uint32_t h = 0; h < 2; h++) {
                        const float s = scale(i0 + h);
                        float y[8];
#pragma unroll
                        for (uint32_t t = 0; t < 8; t++) y[t] = qv(8u * h + t) * s;
                        *(f4v *)(rowbuf + 32u * (i0 + h) + 8u * qq) = f4v{y[0], y[1], y[2], y[3]};
                        *(f4v *)(rowbuf + 32u * (i0 + h) + 8u * qq + 4) = f4v{y[4], y[5], y[6], y[7]};
                    }
                    lds_order();
#pragma unroll
                    for (uint32_t k = 0; k < 4; k++)
                        st_g_nt((f4v *)(dst[u] + 32u * k + 4u * j),
                                *(const f4v *)(rowbuf + 32u * k + 4u * j));
                    lds_order();
                } else {
#pragma unroll
                for (uint32_t h = 0; h < 2; h++) {
                    const float s = scale(i0 + h);
                    float y[8];
#pragma unroll
                    for (uint32_t t = 0; t < 8; t++) y[t] = qv(8u * h + t) * s;
                    store_f8(dst[u] + 32u * (i0 + h) + 8u * qq, y);
                }
                }
            } else {
                const uint32_t c0 = (16u * j) / PR, g0 = ((16u * j) % PR) / 2u;
#pragma unroll
                for (uint32_t gi = 0; gi < NG; gi++) {
                    const float s = scale(g0 + gi);
                    float y[2 * NC];
#pragma unroll
                    for (uint32_t ci = 0; ci < NC; ci++) {
                        y[2 * ci] = qv(ci * PR + 2u * gi) * s;
                        y[2 * ci + 1] = qv(ci * PR + 2u * gi + 1u) * s;
                    }
                    store_run<D>(dst[u] + 32u * (g0 + gi) + 2u * c0, y, 2 * NC);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------
// Block copy: workgroup = T threads x U x 16 bytes of one (src, dst) pair, all loads before
// stores.
// ---------------------------------------------------------------------------------
template <int U, int T = 256>
__global__ __launch_bounds__(T) void k_block_copy(uint8_t *__restrict__ pool,
                                                  uint64_t pool_blocks,
                                                  const uint32_t *__restrict__ src,
                                                  const uint32_t *__restrict__ dst,
                                                  uint32_t n, uint32_t wgs_per_block,
                                                  uint64_t bb, int *err) {
    const uint32_t pair = blockIdx.x / wgs_per_block;
    const uint32_t part = blockIdx.x - pair * wgs_per_block;
    if (pair >= n) return;
    const uint32_t s = src[pair], d = dst[pair];
    if (s >= pool_blocks || d >= pool_blocks) {
        if (threadIdx.x == 0 && part == 0) flag(err, ERR_BLOCK);
        return;
    }
    const u4v *from = (const u4v *)(pool + (uint64_t)s * bb);
    u4v *to = (u4v *)(pool + (uint64_t)d * bb);
    const uint64_t words = bb >> 4;
    const uint64_t begin = (uint64_t)part * T * U;
    u4v r[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint64_t i = begin + threadIdx.x + u * T;
        if (i < words) r[u] = __builtin_nontemporal_load(from + i);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint64_t i = begin + threadIdx.x + u * T;
        if (i < words) __builtin_nontemporal_store(r[u], to + i);
    }
}

// ---------------------------------------------------------------------------------
// Decode attention, MFMA form.  Workgroup = 4 waves on one (item, KV head, head chunk
// of <= 8 query heads, context chunk); wave w takes the chunk's tiles w, w+4, ...
// ---------------------------------------------------------------------------------
#define QV_ATTN_PARAMS                                                                          \
    const uint8_t *__restrict__ pool, uint64_t pool_blocks, const float *__restrict__ q,        \
        const uint32_t *__restrict__ blocks, uint64_t n_table,                                  \
        const uint32_t *__restrict__ table_at, const uint32_t *__restrict__ pos,                \
        uint32_t n_items, uint32_t H, uint32_t max_pos, float *__restrict__ out,                \
        float *__restrict__ ws, uint32_t hc_n, uint32_t n_chunks, uint32_t tpc, Geo geo,        \
        int *err, NewRows nr
#define QV_ATTN_ARGS                                                                            \
    pool, pool_blocks, q, blocks, n_table, table_at, pos, n_items, H, max_pos, out, ws, hc_n,   \
        n_chunks, tpc, geo, err, nr

template <int D, bool Q8, bool NT, bool PK, bool NR, bool IDS = false>
__device__ __forceinline__ void attn_body(QV_ATTN_PARAMS);
template <int D, bool Q8, bool NT, bool PK, bool NR, bool IDS = false>
__device__ __forceinline__ void attn_unit(const uint8_t *__restrict__ pool, uint64_t pool_blocks,
                                          const float *__restrict__ q,
                                          const uint32_t *__restrict__ blocks, uint32_t H,
                                          const Geo &geo, int *err, uint32_t item, uint32_t g,
                                          uint32_t hc, uint32_t n, uint32_t tab, uint32_t t_begin,
                                          uint32_t t_end, float *o_base, uint64_t o_stride,
                                          float *ml_base, uint64_t ml_stride, NewRows nr);

template <int D, bool Q8, bool NT, bool PK>
__global__ __launch_bounds__(256) void k_attn_mfma(QV_ATTN_PARAMS) {
    attn_body<D, Q8, NT, PK, false>(QV_ATTN_ARGS);
}
// The fused append + attention form (f16; new rows in nr): a separate build, so the plain
// kernel keeps its registers, held to the plain kernel's occupancy (3 waves/SIMD; 1 at
// d = 256).
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 3)))
void k_attn_mfma_nr(QV_ATTN_PARAMS) {
    attn_body<D, false, true, false, true, true>(QV_ATTN_ARGS);
}
// f16 launches of one layer's items (below 2048 units): the tile loop fetches its table
// entries ahead of the tiles (IDS; the batched launch is faster without).
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 3)))
void k_attn_mfma_ids(QV_ATTN_PARAMS) {
    attn_body<D, false, true, false, false, true>(QV_ATTN_ARGS);
}
// q8_0: held to the plain q8_0 kernel's occupancy (4 waves/SIMD at d = 128)
template <int D, bool PK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 ? 4 : 1)))
void k_attn_mfma_q8nr(QV_ATTN_PARAMS) {
    attn_body<D, true, true, PK, true>(QV_ATTN_ARGS);
}

// The same kernel held to the registers of W waves per SIMD (512 / W per lane).
template <int D, bool Q8, bool NT, bool PK, int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W)))
void k_attn_mfma_w(QV_ATTN_PARAMS) {
    attn_body<D, Q8, NT, PK, false>(QV_ATTN_ARGS);
}

template <int D, bool Q8, bool NT, bool PK, bool NR, bool IDS>
__device__ __forceinline__ void attn_body(QV_ATTN_PARAMS) {
    const uint32_t G = (uint32_t)geo.G, B = (uint32_t)geo.B;
    const uint32_t GS = H / G;
    // Workgroups are dealt to the 8 XCDs round-robin (id % 8).  With xcd_map set, logical
    // unit ids are laid out so consecutive units (the KV heads and context chunks of one
    // item, which read the same blocks) run on the same XCD and share its L2.
    uint32_t bid = blockIdx.x;
    if (geo.xcd_map) {
        const uint32_t nb = gridDim.x, qn = nb / 8, rn = nb % 8;
        const uint32_t x = bid % 8, i = bid / 8;
        bid = x < rn ? x * (qn + 1) + i : rn * (qn + 1) + (x - rn) * qn + i;
    }
    const uint32_t chunk = bid % n_chunks;
    const uint32_t unit = bid / n_chunks;
    const uint32_t hc = unit % hc_n;
    const uint32_t ug = unit / hc_n;
    const uint32_t g = ug % G;
    const uint32_t item = ug / G;
    if (item >= n_items) return;
    const uint32_t plast = pos[item];
    if (plast > max_pos) {
        if (threadIdx.x == 0) flag(err, ERR_POS);
        return;
    }
    const uint32_t n = plast + 1;
    const uint32_t ntiles = (n + 15) / 16;
    const uint32_t tab = table_at[item];
    if ((uint64_t)tab + (n + B - 1) / B > n_table) {
        if (threadIdx.x == 0) flag(err, ERR_TABLE);
        return;
    }
    const uint32_t t_begin = chunk * tpc;
    const uint32_t t_end = min(ntiles, t_begin + tpc);
    if (t_begin >= t_end) return;

    const uint64_t oh0 = (uint64_t)item * H + (uint64_t)g * GS + hc * 8;
    if (n_chunks == 1) {
        attn_unit<D, Q8, NT, PK, NR, IDS>(pool, pool_blocks, q, blocks, H, geo, err, item, g, hc, n, tab,
                                 t_begin, t_end, out + oh0 * D, D, nullptr, 0, nr);
    } else {
        float *ml = ws + (uint64_t)n_items * H * n_chunks * D;
        attn_unit<D, Q8, NT, PK, NR, IDS>(pool, pool_blocks, q, blocks, H, geo, err, item, g, hc, n, tab,
                                 t_begin, t_end, ws + (oh0 * n_chunks + chunk) * D,
                                 (uint64_t)n_chunks * D, ml + (oh0 * n_chunks + chunk) * 2,
                                 (uint64_t)n_chunks * 2, nr);
    }
}

// One unit's attention: KV head g of item `item` (positions 0..n-1, table at `tab`), query
// heads hc*8 .. hc*8+7 of its group, over 16-position tiles t_begin .. t_end-1 shared out to
// the 4 waves.  Head hh's result goes to o_base[hh * o_stride + d]: the output (ml_base
// null) or, for part of the context, the unnormalised partial with its max and sum at
// ml_base[hh * ml_stride] (log2 domain).
template <int D, bool Q8, bool NT, bool PK, bool NR, bool IDS>
__device__ __forceinline__ void attn_unit(const uint8_t *__restrict__ pool, uint64_t pool_blocks,
                                          const float *__restrict__ q,
                                          const uint32_t *__restrict__ blocks, uint32_t H,
                                          const Geo &geo, int *err, uint32_t item, uint32_t g,
                                          uint32_t hc, uint32_t n, uint32_t tab, uint32_t t_begin,
                                          uint32_t t_end, float *o_base, uint64_t o_stride,
                                          float *ml_base, uint64_t ml_stride, NewRows nr) {
    constexpr int NJ = D / 16;  // MFMA steps over d
    __shared__ float sm[4][8], sl[4][8];
    __shared__ float so[4][8][D];
    const uint32_t G = (uint32_t)geo.G, B = (uint32_t)geo.B;
    const uint32_t GS = H / G;
    const uint32_t lane = threadIdx.x & 63u;
    // q8_0: the wave index is made scalar so the tile loop and its address arithmetic run
    // on the scalar unit, leaving the vector ALUs to the dequantisation (cfg3 +8 %).  The
    // f16 kernel is faster in its vector-loop form (the scalar loop moved its accumulators
    // between AGPRs and VGPRs on every tile).
    const uint32_t w = Q8 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : threadIdx.x >> 6;
    const uint32_t c = lane & 15u, qg = lane >> 4;
    const bool hi_col = c < 8;
    const uint32_t hidx = PK ? (c & 3u) : hc * 8 + (c & 7u);  // query head within the group
    const bool hvalid = hidx < GS;
    const uint32_t sigma = (c >> 2) & 1u;  // PK: which group of a pair this lane scales for

    // q8_0 NR: the wave that will take the unit's last tile copies the new K and V rows
    // (2 d floats) into LDS first, so they are there when it reaches that tile
    __shared__ __attribute__((aligned(16))) float nrow[Q8 && NR ? 2 * D : 4];
    if constexpr (Q8 && NR) {
        const uint32_t t_last = (n - 1) / 16;
        if (t_last >= t_begin && t_last < t_end && w == (t_last - t_begin) % 4u) {
            const uint64_t at = (uint64_t)item * geo.kv_out + (uint64_t)g * D;
#pragma unroll
            for (int i = 0; i < (2 * D + 255) / 256; i++) {  // 64 lanes x 4 floats a load
                const uint32_t e = 4u * (lane + 64u * i);
                if (e < 2u * D)
                    *(float4 *)(nrow + e) = *(const float4 *)(e < D ? nr.k + at + e
                                                                    : nr.v + at + (e - D));
            }
        }
    }

    // Query fragments (B operand of QK^T): column c, k-step j holds d = dset(qg, j).
    h4 qf[NJ];
    {
        const float qs = (1.0f / sqrtf((float)D)) * LOG2E_F;
        const float *qrow = q + ((uint64_t)item * H + (uint64_t)g * GS + hidx) * D;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int d0 = 32 * (j >> 1) + 8 * (int)qg + 4 * (j & 1);
            float4 x = hvalid ? *(const float4 *)(qrow + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
            qf[j] = h4{split_part(mul_rn(x.x, qs), hi_col), split_part(mul_rn(x.y, qs), hi_col),
                       split_part(mul_rn(x.z, qs), hi_col), split_part(mul_rn(x.w, qs), hi_col)};
        }
    }

    SoftmaxState<D> st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) st.acc[j] = f4{0.f, 0.f, 0.f, 0.f};

    if constexpr (Q8) {
        // The table entries of the wave's next 64 tiles are fetched one per lane ahead of
        // the tiles; a tile's block id is then a lane read into a scalar register.
        // NR: the unit's last tile holds the appended position, patched from nrow
        const uint32_t t_last = NR ? (n - 1) / 16 : t_end;
        uint32_t ids = 0;
        for (uint32_t tt = t_begin + w, k = 0; tt < t_end; tt += 4, k = (k + 1) & 63u) {
            if (k == 0) {
                const uint32_t tl = tt + 4u * lane;
                ids = tl < t_end ? blocks[tab + tl * 16u / B] : 0u;
            }
            Tile<D, Q8> cur;
            load_tile_of<D, Q8, NT>(cur, tt, __builtin_amdgcn_readlane(ids, k), pool, pool_blocks,
                                    g, c, qg, geo, err);
            if (NR && tt == t_last && cur.ok) {  // (the block is valid)
                // the first head chunk also stores the rows
                uint8_t *base = hc == 0 ? (uint8_t *)pool + (uint64_t)blocks[tab + (n - 1) / B] * geo.bb
                                        : nullptr;
                const uint64_t rowidx = (uint64_t)g * B + (n - 1) % B;
                q8_patch_new_row<D>(cur, (n - 1) & 15u, nrow, nrow + D,
                                    base ? base + geo.k_off + rowidx * D : nullptr,
                                    base ? base + geo.ks_off + rowidx * (D / 32) * 2u : nullptr,
                                    base ? base + geo.v_off + rowidx * D : nullptr,
                                    base ? base + geo.vs_off + rowidx * (D / 32) * 2u : nullptr,
                                    c, qg);
            }
            compute_tile<D, Q8, PK>(cur, st, qf, n, n, qg, hi_col, sigma);
        }
    } else {
        // NR: the unit's last tile holds the appended position; its wave takes it after
        // the loop (the same order), so the loop body is the plain kernel's
        // IDS: the table entries of the wave's next 64 tiles are fetched one per lane ahead
        // of the tiles (as in the q8_0 loop), so a tile's loads wait on no table load.
        const uint32_t t_last = NR ? (n - 1) / 16 : t_end;
        uint32_t tt = t_begin + w;
        uint32_t ids = 0;
        for (uint32_t k = 0; tt < t_end && tt != t_last; tt += 4, k = (k + 1) & 63u) {
            if (IDS && k == 0) {
                const uint32_t tl = tt + 4u * lane;
                ids = tl < t_end ? blocks[tab + tl * 16u / B] : 0u;
            }
            Tile<D, Q8> cur;
            load_tile_of<D, Q8, NT>(cur, tt,
                                    IDS ? __builtin_amdgcn_readlane(ids, k) : blocks[tab + tt * 16u / B],
                                    pool, pool_blocks, g, c, qg, geo, err);
            compute_tile<D, Q8, PK>(cur, st, qf, n, n, qg, hi_col, sigma);
        }
        if (NR && tt < t_end) {  // tt == t_last: position n - 1 comes from the new rows
            Tile<D, Q8> cur;
            load_tile<D, Q8, NT>(cur, tt, pool, pool_blocks, blocks, tab, g, c, qg, geo, err);
            if (cur.ok) {  // (the block is valid) the first head chunk also stores the rows
                const uint32_t blk = blocks[tab + (n - 1) / B];
                uint8_t *row = (uint8_t *)pool + (uint64_t)blk * geo.bb +
                               ((uint64_t)g * B + (n - 1) % B) * D * 2u;
                const uint64_t at = (uint64_t)item * geo.kv_out + (uint64_t)g * D;
                patch_new_row<D>(cur, (n - 1) & 15u, nr.k + at, nr.v + at, row + geo.k_off,
                                 row + geo.v_off, c, qg, hc == 0);
            }
            compute_tile<D, Q8, PK>(cur, st, qf, n, n, qg, hi_col, sigma);
        }
    }
    float l = st.l;
    const float m = st.m;
    f4 *acc = st.acc;

    // ---- wave totals: l over the 4 row groups; O high rows + residual rows
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float o = __shfl_xor(acc[j][i], 32);
            // rows 0-7 hold P_hi . V, rows 8-15 P_lo . V (lanes qg < 2 keep the sum)
            acc[j][i] = Q8 ? acc[j][i] + o : split_sum32(acc[j][i], o);
        }
    if (qg == 0 && c < 8) {
        sm[w][c] = m;
        sl[w][c] = l;
    }
    if (qg < 2) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int d = Q8 ? 32 * (j >> 1) + 2 * (int)c + (j & 1) : (int)c * (D / 16) + j;
            // PK: rows 4*sigma + h hold head h for the groups with (group & 1) == sigma
            if (PK && qg != (uint32_t)((j >> 1) & 1)) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) so[w][PK ? i : 4 * qg + i][d] = acc[j][i];
        }
    }
    __syncthreads();

    // ---- merge the 4 waves; write the result or this chunk's partial
    for (uint32_t idx = threadIdx.x; idx < 8u * D; idx += 256u) {
        const uint32_t hh = idx / D, d = idx - hh * D;
        const uint32_t hi2 = hc * 8 + hh;
        if (hi2 >= GS) continue;
        float M = sm[0][hh];
#pragma unroll
        for (int x = 1; x < 4; x++) M = fmaxf(M, sm[x][hh]);
        const float Ms = M == -INFINITY ? 0.0f : M;
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const float f = sm[x][hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm[x][hh] - Ms);
            L = fmaf(sl[x][hh], f, L);
            O = fmaf(so[x][hh][d], f, O);
        }
        if (!ml_base) {
            o_base[hh * o_stride + d] = O / L;
        } else {
            o_base[hh * o_stride + d] = O;
            if (d == 0) {
                ml_base[hh * ml_stride] = M;
                ml_base[hh * ml_stride + 1] = L;
            }
        }
    }
    __syncthreads();  // the LDS above is free for the workgroup's next unit
}


// ---------------------------------------------------------------------------------
// Decode attention split by work, for launches with few units (one layer of a decode step
// in model order): the slots of every item, unit-major, are shared out evenly to the P
// workgroups, so ragged contexts leave no partial rounds of workgroups.  A unit holds
// `ucost` set-up slots (no tiles: its fixed cost in tile-equivalents) and then one slot
// per 16-position tile; a workgroup whose range holds only set-up slots of a unit skips it.  Each
// workgroup works through its range unit by unit: a unit wholly inside the range is
// written out directly; a unit cut by a range boundary leaves a partial in the
// workgroup's slot 0 (its first unit) or 1 (its last), merged by k_attn_stream_merge.
// Each workgroup computes the units' prefix sums itself from pos (n_items <= 2048).
// Workspace: partials [P][2][8][D], their (max, sum) [P][2][8][2], the prefix sums
// [n_items + 1] (u64), then at the next 16-byte boundary one record per unit for the
// merge (StreamRec; the sums and the records are written by workgroup 0).
// ---------------------------------------------------------------------------------
constexpr uint32_t STREAM_MAX_ITEMS = 2048;

// A unit's place in the split for the merge: its range of the work order lies in
// workgroups w0 .. w1 (w0 == w1: written out whole, nothing to merge), and w0 holds its
// partial in slot s0 (1 when the unit starts inside w0's range after w0's first unit).
struct StreamRec {
    uint32_t w0, w1, s0, pad;
};
__host__ __device__ constexpr uint64_t stream_rec_at(uint64_t P, uint64_t D, uint64_t n_items) {
    return (P * 2 * 8 * (D + 2) * 4 + (n_items + 1) * 8 + 15) / 16 * 16;  // bytes into ws
}

// Unit-tiles of every item before item i (cum[i]) and in total (cum[n_items]).  Items with
// a position past max_pos or a table too short count no tiles (and are reported).
__device__ __forceinline__ void stream_prefix(uint64_t *cum, const uint32_t *__restrict__ pos,
                                              const uint32_t *__restrict__ table_at,
                                              uint64_t n_table, uint32_t n_items,
                                              uint32_t max_pos, uint32_t per_unit_heads,
                                              uint32_t B, uint32_t ucost, int *err) {
    __shared__ uint64_t part[256];
    const uint32_t tid = threadIdx.x;
    const uint32_t per = (n_items + 255) / 256;  // <= 8
    uint64_t loc[8], sum = 0;
#pragma unroll
    for (uint32_t k = 0; k < 8; k++) {
        const uint32_t i = tid * per + k;
        uint64_t v = 0;
        if (k < per && i < n_items) {
            const uint32_t pl = pos[i];
            if (pl > max_pos) {
                if (blockIdx.x == 0) flag(err, ERR_POS);
            } else if ((uint64_t)table_at[i] + (pl + B) / B > n_table) {
                if (blockIdx.x == 0) flag(err, ERR_TABLE);
            } else {
                v = (uint64_t)((pl + 16) / 16 + ucost) * per_unit_heads;
            }
        }
        loc[k] = v;
        sum += v;
    }
    part[tid] = sum;
    __syncthreads();
    for (uint32_t off = 1; off < 256; off <<= 1) {
        const uint64_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    uint64_t base = tid ? part[tid - 1] : 0;
#pragma unroll
    for (uint32_t k = 0; k < 8; k++) {
        const uint32_t i = tid * per + k;
        if (k < per && i < n_items) cum[i] = base;
        base += loc[k];
    }
    if (tid == 0) cum[n_items] = part[255];
    __syncthreads();
}

// The item whose range [cum[i], cum[i+1]) holds x (x < cum[n_items]).
__device__ __forceinline__ uint32_t stream_item(const uint64_t *cum, uint32_t n_items, uint64_t x) {
    uint32_t lo = 0, hi = n_items;  // cum[lo] <= x < cum[hi]
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (cum[mid] <= x) lo = mid; else hi = mid;
    }
    return lo;
}

#define QV_STREAM_PARAMS                                                                        \
    const uint8_t *__restrict__ pool, uint64_t pool_blocks, const float *__restrict__ q,        \
        const uint32_t *__restrict__ blocks, uint64_t n_table,                                  \
        const uint32_t *__restrict__ table_at, const uint32_t *__restrict__ pos,                \
        uint32_t n_items, uint32_t H, uint32_t max_pos, float *__restrict__ out,                \
        float *__restrict__ ws, uint32_t hc_n, uint32_t ucost, Geo geo, int *err, NewRows nr

// A value every lane holds alike, moved to scalar registers.
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t uni(uint64_t v) {
    return (uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32 |
           __builtin_amdgcn_readfirstlane((uint32_t)v);
}

template <int D, bool Q8, bool NT, bool PK, bool NR>
__device__ __forceinline__ void attn_stream_body(QV_STREAM_PARAMS) {
    __shared__ uint64_t cum[STREAM_MAX_ITEMS + 1];
    const uint32_t G = (uint32_t)geo.G, B = (uint32_t)geo.B;
    const uint32_t GS = H / G;
    const uint32_t upi = G * hc_n;  // units per item
    stream_prefix(cum, pos, table_at, n_table, n_items, max_pos, upi, B, ucost, err);
    const uint64_t T = uni(cum[n_items]);
    const uint32_t P = gridDim.x, w = blockIdx.x;
    const uint64_t s0 = (uint64_t)w * T / P, s1 = (uint64_t)(w + 1) * T / P;
    float *ml = ws + (uint64_t)P * 2 * 8 * D;
    if (w == 0) {  // the prefix sums and the units' records, for the merge
        uint64_t *wc = (uint64_t *)(ml + (uint64_t)P * 2 * 8 * 2);
        for (uint32_t i = threadIdx.x; i <= n_items; i += 256) wc[i] = cum[i];
        StreamRec *rec = (StreamRec *)((uint8_t *)ws + stream_rec_at(P, D, n_items));
        for (uint32_t u = threadIdx.x; u < n_items * upi; u += 256) {
            const uint32_t item = u / upi, ul = u % upi;
            const uint64_t per_unit = (cum[item + 1] - cum[item]) / upi;
            StreamRec r{0u, 0u, 0u, 0u};
            if (per_unit != 0) {
                // the unit's slots [a0, b): ucost set-up slots, then its tiles [a, b)
                const uint64_t a0 = cum[item] + (uint64_t)ul * per_unit, a = a0 + ucost;
                const uint64_t b = a0 + per_unit;
                // workgroup holding position x: the largest v with floor(v T / P) <= x
                auto owner = [&](uint64_t x) { return (uint32_t)(((x + 1) * P + T - 1) / T - 1); };
                r.w0 = owner(a);
                r.w1 = owner(b - 1);
                // slot 1 when w0 took tiles of an earlier unit: its range starts before a0
                // (the slot before a0 is the previous unit's last tile)
                r.s0 = (uint64_t)r.w0 * T / P < a0 ? 1u : 0u;
            }
            rec[u] = r;
        }
    }
    bool first = true;
    for (uint64_t x = s0; x < s1;) {
        const uint32_t item = uni(stream_item(cum, n_items, x));
        const uint64_t c0 = uni(cum[item]);
        const uint64_t per_unit = (uni(cum[item + 1]) - c0) / upi;  // slots of a unit
        const uint64_t rel = x - c0;
        const uint32_t ul = (uint32_t)(rel / per_unit);  // unit within the item
        const uint32_t g = ul / hc_n, hc = ul % hc_n;
        const uint64_t tiles_at = c0 + (uint64_t)ul * per_unit + ucost;  // its first tile
        const uint64_t unit_end = c0 + (uint64_t)(ul + 1) * per_unit;
        const uint64_t seg_end = unit_end < s1 ? unit_end : s1;
        if (seg_end <= tiles_at) {  // only set-up slots of this unit: nothing to do
            x = seg_end;
            continue;
        }
        const uint32_t t0 = x > tiles_at ? (uint32_t)(x - tiles_at) : 0u;
        const uint32_t t1 = (uint32_t)(seg_end - tiles_at);
        const uint32_t n = uni(pos[item]) + 1, tab = uni(table_at[item]);
        const uint64_t oh0 = (uint64_t)item * H + (uint64_t)g * GS + hc * 8;
        if (t0 == 0 && seg_end == unit_end) {
            attn_unit<D, Q8, NT, PK, NR>(pool, pool_blocks, q, blocks, H, geo, err, item, g, hc, n,
                                     tab, t0, t1, out + oh0 * D, D, nullptr, 0, nr);
        } else {
            const uint64_t slot = 2ull * w + (first ? 0u : 1u);
            attn_unit<D, Q8, NT, PK, NR>(pool, pool_blocks, q, blocks, H, geo, err, item, g, hc, n,
                                     tab, t0, t1, ws + slot * 8 * D, D, ml + slot * 8 * 2, 2,
                                     nr);
        }
        first = false;
        x = seg_end;
    }
}

template <int D, bool Q8, bool NT, bool PK>
__global__ __launch_bounds__(256) void k_attn_stream(QV_STREAM_PARAMS) {
    attn_stream_body<D, Q8, NT, PK, false>(pool, pool_blocks, q, blocks, n_table, table_at, pos, n_items,
                                    H, max_pos, out, ws, hc_n, ucost, geo, err, nr);
}
template <int D, bool Q8, bool NT, bool PK, int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W)))
void k_attn_stream_w(QV_STREAM_PARAMS) {
    attn_stream_body<D, Q8, NT, PK, false>(pool, pool_blocks, q, blocks, n_table, table_at, pos, n_items,
                                    H, max_pos, out, ws, hc_n, ucost, geo, err, nr);
}
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 3)))
void k_attn_stream_nr(QV_STREAM_PARAMS) {
    attn_stream_body<D, false, true, false, true>(pool, pool_blocks, q, blocks, n_table,
                                                  table_at, pos, n_items, H, max_pos, out, ws,
                                                  hc_n, ucost, geo, err, nr);
}
// (3 waves/SIMD at d = 128: at the plain stream kernel's 4 its registers spill.  Its q8_0
// tile code is the 4-wave builds' source; the 3-wave builds' wrong outputs were the
// v_exp_f32 -> inline-asm v_mul_legacy_f32 wait state, now in the asm itself.)
template <int D, bool PK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 ? 3 : 1)))
void k_attn_stream_q8nr(QV_STREAM_PARAMS) {
    attn_stream_body<D, true, true, PK, true>(pool, pool_blocks, q, blocks, n_table, table_at,
                                              pos, n_items, H, max_pos, out, ws, hc_n, ucost, geo,
                                              err, nr);
}

// Merge for k_attn_stream: block = one (item, query head), D threads.  The unit's
// range [a, b) of the work order lies in workgroups w0 .. w1 (its StreamRec); with
// w0 == w1 it was written out whole.  Workgroup w's partial of it is in slot 1 when the
// unit starts inside w's range after its first unit, else in slot 0; workgroups between
// them with an empty range (more workgroups than tiles) hold none.  The same bookkeeping
// is restated in tests/test_attention_split.py and checked there on random shapes.
__global__ __launch_bounds__(256) void k_attn_stream_merge(const float *__restrict__ ws,
                                                           uint32_t n_items, uint32_t H,
                                                           uint32_t G, uint32_t hc_n,
                                                           uint32_t P, uint32_t D,
                                                           float *__restrict__ out) {
    const uint32_t oh = blockIdx.x;
    const uint32_t item = oh / H, h = oh % H;
    if (item >= n_items) return;
    const float *ml = ws + (uint64_t)P * 2 * 8 * D;
    const uint64_t *cum = (const uint64_t *)(ml + (uint64_t)P * 2 * 8 * 2);
    const StreamRec *recs = (const StreamRec *)((const uint8_t *)ws + stream_rec_at(P, D, n_items));
    const uint32_t GS = H / G;
    const uint32_t g = h / GS, hin = h % GS, hc = hin / 8, hh = hin % 8;
    const StreamRec r = recs[(uint64_t)item * G * hc_n + g * hc_n + hc];
    const uint64_t T = cum[n_items];  // (loaded beside the record, not after it)
    const uint32_t w0 = r.w0, w1 = r.w1;
    if (w0 == w1) return;
    // Workgroups with an empty range (only when there are fewer tiles than workgroups)
    // hold no partial.
    auto empty = [&](uint32_t w) {
        return T < P && (uint64_t)w * T / P == (uint64_t)(w + 1) * T / P;
    };
    // The unit's partials are read 4 workgroups at a time, every load of a group issued
    // before any is used (one memory round trip per group instead of one per partial);
    // they are combined in workgroup order.
    auto slot_of = [&](uint32_t w) { return 2ull * w + (w == w0 ? r.s0 : 0u); };
    float M = -INFINITY;
    for (uint32_t wb = w0; wb <= w1; wb += 4) {
        float mc[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t w = wb + k;
            mc[k] = w <= w1 && !empty(w) ? ml[(slot_of(w) * 8 + hh) * 2] : -INFINITY;
        }
#pragma unroll
        for (int k = 0; k < 4; k++) M = fmaxf(M, mc[k]);
    }
    const float Ms = M == -INFINITY ? 0.0f : M;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
        float L = 0.0f, O = 0.0f;
        for (uint32_t wb = w0; wb <= w1; wb += 4) {
            float mc[4], lc[4], oc[4];
            bool live[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t w = wb + k;
                live[k] = w <= w1 && !empty(w);
                const uint64_t slot = live[k] ? slot_of(w) : 0u;
                mc[k] = live[k] ? ml[(slot * 8 + hh) * 2] : -INFINITY;
                lc[k] = live[k] ? ml[(slot * 8 + hh) * 2 + 1] : 0.0f;
                oc[k] = live[k] ? ws[(slot * 8 + hh) * D + d] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (!live[k]) continue;
                const float f = mc[k] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc[k] - Ms);
                L = fmaf(lc[k], f, L);
                O = fmaf(oc[k], f, O);
            }
        }
        out[(uint64_t)oh * D + d] = O / L;
    }
}

// Merge of context-chunk partials: block = one (item, query head), D threads.
__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ ws,
                                                    const uint32_t *__restrict__ pos,
                                                    uint32_t n_items, uint32_t H,
                                                    uint32_t max_pos, uint32_t n_chunks,
                                                    uint32_t tpc, uint32_t D,
                                                    float *__restrict__ out) {
    const uint32_t oh = blockIdx.x;
    const uint32_t item = oh / H;
    if (item >= n_items) return;
    const uint32_t plast = pos[item];
    if (plast > max_pos) return;
    const uint32_t ntiles = (plast + 1 + 15) / 16;
    const uint32_t nch = (ntiles + tpc - 1) / tpc;
    const float *ml = ws + (uint64_t)n_items * H * n_chunks * D;
    float M = -INFINITY;
    for (uint32_t cidx = 0; cidx < nch; cidx++) M = fmaxf(M, ml[((uint64_t)oh * n_chunks + cidx) * 2]);
    const float Ms = M == -INFINITY ? 0.0f : M;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
        float L = 0.0f, O = 0.0f;
        for (uint32_t cidx = 0; cidx < nch; cidx++) {
            const uint64_t at = (uint64_t)oh * n_chunks + cidx;
            const float mc = ml[at * 2];
            const float f = mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc - Ms);
            L = fmaf(ml[at * 2 + 1], f, L);
            O = fmaf(ws[at * D + d], f, O);
        }
        out[(uint64_t)oh * D + d] = O / L;
    }
}

template <bool Q8>
__global__ __launch_bounds__(64) void k_attn_generic(
    const uint8_t *__restrict__ pool, uint64_t pool_blocks, const float *__restrict__ q,
    const uint32_t *__restrict__ blocks, uint64_t n_table, const uint32_t *__restrict__ table_at,
    const uint32_t *__restrict__ pos, uint32_t n_items, uint32_t H, uint32_t max_pos,
    float *__restrict__ out, Geo geo, int *err) {
    const uint32_t item = blockIdx.x / H, h = blockIdx.x - item * H;
    if (item >= n_items) return;
    const uint32_t B = (uint32_t)geo.B, G = (uint32_t)geo.G, D = (uint32_t)geo.D;
    const uint32_t plast = pos[item];
    if (plast > max_pos) {
        if (threadIdx.x == 0) flag(err, ERR_POS);
        return;
    }
    const uint32_t n = plast + 1;
    const uint32_t tab = table_at[item];
    if ((uint64_t)tab + (n + B - 1) / B > n_table) {
        if (threadIdx.x == 0) flag(err, ERR_TABLE);
        return;
    }
    const uint64_t row = (uint64_t)item * H + h;
    generic_body<Q8>(pool, pool_blocks, blocks, tab, n, h / (H / G), q + row * D, out + row * D,
                     geo, err);
}

// =================================================================================
// Host side: geometry and launchers.
// =================================================================================

int make_geometry(const qvkv_layout *l, Geometry *g, const char **why) {
    if (!l) { *why = "null layout"; return QVKV_E_SHAPE; }
    if (l->dtype != QVKV_F16 && l->dtype != QVKV_Q8_0) {
        *why = "pool dtype must be F16 or Q8_0";
        return QVKV_E_UNSUPPORTED;
    }
    if (l->kv_heads == 0 || l->head_dim == 0 || l->block == 0) {
        *why = "kv_heads, head_dim and block must be positive";
        return QVKV_E_SHAPE;
    }
    if (l->block % 16 != 0 || l->block > 4096) {
        *why = "block must be a multiple of 16 positions (at most 4096)";
        return QVKV_E_SHAPE;
    }
    if (l->head_dim > 512 || l->head_dim % (l->dtype == QVKV_Q8_0 ? 32 : 8) != 0) {
        *why = "head_dim must be a multiple of 8 (f16) or 32 (q8_0), at most 512";
        return QVKV_E_SHAPE;
    }
    if ((uint64_t)l->kv_heads * l->head_dim > (1u << 20)) {
        *why = "kv_heads * head_dim too large";
        return QVKV_E_SHAPE;
    }
    g->dtype = (int)l->dtype;
    g->G = (int)l->kv_heads;
    g->D = (int)l->head_dim;
    g->B = (int)l->block;
    g->kv_out = (uint64_t)l->kv_heads * l->head_dim;
    const uint64_t rows = (uint64_t)l->kv_heads * l->block;  // (head, position) rows per block
    if (l->dtype == QVKV_F16) {
        g->k_off = 0;
        g->ks_off = 0;
        g->v_off = rows * l->head_dim * 2;
        g->vs_off = 0;
        g->block_bytes = 2 * rows * l->head_dim * 2;
    } else {
        const uint64_t q = rows * l->head_dim, s = rows * (l->head_dim / 32) * 2;
        g->k_off = 0;
        g->ks_off = q;
        g->v_off = q + s;
        g->vs_off = 2 * q + s;
        g->block_bytes = 2 * (q + s);
    }
    return QVKV_OK;
}

// Launch-shape knobs: relaxed atomics, so a qvkv_tune on one thread and launches on others
// are race-free (a launch sees the old or the new value).
static const char *const kKnobName[KNOB_COUNT] = {
#define QVKV_KNOB_NAME(id, name, def) name,
    QVKV_KNOBS(QVKV_KNOB_NAME)
#undef QVKV_KNOB_NAME
};
static constexpr int kKnobDefault[KNOB_COUNT] = {
#define QVKV_KNOB_DEF(id, name, def) def,
    QVKV_KNOBS(QVKV_KNOB_DEF)
#undef QVKV_KNOB_DEF
};
static std::atomic<int> g_knob[KNOB_COUNT] = {
#define QVKV_KNOB_DEF(id, name, def) {def},
    QVKV_KNOBS(QVKV_KNOB_DEF)
#undef QVKV_KNOB_DEF
};

int tune(Knob k) { return g_knob[k].load(std::memory_order_relaxed); }

static int knob_of(const char *name) {
    if (name)
        for (int i = 0; i < KNOB_COUNT; i++)
            if (strcmp(name, kKnobName[i]) == 0) return i;
    return -1;
}

int set_tune(const char *name, int v) {
    const int i = knob_of(name);
    if (i < 0) return set_error(QVKV_E_SHAPE, "unknown knob '%s'", name ? name : "(null)");
    g_knob[i].store(v, std::memory_order_relaxed);
    return QVKV_OK;
}

int get_tune(const char *name, int *v) {
    const int i = knob_of(name);
    if (i < 0) return set_error(QVKV_E_SHAPE, "unknown knob '%s'", name ? name : "(null)");
    if (v) *v = g_knob[i].load(std::memory_order_relaxed);
    return QVKV_OK;
}

void reset_tune() {
    for (int i = 0; i < KNOB_COUNT; i++) g_knob[i].store(kKnobDefault[i], std::memory_order_relaxed);
}

// Workgroups for a grid-stride kernel over `threads` work items, at most per_cu per CU.
// A streaming kernel runs best with short-lived workgroups (one pass each): the hardware
// dispatcher then keeps every CU full through the tail, where strided loops leave
// stragglers.
static unsigned grid_for(uint64_t threads, uint64_t per_cu, uint64_t wg = 256) {
    uint64_t wgs = (threads + wg - 1) / wg;
    const uint64_t cap = 256ull * per_cu;
    return (unsigned)(wgs < 1 ? 1 : (wgs > cap ? cap : wgs));
}

hipError_t launch_append(const Geometry &g, void *pool, uint64_t pool_blocks, const float *k,
                         const float *v, const uint32_t *slots, uint32_t n, int *err,
                         hipStream_t s) {
    const Geo geo = to_geo(g);
    const uint64_t per_row = 2 * (g.kv_out / 8);
    // rows per thread group: the builds are 2 and 4, and the grid follows the build that
    // runs (3 rows per thread group measured no faster for q8_0 at cfg3: 5.41-5.43 against
    // 5.38-5.50 TB/s)
    const bool q8fast = g.dtype == QVKV_Q8_0 && (g.D == 64 || g.D == 128 || g.D == 256) &&
                        tune(KNOB_APPEND_Q8_FAST) != 0;
    const int U = tune(KNOB_APPEND_U) <= 2 ? 2 : 4;
    const uint64_t per_cu = (uint64_t)tune(KNOB_APPEND_GRID_PER_CU);
    // f16: non-temporal f32 loads and f16 stores (a pure stream); q8_0 is faster with
    // cached loads (measured at cfg3: 4.78 vs 4.40 TB/s).
    const int nt = tune(KNOB_APPEND_NT);
    const bool NT = nt < 0 ? g.dtype == QVKV_F16 : nt != 0;
    // keep the flat index inside 32 bits: launch in batches of whole 16-row tiles
    const uint32_t max_rows = (uint32_t)((0x7fffffffull / per_row)) & ~15u;
    const bool tiled = g.D == 64 || g.D == 128 || g.D == 256;
    const FastDiv fd_row((uint32_t)(tiled ? 16 * per_row : per_row));
    for (uint32_t r0 = 0; r0 < n; r0 += max_rows) {
        const uint32_t nr = n - r0 < max_rows ? n - r0 : max_rows;
        const uint64_t items = (tiled ? (uint64_t)(nr + 15) / 16 * 16 : nr) * per_row;
        const unsigned grid = grid_for((items + U - 1) / U, per_cu);
        const float *kk = k + (uint64_t)r0 * g.kv_out, *vv = v + (uint64_t)r0 * g.kv_out;
#define QV_APPEND(DT, UU, NN, DD)                                                              \
    hipLaunchKernelGGL((k_append<DT, UU, NN, DD>), dim3(grid), dim3(256), 0, s, (uint8_t *)pool,   \
                       pool_blocks, kk, vv, slots + r0, nr, fd_row, geo, err)
#define QV_APPEND_D(DT, UU, NN)                                                                \
    if (g.D == 64) QV_APPEND(DT, UU, NN, 64);                                                  \
    else if (g.D == 128) QV_APPEND(DT, UU, NN, 128);                                           \
    else if (g.D == 256) QV_APPEND(DT, UU, NN, 256);                                           \
    else QV_APPEND(DT, UU, NN, 0);
#define QV_APPEND_U(DT)                                                                        \
    if (U <= 2) { if (NT) { QV_APPEND_D(DT, 2, true) } else { QV_APPEND_D(DT, 2, false) } }    \
    else { if (NT) { QV_APPEND_D(DT, 4, true) } else { QV_APPEND_D(DT, 4, false) } }
#define QV_APPEND_Q8(UU, NN, DD)                                                               \
    hipLaunchKernelGGL((k_append_q8<UU, NN, DD>), dim3(grid), dim3(256), 0, s, (uint8_t *)pool, \
                       pool_blocks, kk, vv, slots + r0, nr, fd_row, geo, err)
#define QV_APPEND_Q8_D(UU, NN)                                                                 \
    if (g.D == 64) QV_APPEND_Q8(UU, NN, 64);                                                   \
    else if (g.D == 128) QV_APPEND_Q8(UU, NN, 128);                                            \
    else QV_APPEND_Q8(UU, NN, 256);
        if (q8fast) {
            // cached loads, non-temporal stores (measured at cfg3: 5.50 / 5.57 TB/s with cached
            // / non-temporal stores, 5.3 with non-temporal loads; 2 chunks per thread ahead of 4)
            const int mode = (NT ? 1 : 0) | (tune(KNOB_APPEND_NTS) ? 2 : 0);
#define QV_APPEND_Q8_M(UU)                                                                     \
    if (mode == 0) { QV_APPEND_Q8_D(UU, 0) } else if (mode == 1) { QV_APPEND_Q8_D(UU, 1) }     \
    else if (mode == 2) { QV_APPEND_Q8_D(UU, 2) } else { QV_APPEND_Q8_D(UU, 3) }
            if (U == 2) { QV_APPEND_Q8_M(2) } else { QV_APPEND_Q8_M(4) }
#undef QV_APPEND_Q8_M
        } else if (g.dtype == QVKV_F16) {
            QV_APPEND_U(QVKV_F16)
        } else {
            QV_APPEND_U(QVKV_Q8_0)
        }
#undef QV_APPEND_Q8_D
#undef QV_APPEND_Q8
#undef QV_APPEND_U
#undef QV_APPEND_D
#undef QV_APPEND
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gather(const Geometry &g, const void *pool, uint64_t pool_blocks,
                         const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                         const uint32_t *lens, const uint64_t *out_at, uint32_t n_items,
                         uint32_t max_len, int out_dtype, uint64_t out_positions, void *out_k,
                         void *out_v, int *err, hipStream_t s) {
    const Geo geo = to_geo(g);
    const uint32_t tiles = (max_len + 15) / 16;
    if (tiles == 0 || n_items == 0) return hipSuccess;
    const uint64_t grid = (uint64_t)tiles * n_items;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    const uint8_t *p = (const uint8_t *)pool;
    // f16 tiles of many heads: several workgroups per tile, each one batch of 8 loads in
    // flight per thread (the f16 -> f16 copy moves 8 values per load, f16 -> f32 4)
    const uint64_t per_batch = 256ull * 8 * (out_dtype == QVKV_F16 ? 8 : 4);
    const uint64_t vals = 2ull * g.G * 16 * g.D;
    uint32_t parts = tune(KNOB_GATHER_SPLIT) ? (uint32_t)((vals + per_batch - 1) / per_batch) : 1u;
    if (g.dtype != QVKV_F16 || grid * parts > 0x7fffffffull) parts = 1;
#define QV_GATHER(DT, OT)                                                                      \
    hipLaunchKernelGGL((k_gather<DT, OT>), dim3((unsigned)(grid * parts)), dim3(256), 0, s, p,  \
                       pool_blocks, blocks, n_table, table_at, lens, out_at, n_items, tiles,   \
                       out_positions, out_k, out_v, parts, geo, err)
#define QV_GATHER_Q8(DD)                                                                       \
    hipLaunchKernelGGL((k_gather_q8<DD>), dim3((unsigned)grid), dim3(256), 0, s, p,            \
                       pool_blocks, blocks, n_table, table_at, lens, out_at, n_items, tiles,   \
                       out_positions, (float *)out_k, (float *)out_v, geo, err)
    const bool q8fast = tune(KNOB_GATHER_Q8_FAST) != 0;
    if (g.dtype == QVKV_Q8_0 && q8fast && g.D == 64) QV_GATHER_Q8(64);
    else if (g.dtype == QVKV_Q8_0 && q8fast && g.D == 128) QV_GATHER_Q8(128);
    else if (g.dtype == QVKV_Q8_0 && q8fast && g.D == 256) QV_GATHER_Q8(256);
    else if (g.dtype == QVKV_F16 && out_dtype == QVKV_F16 && tune(KNOB_GATHER_T) == 64) {
        // f16 -> f16: one-wave workgroups of 4 loads per lane (4 KiB of a tile each), as for
        // the block copy.  Measured (4 runs each): cfg2 6.25-6.59 against 5.77-6.30 TB/s
        // for 256 threads x 8, cfg5 5.96-6.41 against 5.74-6.39; 1, 2 or 8 per lane slower.
        const int uf = tune(KNOB_GATHER_UF);
        const uint32_t UFv = uf >= 8 ? 8 : uf >= 4 ? 4 : uf >= 2 ? 2 : 1;
        const uint32_t parts64 = (uint32_t)((vals + 64ull * UFv * 8 - 1) / (64ull * UFv * 8));
#define QV_G64(UU)                                                                              \
    hipLaunchKernelGGL((k_gather<QVKV_F16, QVKV_F16, 64, UU>), dim3((unsigned)(grid * parts64)),  \
                       dim3(64), 0, s, p, pool_blocks, blocks, n_table, table_at, lens, out_at,  \
                       n_items, tiles, out_positions, out_k, out_v, parts64, geo, err)
        if (grid * parts64 > 0x7fffffffull) return hipErrorInvalidValue;
        if (UFv == 8) QV_G64(8); else if (UFv == 4) QV_G64(4); else if (UFv == 2) QV_G64(2);
        else QV_G64(1);
#undef QV_G64
    }
    else if (g.dtype == QVKV_F16 && out_dtype == QVKV_F16) QV_GATHER(QVKV_F16, QVKV_F16);
    else if (g.dtype == QVKV_F16) QV_GATHER(QVKV_F16, QVKV_F32);
    else QV_GATHER(QVKV_Q8_0, QVKV_F32);
#undef QV_GATHER_Q8
#undef QV_GATHER
    return hipGetLastError();
}

hipError_t launch_block_copy(const Geometry &g, void *pool, uint64_t pool_blocks,
                             const uint32_t *src, const uint32_t *dst, uint32_t n, int *err,
                             hipStream_t s) {
    if (n == 0) return hipSuccess;
    // One wave per workgroup, 16 bytes per lane (1 KiB of a pair per workgroup): many short
    // workgroups keep the most copies in flight.  Measured against 256 threads x 4 (16 KiB):
    // 32 KiB blocks 6.34-6.39 vs 5.61-5.66 TB/s, cfg4 compaction (64 KiB blocks) 5.43-5.53
    // vs 5.00-5.05; 2 or 4 per lane, 128 or 256 threads, and 8 per lane were slower.
    const int ut = tune(KNOB_COPY_U);
    const int U = ut >= 8 ? 8 : ut >= 4 ? 4 : ut >= 2 ? 2 : 1;
    const int tt = tune(KNOB_COPY_T);
    const int T = tt >= 256 ? 256 : tt >= 128 ? 128 : 64;
    const uint32_t per = (uint32_t)((g.block_bytes / 16 + (uint64_t)T * U - 1) / ((uint64_t)T * U));
    const uint64_t grid = (uint64_t)per * n;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
#define QV_BC(UU, TT)                                                                           \
    hipLaunchKernelGGL((k_block_copy<UU, TT>), dim3((unsigned)grid), dim3(TT), 0, s,             \
                       (uint8_t *)pool, pool_blocks, src, dst, n, per, g.block_bytes, err)
    if (T == 256) {
        if (U == 8) QV_BC(8, 256);
        else if (U == 4) QV_BC(4, 256);
        else if (U == 2) QV_BC(2, 256);
        else QV_BC(1, 256);
    } else if (T == 128) {
        QV_BC(1, 128);
    } else {
        if (U >= 4) QV_BC(4, 64);
        else if (U == 2) QV_BC(2, 64);
        else QV_BC(1, 64);
    }
#undef QV_BC
    return hipGetLastError();
}

int plan_attention(const Geometry &g, uint32_t n_items, uint32_t heads, uint32_t max_pos,
                   AttnPlan *p, const char **why) {
    if (heads == 0 || heads % (uint32_t)g.G != 0) {
        *why = "query heads must be a positive multiple of kv_heads";
        return QVKV_E_SHAPE;
    }
    const uint32_t GS = heads / (uint32_t)g.G;
    const bool mfma = g.D == 64 || g.D == 128 || g.D == 256;
    p->kind = mfma ? 0 : 1;
    p->hc = (GS + 7) / 8;
    p->n_chunks = 1;
    p->tpc = 0;
    p->ws_bytes = 0;
    p->ucost = 0;
    if (!mfma) {
        if ((uint64_t)n_items * heads > 0x7fffffffull) { *why = "batch too large"; return QVKV_E_SHAPE; }
        return QVKV_OK;
    }
    const uint64_t units = (uint64_t)n_items * g.G * p->hc;
    const uint64_t max_tiles = ((uint64_t)max_pos + 1 + 15) / 16;
    // workgroups to aim for: 8 per CU keeps all 256 CUs busy
    // Launches too small to fill the chip with one workgroup per unit (below 2 per CU) are
    // split.  By work (k_attn_stream, the default): every workgroup gets an equal share
    // of the (unit, tile) pairs, whatever the contexts; 768 workgroups (3 per CU, one
    // round).  Measured per layer of cfg2 (256 ragged units): 4.21 TB/s, against 3.77 for
    // the best context-chunk split and 3.98 / 3.48 with 512 / 1024 workgroups.  Launches of
    // 512 units and more (a layer of 128 x 8k, or of cfg3) run best unsplit: 6.0 and 4.8
    // TB/s, against 5.7 and 3.3-4.3 split by work.
    const uint64_t full = (uint64_t)tune(KNOB_ATTN_FULL);
    if (tune(KNOB_ATTN_STREAM) != 0 && units < full && n_items <= STREAM_MAX_ITEMS) {
        const uint64_t work = units * max_tiles;  // bound: the actual work is known on the device
        uint64_t wgs = (uint64_t)tune(KNOB_ATTN_STREAM_WG);
        if (wgs > (work + 3) / 4) wgs = (work + 3) / 4;  // at least a tile per wave
        if (wgs < 1) wgs = 1;
        p->kind = 2;
        p->n_chunks = (uint32_t)wgs;
        // Each unit also costs set-up work (its query rows, table start, the workgroup's
        // LDS merge and output) worth about 8 tiles: counting it in the shares evens out
        // workgroups that start several short units (cfg2-like layer of 32 ragged items:
        // 64.2 -> 60.1 us; contexts / 8: 31.7 -> 22.0 us; 4-24 within 2 % of 8).
        p->ucost = (uint32_t)tune(KNOB_STREAM_UNIT_COST);
        p->ws_bytes = stream_rec_at(wgs, g.D, n_items) +
                      (uint64_t)n_items * g.G * p->hc * sizeof(StreamRec);
        return QVKV_OK;
    }
    // Else (knob attn_stream=0) into context chunks, aiming at about 6 workgroups per CU.
    const uint64_t target = (uint64_t)tune(KNOB_ATTN_TARGET);
    uint64_t nch = units >= full ? 1 : (target + units - 1) / units;
    const uint64_t cap = (max_tiles + 3) / 4;  // at least one tile per wave
    if (nch > cap) nch = cap;
    if (nch < 1) nch = 1;
    uint64_t tpc = (max_tiles + nch - 1) / nch;
    nch = (max_tiles + tpc - 1) / tpc;
    if (units * nch > 0x7fffffffull) { *why = "batch too large"; return QVKV_E_SHAPE; }
    p->n_chunks = (uint32_t)nch;
    p->tpc = (uint32_t)tpc;
    p->ws_bytes = nch > 1 ? (uint64_t)n_items * heads * nch * (g.D + 2) * 4 : 0;
    return QVKV_OK;
}

bool fused_append_attention(const Geometry &g) {
    return (g.dtype == QVKV_F16 || tune(KNOB_FUSED_Q8) != 0) &&
           (g.D == 64 || g.D == 128 || g.D == 256);
}

__global__ __launch_bounds__(256) void k_slots_at(const uint32_t *__restrict__ blocks,
                                                  uint64_t n_table,
                                                  const uint32_t *__restrict__ table_at,
                                                  const uint32_t *__restrict__ pos,
                                                  uint32_t n_items, uint32_t max_pos, uint32_t B,
                                                  uint32_t *__restrict__ slots, int *err) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n_items) return;
    const uint32_t p = pos[i];
    uint32_t slot = 0xffffffffu;
    if (p > max_pos) flag(err, ERR_POS);
    else if ((uint64_t)table_at[i] + p / B >= n_table) flag(err, ERR_TABLE);
    else slot = blocks[table_at[i] + p / B] * B + p % B;
    slots[i] = slot;
}

__global__ __launch_bounds__(256) void k_table_scatter(const uint32_t *__restrict__ staged,
                                                      uint32_t n_pos, uint64_t n_pairs,
                                                      uint32_t *__restrict__ pos,
                                                      uint32_t *__restrict__ lens,
                                                      uint32_t *__restrict__ blocks) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n_pos) {
        pos[i] = staged[i];
        lens[i] = staged[i] + 1;
    }
    if (i < n_pairs) blocks[staged[n_pos + 2 * i]] = staged[n_pos + 2 * i + 1];
}

hipError_t launch_table_scatter(const uint32_t *staged, uint32_t n_pos, uint64_t n_pairs,
                                uint32_t *pos, uint32_t *lens, uint32_t *blocks, hipStream_t s) {
    const uint64_t n = n_pos > n_pairs ? n_pos : n_pairs;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_table_scatter, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, staged,
                       n_pos, n_pairs, pos, lens, blocks);
    return hipGetLastError();
}

hipError_t launch_slots_at(const Geometry &g, const uint32_t *blocks, uint64_t n_table,
                           const uint32_t *table_at, const uint32_t *pos, uint32_t n_items,
                           uint32_t max_pos, uint32_t *slots, int *err, hipStream_t s) {
    if (n_items == 0) return hipSuccess;
    hipLaunchKernelGGL(k_slots_at, dim3((n_items + 255) / 256), dim3(256), 0, s, blocks, n_table,
                       table_at, pos, n_items, max_pos, (uint32_t)g.B, slots, err);
    return hipGetLastError();
}

hipError_t launch_attention(const Geometry &g, const AttnPlan &p, const void *pool,
                            uint64_t pool_blocks, const float *q, const uint32_t *blocks,
                            uint64_t n_table, const uint32_t *table_at, const uint32_t *pos,
                            uint32_t n_items, uint32_t heads, uint32_t max_pos, float *out,
                            void *ws, int *err, hipStream_t s, NewRows nr) {
    if (n_items == 0) return hipSuccess;
    const Geo geo = to_geo(g);
    const uint8_t *pp = (const uint8_t *)pool;
    if (p.kind == 1) {
        if (g.dtype == QVKV_F16)
            hipLaunchKernelGGL(k_attn_generic<false>, dim3(n_items * heads), dim3(64), 0, s, pp,
                               pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads,
                               max_pos, out, geo, err);
        else
            hipLaunchKernelGGL(k_attn_generic<true>, dim3(n_items * heads), dim3(64), 0, s, pp,
                               pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads,
                               max_pos, out, geo, err);
        return hipGetLastError();
    }
    float *wsf = (float *)ws;
    const bool q8 = g.dtype == QVKV_Q8_0;
    // q8_0 at d = 128 runs its 4-wave builds (k_attn_mfma_w / k_attn_stream_w): its dequant
    // VALU work needs the extra wave (4.82 vs 4.14 TB/s at cfg3).  The 3-wave builds
    // (knob attn_waves3_q8) are kept for measurement and tested like the others.  f16
    // selects its 4-wave build by the knob attn_waves4_f16 (measured slower).
    const bool w4 = q8 ? tune(KNOB_ATTN_WAVES3_Q8) == 0 : tune(KNOB_ATTN_WAVES4_F16) != 0;
    // q8_0 with <= 4 query heads per KV head: two groups' probabilities per A operand
    const bool pk = q8 && heads / (uint32_t)g.G <= 4 && tune(KNOB_ATTN_PACK) != 0;
    if (p.kind == 2) {
        const unsigned P = p.n_chunks;
#define QV_AS(DD, QQ, PK)                                                                       \
    hipLaunchKernelGGL((k_attn_stream<DD, QQ, true, PK>), dim3(P), dim3(256), 0, s, pp,          \
                       pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads, max_pos,  \
                       out, wsf, p.hc, p.ucost, geo, err, nr)
#define QV_AS_NR(DD)                                                                            \
    hipLaunchKernelGGL((k_attn_stream_nr<DD>), dim3(P), dim3(256), 0, s,                        \
                       pp, pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads,      \
                       max_pos, out, wsf, p.hc, p.ucost, geo, err, nr)
#define QV_AS_W4(DD, QQ, PK)                                                                    \
    hipLaunchKernelGGL((k_attn_stream_w<DD, QQ, true, PK, 4>), dim3(P), dim3(256), 0, s, pp,     \
                       pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads, max_pos,  \
                       out, wsf, p.hc, p.ucost, geo, err, nr)
#define QV_AS_Q8NR(DD, PK)                                                                      \
    hipLaunchKernelGGL((k_attn_stream_q8nr<DD, PK>), dim3(P), dim3(256), 0, s, pp, pool_blocks,  \
                       q, blocks, n_table, table_at, pos, n_items, heads, max_pos, out, wsf,    \
                       p.hc, p.ucost, geo, err, nr)
        if (q8 && nr.k) {
            if (g.D == 64) { if (pk) QV_AS_Q8NR(64, true); else QV_AS_Q8NR(64, false); }
            else if (g.D == 128) { if (pk) QV_AS_Q8NR(128, true); else QV_AS_Q8NR(128, false); }
            else { if (pk) QV_AS_Q8NR(256, true); else QV_AS_Q8NR(256, false); }
        } else if (g.D == 64) {
            if (!q8) { if (nr.k) QV_AS_NR(64); else QV_AS(64, false, false); }
            else if (pk) QV_AS(64, true, true);
            else QV_AS(64, true, false);
        } else if (g.D == 128) {
            if (!q8) {
                if (nr.k) QV_AS_NR(128);
                else if (w4) QV_AS_W4(128, false, false);
                else QV_AS(128, false, false);
            }
            else if (pk) { if (w4) QV_AS_W4(128, true, true); else QV_AS(128, true, true); }
            else { if (w4) QV_AS_W4(128, true, false); else QV_AS(128, true, false); }
        } else {
            if (!q8) { if (nr.k) QV_AS_NR(256); else QV_AS(256, false, false); }
            else if (pk) QV_AS(256, true, true);
            else QV_AS(256, true, false);
        }
#undef QV_AS_Q8NR
#undef QV_AS_NR
#undef QV_AS_W4
#undef QV_AS
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_attn_stream_merge, dim3(n_items * heads), dim3(g.D), 0, s,
                           (const float *)ws, n_items, heads, (uint32_t)g.G, p.hc, P,
                           (uint32_t)g.D, out);
        return hipGetLastError();
    }
    const uint64_t grid = (uint64_t)n_items * g.G * p.hc * p.n_chunks;
    // f16, d = 128, launches of one layer's items (cfg5: 512 workgroups): the table entries
    // fetched ahead of the tiles (per layer cfg5 16.7-17.2 -> 16.2 ms per step; the batched
    // launch of every layer lost 2-4 % with it)
    const bool per_layer = grid < (uint64_t)tune(KNOB_ATTN_IDS_BELOW);
    // K/V tiles are streamed with non-temporal loads (read once).
    // Occupancy: `mode` 0 is the compiler's register choice (3 waves/SIMD at d=128), 4
    // holds the kernel to 4 waves per SIMD (125 VGPRs, no spill).  Measured (cfg5 f16,
    // cfg3 q8_0): f16 is best at 0 (6.48 vs 5.90 TB/s), q8_0 at 4 (4.82 vs 4.14 TB/s):
    // the q8_0 tile has about twice the VALU work per byte and more waves hide it.
    // Software pipelining one tile ahead (2 waves/SIMD) and 5 waves/SIMD (spills) were
    // slower for both.
#define QV_ATTN(DD, QQ, PK)                                                                     \
    hipLaunchKernelGGL((k_attn_mfma<DD, QQ, true, PK>), dim3((unsigned)grid), dim3(256), 0, s,  \
                       pp, pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads,      \
                       max_pos, out, wsf, p.hc, p.n_chunks, p.tpc, geo, err, nr)
#define QV_ATTN_W4(DD, QQ, PK)                                                                  \
    hipLaunchKernelGGL((k_attn_mfma_w<DD, QQ, true, PK, 4>), dim3((unsigned)grid), dim3(256),   \
                       0, s, pp, pool_blocks, q, blocks, n_table, table_at, pos, n_items,       \
                       heads, max_pos, out, wsf, p.hc, p.n_chunks, p.tpc, geo, err, nr)
#define QV_ATTN_NR(DD)                                                                          \
    hipLaunchKernelGGL((k_attn_mfma_nr<DD>), dim3((unsigned)grid),                              \
                       dim3(256), 0, s, pp, pool_blocks, q, blocks, n_table, table_at, pos,     \
                       n_items, heads, max_pos, out, wsf, p.hc, p.n_chunks, p.tpc, geo, err, nr)
#define QV_ATTN_IDS(DD)                                                                         \
    hipLaunchKernelGGL((k_attn_mfma_ids<DD>), dim3((unsigned)grid), dim3(256), 0, s, pp,        \
                       pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads, max_pos,  \
                       out, wsf, p.hc, p.n_chunks, p.tpc, geo, err, nr)
#define QV_ATTN_Q8NR(DD, PK)                                                                    \
    hipLaunchKernelGGL((k_attn_mfma_q8nr<DD, PK>), dim3((unsigned)grid), dim3(256), 0, s, pp,    \
                       pool_blocks, q, blocks, n_table, table_at, pos, n_items, heads, max_pos,  \
                       out, wsf, p.hc, p.n_chunks, p.tpc, geo, err, nr)
    if (q8 && nr.k) {
        if (g.D == 64) { if (pk) QV_ATTN_Q8NR(64, true); else QV_ATTN_Q8NR(64, false); }
        else if (g.D == 128) { if (pk) QV_ATTN_Q8NR(128, true); else QV_ATTN_Q8NR(128, false); }
        else { if (pk) QV_ATTN_Q8NR(256, true); else QV_ATTN_Q8NR(256, false); }
    } else if (g.D == 64) {
        if (!q8) { if (nr.k) QV_ATTN_NR(64); else QV_ATTN(64, false, false); }
        else if (pk) QV_ATTN(64, true, true);
        else QV_ATTN(64, true, false);
    } else if (g.D == 128) {
        if (!q8) {
            if (nr.k) QV_ATTN_NR(128);
            else if (w4) QV_ATTN_W4(128, false, false);
            else if (per_layer) QV_ATTN_IDS(128);
            else QV_ATTN(128, false, false);
        }
        else if (pk) { if (w4) QV_ATTN_W4(128, true, true); else QV_ATTN(128, true, true); }
        else { if (w4) QV_ATTN_W4(128, true, false); else QV_ATTN(128, true, false); }
    } else {
        if (!q8) { if (nr.k) QV_ATTN_NR(256); else QV_ATTN(256, false, false); }
        else if (pk) QV_ATTN(256, true, true);
        else QV_ATTN(256, true, false);
    }
#undef QV_ATTN_Q8NR
#undef QV_ATTN_IDS
#undef QV_ATTN_NR
#undef QV_ATTN_W4
#undef QV_ATTN
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.n_chunks == 1) return e;
    hipLaunchKernelGGL(k_attn_merge, dim3(n_items * heads), dim3(g.D), 0, s, (const float *)ws,
                       pos, n_items, heads, max_pos, p.n_chunks, p.tpc, (uint32_t)g.D, out);
    return hipGetLastError();
}

}  // namespace qvkv
