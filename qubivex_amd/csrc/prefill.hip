// Paged prefill attention kernels (gfx950): causal attention of segments of
// consecutive stored tokens over the paged pool.  Built with MFMA operands in VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form): the online-softmax rescale and the P split work on
// the accumulators with plain VALU ops instead of copying them to and from AGPRs.
#include "device.h"

namespace qvkv {

// ---------------------------------------------------------------------------------
// Paged prefill attention: segment i holds n_tok[i] consecutive tokens of one sequence at
// positions pos0[i], pos0[i]+1, ... (q / out rows q_at[i] + j); token j attends over
// positions 0..pos0[i]+j of its table (causal), after all of the segment's rows are stored.
// Workgroup = (segment, KV head, block of 32 query columns); a query column is one
// (token, head) pair, column index j * GS + h.  Each wave owns 8 columns (MFMA columns
// c and c + 8 carry their f16 high parts and residuals, as in decode) and streams every
// tile up to its last token's position; the 4 waves read the same tiles, so L1/L2 serve
// the repeats.  Columns see their own causal limit; the wave's outputs need no merge.
// ---------------------------------------------------------------------------------
#define QV_PREFILL_PARAMS                                                                       \
    const uint8_t *__restrict__ pool, uint64_t pool_blocks, const float *__restrict__ q,        \
        const uint32_t *__restrict__ blocks, uint64_t n_table,                                  \
        const uint32_t *__restrict__ table_at, const uint32_t *__restrict__ pos0,               \
        const uint32_t *__restrict__ q_at, const uint32_t *__restrict__ n_tok, uint32_t n_seg,  \
        uint32_t H, uint32_t max_pos, uint32_t max_tok, uint64_t q_rows, uint32_t n_cb,         \
        float *__restrict__ out, Geo geo, int *err

template <int D, bool Q8>
__global__ __launch_bounds__(256) void k_prefill_mfma(QV_PREFILL_PARAMS) {
    constexpr int NJ = D / 16;
    const uint32_t G = (uint32_t)geo.G, B = (uint32_t)geo.B;
    const uint32_t GS = H / G;
    uint32_t bid = blockIdx.x;
    if (geo.xcd_map) {  // column blocks of one (segment, KV head) share an XCD's L2
        const uint32_t nb = gridDim.x, qn = nb / 8, rn = nb % 8;
        const uint32_t x = bid % 8, i = bid / 8;
        bid = x < rn ? x * (qn + 1) + i : rn * (qn + 1) + (x - rn) * qn + i;
    }
    const uint32_t cb = bid % n_cb;
    const uint32_t sg = bid / n_cb;
    const uint32_t g = sg % G;
    const uint32_t seg = sg / G;
    if (seg >= n_seg) return;
    const uint32_t nt = n_tok[seg], p0s = pos0[seg], qa = q_at[seg], tab = table_at[seg];
    if (nt == 0) return;
    if (nt > max_tok || (uint64_t)p0s + nt - 1 > max_pos) {
        if (threadIdx.x == 0 && cb == 0 && g == 0) flag(err, ERR_POS);
        return;
    }
    if ((uint64_t)qa + nt > q_rows) {
        if (threadIdx.x == 0 && cb == 0 && g == 0) flag(err, ERR_OUT);
        return;
    }
    const uint32_t n_all = p0s + nt;
    if ((uint64_t)tab + (n_all + B - 1) / B > n_table) {
        if (threadIdx.x == 0 && cb == 0 && g == 0) flag(err, ERR_TABLE);
        return;
    }
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const uint32_t c = lane & 15u, qg = lane >> 4;
    const bool hi_col = c < 8;
    const uint32_t cc0 = cb * 32u + w * 8u;          // the wave's first column
    const uint32_t ncols = nt * GS;
    if (cc0 >= ncols) return;
    const uint32_t last_tok = min(nt - 1, (cc0 + 7u) / GS);
    const uint32_t n_max = p0s + last_tok + 1;        // the wave's furthest causal limit
    const uint32_t cc = cc0 + (c & 7u);
    const bool valid = cc < ncols;
    const uint32_t tj = valid ? cc / GS : 0u, hh = valid ? cc % GS : 0u;
    const uint32_t n_col = valid ? p0s + tj + 1 : n_max;

    h4 qf[NJ];
    {
        const float qs = (1.0f / sqrtf((float)D)) * LOG2E_F;
        const float *qrow = q + ((uint64_t)(qa + tj) * H + (uint64_t)g * GS + hh) * D;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int d0 = 32 * (j >> 1) + 8 * (int)qg + 4 * (j & 1);
            float4 x = valid ? *(const float4 *)(qrow + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
            qf[j] = h4{split_part(mul_rn(x.x, qs), hi_col), split_part(mul_rn(x.y, qs), hi_col),
                       split_part(mul_rn(x.z, qs), hi_col), split_part(mul_rn(x.w, qs), hi_col)};
        }
    }
    SoftmaxState<D> st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) st.acc[j] = f4{0.f, 0.f, 0.f, 0.f};
    const uint32_t ntiles = (n_max + 15) / 16;
    for (uint32_t tt = 0; tt < ntiles; tt++) {
        Tile<D, Q8> cur;
        load_tile<D, Q8, false>(cur, tt, pool, pool_blocks, blocks, tab, g, c, qg, geo, err);
        compute_tile<D, Q8, false>(cur, st, qf, n_col, n_max, qg, hi_col, 0u);
    }
    // column totals; output rows 4qg + i (qg < 2) after adding the residual rows
    float l = st.l;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float o = __shfl_xor(st.acc[j][i], 32);
            st.acc[j][i] = Q8 ? st.acc[j][i] + o : split_sum32(st.acc[j][i], o);
        }
    float lr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) lr[i] = __shfl(l, 4 * (int)(qg & 1u) + i);
    if (qg >= 2) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t ccr = cc0 + 4 * qg + i;
        if (ccr >= ncols) continue;
        const uint32_t tr = ccr / GS, hr = ccr % GS;
        float *orow = out + ((uint64_t)(qa + tr) * H + (uint64_t)g * GS + hr) * D;
        const float inv = 1.0f / lr[i];
        if constexpr (!Q8) {
            float o[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) o[j] = st.acc[j][i] * inv;
#pragma unroll
            for (int j = 0; j < NJ; j += 4)
                *(float4 *)(orow + c * (D / 16) + j) = make_float4(o[j], o[j + 1], o[j + 2], o[j + 3]);
        } else {
#pragma unroll
            for (int j = 0; j < NJ; j += 2)
                *(float2 *)(orow + 32 * (j >> 1) + 2 * c) =
                    make_float2(st.acc[j][i] * inv, st.acc[j + 1][i] * inv);
        }
    }
}

// ---------------------------------------------------------------------------------
// Paged prefill attention, f16 pools, d = 64 or 128: the MFMA-throughput form.
// Workgroup = (segment, KV head, block of 64 query rows); row r = token j * GS + head h.
// The 4 waves stage 32-position K/V tiles once in LDS and each wave computes 16 query
// rows with v_mfma_f32_16x16x32_f16.  Two ways to stage (the math is shared):
//   DMA (d = 128, the default): global_load_lds_dwordx4 streams tiles into three slots
//     two tiles ahead, no staging registers; V stays row-major and the P.V operand comes
//     from ds_read_b64_tr_b16 (a transposed LDS read); XOR swizzles keep every read
//     conflict-free;
//   registers (d = 64): the next tile is loaded into registers during this tile's math
//     and stored double-buffered, V transposed in registers (v_perm).
// The MFMAs:
//   S^T[pos][row] = K . Q^T: A = K rows from LDS (MFMA h, row i <-> position
//     8(i/4) + 4h + i%4, so lane l ends up holding positions 8(l/16)..8(l/16)+7 of row
//     l%16), B = q's f16 high part, then its residual (two accumulating MFMAs);
//   O[row][d] += P . V: A = this lane's 8 probabilities (positions 8(l/16)+t), high part
//     then residual; B = 8 consecutive positions of one d.
// The k index of both MFMAs pairs the same logical element in A and B, so the products
// are exact f16 x f16 in f32 accumulators as in decode.
// ---------------------------------------------------------------------------------

// a compile-time flag passed to a generic lambda
template <bool V>
struct Flag {
    static constexpr bool value = V;
};

template <int D>
struct PrefillLds {
    static constexpr int TP = 32;          // positions per tile
    static constexpr int KR = D + 8;       // K row stride (halves): spreads LDS banks
    static constexpr int VR = TP + 8;      // V^T row stride (halves)
    _Float16 k[2][TP][KR];
    _Float16 v[2][D][VR];
};

// The DMA form's LDS: three tile slots, each K and V for 32 positions, row-major with
// 16-byte pieces XOR-swizzled inside a row (the DMA writes 1 KiB contiguous per
// instruction, so rows cannot be padded): K row lr holds piece p at p ^ kswz(lr); V row r
// at p ^ vswz(r).  The swizzles make the scores' A-operand reads (16 rows, one piece) and
// the transposed V reads (ds_read_b64_tr_b16: 4 rows x 32 bytes per 16 lanes) hit
// distinct banks.
template <int D>
struct DmaSlot {
    _Float16 k[32 * D];
    _Float16 v[32 * D];
};
template <int D>
__device__ __forceinline__ uint32_t kswz(uint32_t lr) {
    return (lr / (16u / (D / 8))) % (D / 8);
}
template <int D>
__device__ __forceinline__ uint32_t vswz(uint32_t r) {
    return D / 8 == 16 ? 2u * ((r & 3u) + 4u * ((r >> 3) & 1u))
                       : 2u * (((r >> 1) & 1u) + 2u * ((r >> 3) & 1u));
}

// DMA: the register budget of 3 waves/SIMD (170 VGPRs; the DMA form holds no staging
// registers): 392 vs 369 TFLOP/s at 2 waves (cfg5).
// PS: P carried as f16 high part + residual (P.V exact in f32, two MFMAs per d block);
// without it P is one RNE f16 (one MFMA per d block) and the row sums add the rounded
// probabilities, so the weights the output is normalised by are exactly those applied.
template <int D, bool DMA, bool PS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DMA ? 3 : 1)))
void k_prefill_f16(QV_PREFILL_PARAMS) {
    constexpr int TP = PrefillLds<D>::TP;
    constexpr int KS = D / 32;                 // QK k-steps
    constexpr int NDB = D / 16;                // PV d blocks
    constexpr int CPR = D / 8;                 // 16-byte chunks per K (or V) row
    constexpr int LPT = 2 * TP * CPR / 256;    // chunks per thread per tile (K and V)
    static_assert(LPT >= 1 && (2 * TP * CPR) % 256 == 0, "tile / thread mismatch");
    __shared__ PrefillLds<D> lds;
    __shared__ __attribute__((aligned(16))) DmaSlot<D> s0, s1, s2;
    if constexpr (!DMA) (void)s0, (void)s1, (void)s2;

    const uint32_t G = (uint32_t)geo.G, B = (uint32_t)geo.B;
    const uint32_t GS = H / G;
    uint32_t bid = blockIdx.x;
    if (geo.xcd_map) {
        const uint32_t nb = gridDim.x, qn = nb / 8, rn = nb % 8;
        const uint32_t x = bid % 8, i = bid / 8;
        bid = x < rn ? x * (qn + 1) + i : rn * (qn + 1) + (x - rn) * qn + i;
    }
    const uint32_t qb = bid % n_cb;
    const uint32_t sg = bid / n_cb;
    const uint32_t g = sg % G;
    const uint32_t seg = sg / G;
    if (seg >= n_seg) return;
    const uint32_t nt = n_tok[seg], p0s = pos0[seg], qa = q_at[seg], tab = table_at[seg];
    if (nt == 0) return;
    const bool lead = threadIdx.x == 0 && qb == 0 && g == 0;
    if (nt > max_tok || (uint64_t)p0s + nt - 1 > max_pos) {
        if (lead) flag(err, ERR_POS);
        return;
    }
    if ((uint64_t)qa + nt > q_rows) {
        if (lead) flag(err, ERR_OUT);
        return;
    }
    const uint32_t n_all = p0s + nt;
    if ((uint64_t)tab + (n_all + B - 1) / B > n_table) {
        if (lead) flag(err, ERR_TABLE);
        return;
    }
    const uint32_t nrows = nt * GS;
    const uint32_t r0 = qb * 64u;
    if (r0 >= nrows) return;  // the whole workgroup: no barrier has run yet
    const uint32_t wg_last = min(nt - 1, (r0 + 63u) / GS);
    const uint32_t n_wg = p0s + wg_last + 1;   // positions the workgroup's rows see
    const uint32_t ntiles = (n_wg + TP - 1) / TP;

    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const uint32_t col = lane & 15u, grp = lane >> 4;
    const uint32_t rw0 = r0 + w * 16u;                      // the wave's first row
    const bool wave_live = rw0 < nrows;
    // (uniform per wave: scalar, so the per-tile tests against them are scalar branches)
    const uint32_t n_wave = [&]() {
        return __builtin_amdgcn_readfirstlane(wave_live ? p0s + min(nt - 1, (rw0 + 15u) / GS) + 1 : 0u);
    }();
    const uint32_t n_wave_min = [&]() {  // the first row's limit
        return __builtin_amdgcn_readfirstlane(wave_live ? p0s + rw0 / GS + 1 : 0u);
    }();
    const uint32_t row = rw0 + col;
    const bool rvalid = row < nrows;
    const uint32_t tj = rvalid ? row / GS : 0u, hh = rvalid ? row % GS : 0u;
    const uint32_t n_row = rvalid ? p0s + tj + 1 : 0u;

    // Q fragments: k-step ks, lane group grp holds d = 32 ks + 8 grp .. +7 (high, residual)
    h8 qh[KS], ql[KS];
    {
        const float qs = (1.0f / sqrtf((float)D)) * LOG2E_F;
        const float *qrow = q + ((uint64_t)(qa + tj) * H + (uint64_t)g * GS + hh) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            float x[8];
            if (rvalid) {
                const float4 a = *(const float4 *)(qrow + 32 * ks + 8 * grp);
                const float4 b = *(const float4 *)(qrow + 32 * ks + 8 * grp + 4);
                x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
                x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float y = mul_rn(x[e], qs);
                const _Float16 hi = (_Float16)y;
                qh[ks][e] = hi;
                ql[ks][e] = (_Float16)(y - (float)hi);
            }
        }
    }

    // ---- tile loader.  The first VW waves move V: lane (q, piece) loads the 4x8 block of
    // positions 4q..4q+3 x d = 8 piece..+7, transposes it in registers and writes 4
    // positions of 8 rows of V^T (8 bytes each).  The other waves move K: 16-byte pieces,
    // position p stored at LDS row 16 ((p >> 2) & 1) + 4 (p >> 3) + (p & 3), the A-operand
    // row order of the scores MFMAs (their reads then walk consecutive rows).
    constexpr int VW = CPR * 8 / 64;               // waves moving V (1 at d 64, 2 at d 128)
    constexpr int KT = 256 - 64 * VW;              // threads moving K
    constexpr int KCH = TP * CPR;                  // K chunks per tile
    constexpr int KPT = (KCH + KT - 1) / KT;       // per K thread
    constexpr int NST = KPT > 4 ? KPT : 4;
    static_assert(VW >= 1 && VW <= 2 && CPR * 8 == 64 * VW, "V blocks fill whole waves");
    u4v stage[NST];
    const bool vwave = w < (uint32_t)VW;
    const uint32_t vq = lane & 7u, vpiece = (lane >> 3) + 8u * w;   // V lanes
    const uint32_t kt = threadIdx.x - 64u * VW;                      // K lanes
    // Block bases of 16-position tile halves (each half lies inside one block since B is a
    // multiple of 16); positions past n_wg read as zero.  The register-staged form takes
    // both halves of every tile; in the DMA form each wave moves the chunks of one half
    // (waves 0-1: positions 0-15 of a tile, waves 2-3: 16-31) and resolves only that one.
    // Tiles are resolved strictly in order, one tile ahead of their use: the (block, row)
    // split of the next half advances by counters (no division by B), and the table
    // entries are scalar loads (constant address space: they count on lgkmcnt, never
    // behind the vmcnt of tiles streaming into LDS) that land while a tile's math runs.
    constexpr int NH = DMA ? 1 : 2;          // halves a wave resolves per tile
    const uint32_t my_half = DMA ? [&]() { return __builtin_amdgcn_readfirstlane(w >> 1); }() : 0u;
    const uint8_t *const kv_g = pool + (uint64_t)g * B * D * 2u;   // this KV head's rows
    const uint64_t bbytes = geo.bb;
    // ids at or past pool_ids are bad (the clamp only matters for id 0xffffffff in a pool of
    // 2^32 blocks or more, which no device holds: a block is at least 2 KiB)
    const uint32_t pool_ids = pool_blocks > 0xffffffffull ? 0xffffffffu : (uint32_t)pool_blocks;
    uint32_t at_bi = 0, at_row = 0;         // block index / row of the next half to resolve
    auto step16 = [&]() {
        at_row += 16u;
        if (at_row == B) {
            at_row = 0u;
            at_bi++;
        }
    };
    if (my_half) step16();
    uint32_t nx_blk[NH], nx_row[NH];
    bool nx_in[NH];
#pragma unroll
    for (int k = 0; k < NH; k++) nx_blk[k] = nx_row[k] = 0u, nx_in[k] = false;
    // the half (halves) of tile t, after tile t - 1; in_range: t is known to be below
    // the last tile
    auto resolve = [&](uint32_t t, bool in_range = false) {
#pragma unroll
        for (int k = 0; k < NH; k++) {
            nx_in[k] = in_range || t * TP + 16u * (NH == 1 ? my_half : (uint32_t)k) < n_wg;
            nx_row[k] = at_row;
            if (nx_in[k])
                nx_blk[k] = ((const __attribute__((address_space(4))) uint32_t *)blocks)[tab + at_bi];
            step16();
            if (NH == 1) step16();          // past the other half
        }
    };
    bool bad_id = false;                    // flagged once, after the tile loop
    auto resolved = [&](int k) -> const uint8_t * {  // a base of the last resolved tile
        const bool bad = nx_in[k] && nx_blk[k] >= pool_ids;
        bad_id |= bad;
        const uint8_t *b = kv_g + (uint64_t)nx_blk[k] * bbytes + nx_row[k] * (uint32_t)(D * 2);
        return nx_in[k] && !bad ? b : nullptr;
    };
    // Row r (0..31) of the tile from the bases of its two 16-position halves; positions
    // past n_wg (r >= valid) and bad blocks read as zero.
    auto fetch = [](const uint8_t *b0, const uint8_t *b1, uint32_t valid, uint32_t r,
                    uint32_t off) -> u4v {
        const uint8_t *b = (r & 16u) ? b1 : b0;
        if (b == nullptr || r >= valid) return u4v{0u, 0u, 0u, 0u};
        return *(const u4v *)(b + off);
    };
    auto load = [&](uint32_t t) {  // t = 0, 1, 2, ... in order
        const uint32_t p0 = t * TP;
        const uint8_t *b0 = resolved(0), *b1 = resolved(1);
        if (t + 1 < ntiles) resolve(t + 1);
        const uint32_t valid = n_wg - p0 < (uint32_t)TP ? n_wg - p0 : (uint32_t)TP;
        const bool full = valid == (uint32_t)TP && b0 != nullptr && b1 != nullptr;  // uniform
        if (vwave) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t row = 4 * vq + r;
                const uint32_t off = (uint32_t)geo.v_off + ((row & 15u) * D + vpiece * 8) * 2u;
                stage[r] = full ? *(const u4v *)(((row & 16u) ? b1 : b0) + off)
                                : fetch(b0, b1, valid, row, off);
            }
        } else {
#pragma unroll
            for (int u = 0; u < KPT; u++) {
                const uint32_t c = kt + (uint32_t)KT * u;
                const uint32_t row = c / CPR;
                const uint32_t off = (uint32_t)geo.k_off + ((row & 15u) * D + (c % CPR) * 8) * 2u;
                if (c < (uint32_t)KCH)
                    stage[u] = full ? *(const u4v *)(((row & 16u) ? b1 : b0) + off)
                                    : fetch(b0, b1, valid, row, off);
            }
        }
    };
    auto store = [&](int buf) {
        if (vwave) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
                u2v o;
                o[0] = __builtin_amdgcn_perm(stage[1][e >> 1], stage[0][e >> 1], sel);
                o[1] = __builtin_amdgcn_perm(stage[3][e >> 1], stage[2][e >> 1], sel);
                *(u2v *)&lds.v[buf][vpiece * 8 + e][4 * vq] = o;
            }
        } else {
#pragma unroll
            for (int u = 0; u < KPT; u++) {
                const uint32_t c = kt + (uint32_t)KT * u;
                if (c < (uint32_t)KCH) {
                    const uint32_t p = c / CPR, piece = c % CPR;
                    const uint32_t lr = 16u * ((p >> 2) & 1u) + 4u * (p >> 3) + (p & 3u);
                    *(u4v *)&lds.k[buf][lr][piece * 8] = stage[u];
                }
            }
        }
    };

    float m = -INFINITY, l = 0.0f;
    f4 acc[NDB];
#pragma unroll
    for (int j = 0; j < NDB; j++) acc[j] = f4{0.f, 0.f, 0.f, 0.f};

    // One tile for this wave's 16 rows.  kread(h, ks): the scores' A operand (K rows 16h +
    // col, d = 32 ks + 8 grp ..); vread(j): the P.V B operand (positions 8 grp + t of
    // d = 16 j + col).
    auto tile = [&](uint32_t tp0, auto kread, auto vread) {
        if (tp0 >= n_wave) return;
        // ---- scores: lane holds positions tp0 + 8 grp + (4h + i) of row `col`
        // the two 16-position halves' accumulation chains interleaved (each keeps its order).
        // The accumulators start at -m0 (m0: the row's max so far, 0 before any), so the
        // scores come out shifted for exp2 without a subtraction per score.
        const float m0 = m == -INFINITY ? 0.0f : m;
        f4 s[2] = {f4{-m0, -m0, -m0, -m0}, f4{-m0, -m0, -m0, -m0}};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const h8 a0 = kread(0, ks), a1 = kread(1, ks);
            s[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qh[ks], s[0], 0, 0, 0);
            s[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qh[ks], s[1], 0, 0, 0);
            s[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, ql[ks], s[0], 0, 0, 0);
            s[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, ql[ks], s[1], 0, 0, 0);
        }
        float sc[8];
#pragma unroll
        for (int e = 0; e < 8; e++) sc[e] = s[e >> 2][e & 3];
        if (tp0 + TP > n_wave_min) {  // the tile reaches some row's causal limit
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (tp0 + 8u * grp + (uint32_t)e >= n_row) sc[e] = -INFINITY;
        }
        float tmax = sc[0];
#pragma unroll
        for (int e = 1; e < 8; e++) tmax = fmaxf(tmax, sc[e]);
        // Lazy rescale: the reference max m moves only when a row's scores exceed it by
        // more than 2^8, so probabilities stay <= 256 (exact under the f16 high +
        // residual split) and the O rescale runs on few tiles.  The test needs no row
        // max: adding m0 and rounding are monotonic, so some lane's own max exceeds
        // m + 8 exactly when its row's max does; the row max is taken on that rare path.
        if (__any(tmax + m0 > m + 8.0f)) {
            const float mnew = fmaxf(m, max_xor16_32(tmax) + m0);
            const float alpha = __builtin_amdgcn_exp2f(m - (mnew == -INFINITY ? 0.0f : mnew));
            l *= alpha;
            float ar[4];
#pragma unroll
            for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * (int)grp + i);
#pragma unroll
            for (int j = 0; j < NDB; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[j][i] *= ar[i];
            m = mnew;
            const float shift = (m == -INFINITY ? 0.0f : m) - m0;
#pragma unroll
            for (int e = 0; e < 8; e++) sc[e] -= shift;
        }
        float pr[8];
#pragma unroll
        for (int e = 0; e < 8; e++) pr[e] = __builtin_amdgcn_exp2f(sc[e]);
        if constexpr (!PS) {
            // one f16 per probability; the row sum takes the rounded values, pairwise in
            // f32 (v_dot2 with ones)
            uint32_t pw[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                pw[k] = __builtin_bit_cast(uint32_t, h2{(_Float16)pr[2 * k], (_Float16)pr[2 * k + 1]});
            const h2 one = h2{(_Float16)1.0f, (_Float16)1.0f};
            float psum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pw[0]), one, 0.0f, false);
#pragma unroll
            for (int k = 1; k < 4; k++)
                psum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pw[k]), one, psum, false);
            l += psum;
            const h8 ph = __builtin_bit_cast(h8, u4v{pw[0], pw[1], pw[2], pw[3]});
#pragma unroll
            for (int j = 0; j < NDB; j += 2) {
                const h8 b0 = vread(j), b1 = vread(j + 1);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, b0, acc[j], 0, 0, 0);
                acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, b1, acc[j + 1], 0, 0, 0);
            }
            return;
        }
        float psum = pr[0];  // (0 + p0 = p0: the same sum without the first add)
#pragma unroll
        for (int e = 1; e < 8; e++) psum += pr[e];
        l += psum;
        uint32_t phw[4], plw[4];  // high parts and exact residuals, one rounding each
#pragma unroll
        for (int k = 0; k < 4; k++) split_pair(pr[2 * k], pr[2 * k + 1], phw[k], plw[k]);
        const h8 ph = __builtin_bit_cast(h8, u4v{phw[0], phw[1], phw[2], phw[3]});
        const h8 pl = __builtin_bit_cast(h8, u4v{plw[0], plw[1], plw[2], plw[3]});
        // two d blocks at a time, so each accumulator's two MFMAs are not back to back
#pragma unroll
        for (int j = 0; j < NDB; j += 2) {
            const h8 b0 = vread(j), b1 = vread(j + 1);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, b0, acc[j], 0, 0, 0);
            acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, b1, acc[j + 1], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, b0, acc[j], 0, 0, 0);
            acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, b1, acc[j + 1], 0, 0, 0);
        }
    };

    resolve(0);
    if constexpr (!DMA) {
        load(0);
        store(0);
        __syncthreads();
        for (uint32_t t = 0; t < ntiles; t++) {
            const int buf = (int)(t & 1u);
            if (t + 1 < ntiles) load(t + 1);
            tile(
                t * TP,
                [&](int h, int ks) {
                    return *(const h8 *)&lds.k[buf][16 * h + col][32 * ks + 8 * grp];
                },
                [&](int j) { return *(const h8 *)&lds.v[buf][16 * j + col][8 * grp]; });
            if (t + 1 < ntiles) store(buf ^ 1);
            __syncthreads();
        }
    } else {
        // Tiles stream into three LDS slots two tiles ahead with global_load_lds_dwordx4
        // (each lane's 16 bytes land at slot + 16 * chunk, chunk = thread + 256 u); a tile
        // with positions past n_wg or a bad block takes the register path and zeros.
        constexpr int CH = TP * CPR;           // chunks per K (or V) tile
        constexpr int CPT = 2 * CH / 256;      // chunks per thread per tile
        static_assert(CH % 64 == 0, "a wave's chunks are all K or all V");
        auto chunk = [&](uint32_t c, uint32_t &pos, uint32_t &piece, bool &isv) {
            isv = c >= (uint32_t)CH;
            const uint32_t cc = isv ? c - CH : c;
            const uint32_t r = cc / CPR, sp = cc % CPR;
            if (!isv) {  // LDS row r = 16h + i holds position 8 (i / 4) + 4h + i % 4
                pos = 8u * ((r & 15u) >> 2) + 4u * (r >> 4) + (r & 3u);
                piece = sp ^ kswz<D>(r);
            } else {
                pos = r;
                piece = sp ^ vswz<D>(r);
            }
        };
        // pool offsets of the K and V parts of a block, as values (a per-lane choice
        // between two kernel-argument fields would otherwise load through a vector address).
        // Chosen below as `koff + (isv ? kv_gap : 0)`: a per-lane choice between the two
        // variables themselves became a choice between their addresses, and the compiler
        // then kept both in scratch memory and read the chosen one back through a pointer
        // on every tile of the register path.
        const uint32_t koff = (uint32_t)geo.k_off, kv_gap = (uint32_t)(geo.v_off - geo.k_off);
        // Chunk u of this thread: wave w moves group 4 (w & 1) + u of its half's 8 groups of
        // 64 chunks (4 LDS rows each): groups 0-3 the K rows holding the half's positions
        // (LDS rows {0-3, 4-7, 16-19, 20-23} + 8 half), 4-7 its V rows (16 half + 4 (g - 4)
        // ..).  Fixed for every tile: the chunk's pool offset inside a block, and for the
        // wave whether it is V and the LDS offset of its first chunk.  The load then takes
        // the half's scalar block base plus a 32-bit lane offset.
        static_assert(CPT == 4 && CPR == 16, "the DMA form is laid out for d = 128");
        auto chunk_u = [&](int u) -> uint32_t {  // chunk index: K 0..CH-1, then V
            const uint32_t gi = 4u * (w & 1u) + (uint32_t)u, hf = w >> 1;
            const uint32_t r0 = gi < 4u ? 4u * (gi & 1u) + 16u * (gi >> 1) + 8u * hf
                                        : 16u * hf + 4u * (gi - 4u);
            return (gi < 4u ? 0u : (uint32_t)CH) + r0 * CPR + lane;
        };
        // (in a lambda: the host pass of a kernel body must not see the device builtins)
        uint32_t c_off[CPT], c_lds[CPT], c_v[CPT];
        [&]() {
#pragma unroll
            for (int u = 0; u < CPT; u++) {
                const uint32_t c = chunk_u(u);
                uint32_t pos, piece;
                bool isv;
                chunk(c, pos, piece, isv);
                c_off[u] = (koff + (isv ? kv_gap : 0u)) + ((pos & 15u) * D + piece * 8) * 2u;
                const uint32_t cc = isv ? c - CH : c;
                c_lds[u] = __builtin_amdgcn_readfirstlane((cc - lane) * 8);
                c_v[u] = __builtin_amdgcn_readfirstlane(isv ? 1u : 0u);
            }
        }();
        // t = 0, 1, 2, ... in order; steady: t + 2 is below the last tile, so tile t is whole
        // and both halves of t + 1 start before n_wg
        auto issue = [&](auto steady, uint32_t t, DmaSlot<D> &sl) {
            constexpr bool STEADY = decltype(steady)::value;
            const uint8_t *hb = resolved(0);
            if (STEADY || t + 1 < ntiles) resolve(t + 1, STEADY);
            const uint32_t p0 = t * TP + 16u * my_half;   // the wave's half
            const uint32_t valid = STEADY ? 16u : n_wg > p0 ? min(n_wg - p0, 16u) : 0u;
            if (valid == 16u && hb != nullptr) {  // uniform
                // Cached loads (aux 0): the n_cb workgroups of a (segment, KV head) read the
                // same tiles and share them through the XCD's L2.
#pragma unroll
                for (int u = 0; u < CPT; u++) {
                    // (operands named first: with them inline, hipcc's host pass dropped the
                    // kernel's launch stub without a diagnostic)
                    const uint8_t *src = hb + c_off[u];
                    _Float16 *lds_dst = (c_v[u] ? sl.v : sl.k) + c_lds[u];
                    __builtin_amdgcn_global_load_lds(src, lds_dst, 16, 0, 0);
                }
            } else {
                // past n_wg or a bad block: through registers, zeros where invalid
#pragma unroll
                for (int u = 0; u < CPT; u++) {
                    const uint32_t c = chunk_u(u);
                    uint32_t pos, piece;
                    bool isv;
                    chunk(c, pos, piece, isv);
                    const uint32_t off = (koff + (isv ? kv_gap : 0u)) + ((pos & 15u) * D + piece * 8) * 2u;
                    // (an offset, not a choice between two pointers: that choice per lane
                    // had put both pointers in scratch memory, read back on every tile)
                    _Float16 *dst = sl.k + (isv ? 32u * D : 0u);
                    const uint32_t cc = isv ? c - CH : c;
                    const u4v x = hb != nullptr && (pos & 15u) < valid ? *(const u4v *)(hb + off)
                                                                       : u4v{0u, 0u, 0u, 0u};
                    *(u4v *)(dst + cc * 8) = x;
                }
            }
        };
        auto kread = [&](DmaSlot<D> &sl) {
            return [&sl, col = col, grp = grp](int h, int ks) {
                const uint32_t r = 16u * h + col, p = 4u * ks + grp;
                return *(const h8 *)(sl.k + (r * CPR + (p ^ kswz<D>(r))) * 8);
            };
        };
        auto vread = [&](DmaSlot<D> &sl) {
            // lane s of a 16-lane group addresses position 8 grp + 4 hf + s / 4, d = 16 j +
            // 4 (s % 4): the transposed read hands lane col those 4 positions at d = 16 j + col
            return [&sl, lane = lane, grp = grp](int j) {
                const uint32_t sidx = lane & 15u;
                u2v w[2];
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const uint32_t r = 8u * grp + 4u * hf + (sidx >> 2);
                    const uint32_t d = 16u * j + 4u * (sidx & 3u);
                    const uint32_t p = d >> 3;
                    const _Float16 *a = sl.v + (r * CPR + (p ^ vswz<D>(r))) * 8 + (d & 7u);
                    // whole registers only (element-wise copies of the 4 x 16-bit result
                    // miscompile); the compiler waits for all DMA in flight before this read
                    // (it cannot prove the slots apart), which measured faster than an asm
                    // form that avoids the wait but spills
                    typedef short s4 __attribute__((ext_vector_type(4)));
                    w[hf] = __builtin_bit_cast(u2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                        (__attribute__((address_space(3))) s4 *)a));
                }
                return __builtin_bit_cast(h8, u4v{w[0][0], w[0][1], w[1][0], w[1][1]});
            };
        };
        // waits: this thread's chunks of tile t have landed when at most `ahead` tiles'
        // chunks (CPT instructions each) are still outstanding
        auto wait_tile = [&](uint32_t t) {
            if (t + 1 < ntiles) {
                if constexpr (CPT == 4) __builtin_amdgcn_s_waitcnt(0x0f74);  // vmcnt(4)
                else __builtin_amdgcn_s_waitcnt(0x0f72);                    // vmcnt(2)
            } else {
                __builtin_amdgcn_s_waitcnt(0x0f70);                         // vmcnt(0)
            }
        };
        // steady: t + 4 is below the last tile (no range checks)
        auto step = [&](auto steady, uint32_t t, DmaSlot<D> &cur, DmaSlot<D> &nxt) {
            constexpr bool STEADY = decltype(steady)::value;
            // Tile t landed everywhere and every wave is past tile t - 1.  A bare barrier:
            // __syncthreads' fence would also wait for the tiles still in flight.
            if constexpr (STEADY) __builtin_amdgcn_s_waitcnt(0x0f74);  // vmcnt(4)
            else wait_tile(t);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): register-path LDS stores
            asm volatile("" ::: "memory");       // no LDS access moves across the barrier
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (STEADY || t + 2 < ntiles) issue(steady, t + 2, nxt);  // into tile t - 1's slot
            tile(t * TP, kread(cur), vread(cur));
        };
        const Flag<false> any;
        const Flag<true> steady;
        issue(any, 0, s0);
        if (ntiles > 1) issue(any, 1, s1);
        uint32_t t = 0;
        // steady steps t .. t + 2 issue tiles up to t + 4 and resolve up to t + 5, which must
        // not be the last tile (its second half may start past n_wg)
        for (; t + 7 <= ntiles; t += 3) {
            step(steady, t, s0, s2);
            step(steady, t + 1, s1, s0);
            step(steady, t + 2, s2, s1);
        }
        for (; t < ntiles; t += 3) {
            step(any, t, s0, s2);
            if (t + 1 < ntiles) step(any, t + 1, s1, s0);
            if (t + 2 < ntiles) step(any, t + 2, s2, s1);
        }
    }
    if (bad_id && lane == 0) flag(err, ERR_BLOCK);  // any wave: each resolves its own half
    if (!wave_live) return;
    // ---- row totals; lane (col, grp) holds O rows 4 grp + i at d = 16 j + col
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    float lr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) lr[i] = __shfl(l, 4 * (int)grp + i);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t rr = rw0 + 4 * grp + i;
        if (rr >= nrows) continue;
        const uint32_t tr = rr / GS, hr = rr % GS;
        float *orow = out + ((uint64_t)(qa + tr) * H + (uint64_t)g * GS + hr) * D;
        const float inv = 1.0f / lr[i];
#pragma unroll
        for (int j = 0; j < NDB; j++) orow[16 * j + col] = acc[j][i] * inv;
    }
}

// ---------------------------------------------------------------------------------
// Paged prefill attention, q8_0 pools, d = 128: the MFMA-throughput form of
// k_prefill_f16 (64 query rows per workgroup, 16 per wave, 32-position tiles in LDS, the
// same swizzled slot layout and operand reads), with the tiles staged through registers:
//   K: int8 values as f16 (exact); each score MFMA pair covers one 32-value group, and the
//      group's per-position scale multiplies its partial scores (v_fma_mix reads the f16
//      scale directly);
//   V: dequantised while staging, v = q * scale split into an f16 high part and its
//      residual (packed f16 multiply, then a packed FMA that forms the residual exactly),
//      so P.V takes three MFMAs per d block: P_hi V_hi + P_lo V_hi + P_hi V_lo.
// Dequantised V values must fit f16: a V scale above 512 (127 * 512 < 65504) latches
// ERR_RANGE and the call reports QVKV_E_UNSUPPORTED.
// Tile t + 1 is loaded into registers during tile t's math, then converted into the other
// LDS buffer; one barrier per tile.
// ---------------------------------------------------------------------------------
template <int D>
struct Q8PrefillSlot {
    _Float16 k[32 * D];           // int8 keys as f16, DMA-slot layout (A-operand row order)
    _Float16 vh[32 * D], vl[32 * D];  // dequantised values: high part, residual
    uint32_t ks[32 * (D / 64)];   // key scales, [position][group] f16
};

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void k_prefill_q8(QV_PREFILL_PARAMS) {
    static_assert(D == 128, "q8_0 MFMA-throughput prefill is built for d = 128");
    constexpr int TP = 32;
    constexpr int KS = D / 32;                 // QK k-steps = quantization groups
    constexpr int NDB = D / 16;                // PV d blocks
    constexpr int CPR = D / 8;                 // 8-value (16-byte f16) pieces per row
    __shared__ __attribute__((aligned(16))) Q8PrefillSlot<D> sb0, sb1;

    const uint32_t G = (uint32_t)geo.G, B = (uint32_t)geo.B;
    const uint32_t GS = H / G;
    uint32_t bid = blockIdx.x;
    if (geo.xcd_map) {
        const uint32_t nb = gridDim.x, qn = nb / 8, rn = nb % 8;
        const uint32_t x = bid % 8, i = bid / 8;
        bid = x < rn ? x * (qn + 1) + i : rn * (qn + 1) + (x - rn) * qn + i;
    }
    const uint32_t qb = bid % n_cb;
    const uint32_t sg = bid / n_cb;
    const uint32_t g = sg % G;
    const uint32_t seg = sg / G;
    if (seg >= n_seg) return;
    const uint32_t nt = n_tok[seg], p0s = pos0[seg], qa = q_at[seg], tab = table_at[seg];
    if (nt == 0) return;
    const bool lead = threadIdx.x == 0 && qb == 0 && g == 0;
    if (nt > max_tok || (uint64_t)p0s + nt - 1 > max_pos) {
        if (lead) flag(err, ERR_POS);
        return;
    }
    if ((uint64_t)qa + nt > q_rows) {
        if (lead) flag(err, ERR_OUT);
        return;
    }
    const uint32_t n_all = p0s + nt;
    if ((uint64_t)tab + (n_all + B - 1) / B > n_table) {
        if (lead) flag(err, ERR_TABLE);
        return;
    }
    const uint32_t nrows = nt * GS;
    const uint32_t r0 = qb * 64u;
    if (r0 >= nrows) return;  // the whole workgroup: no barrier has run yet
    const uint32_t wg_last = min(nt - 1, (r0 + 63u) / GS);
    const uint32_t n_wg = p0s + wg_last + 1;
    const uint32_t ntiles = (n_wg + TP - 1) / TP;

    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const uint32_t col = lane & 15u, grp = lane >> 4;
    const uint32_t rw0 = r0 + w * 16u;
    const bool wave_live = rw0 < nrows;
    const uint32_t n_wave = [&]() {  // scalar: the per-tile tests are scalar branches
        return __builtin_amdgcn_readfirstlane(wave_live ? p0s + min(nt - 1, (rw0 + 15u) / GS) + 1 : 0u);
    }();
    const uint32_t n_wave_min = [&]() {
        return __builtin_amdgcn_readfirstlane(wave_live ? p0s + rw0 / GS + 1 : 0u);
    }();
    const uint32_t row = rw0 + col;
    const bool rvalid = row < nrows;
    const uint32_t tj = rvalid ? row / GS : 0u, hh = rvalid ? row % GS : 0u;
    const uint32_t n_row = rvalid ? p0s + tj + 1 : 0u;

    h8 qh[KS], ql[KS];
    {
        const float qs = (1.0f / sqrtf((float)D)) * LOG2E_F;
        const float *qrow = q + ((uint64_t)(qa + tj) * H + (uint64_t)g * GS + hh) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            float x[8];
            if (rvalid) {
                const float4 a = *(const float4 *)(qrow + 32 * ks + 8 * grp);
                const float4 b = *(const float4 *)(qrow + 32 * ks + 8 * grp + 4);
                x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
                x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float y = mul_rn(x[e], qs);
                const _Float16 hi = (_Float16)y;
                qh[ks][e] = hi;
                ql[ks][e] = (_Float16)(y - (float)hi);
            }
        }
    }

    // ---- staging: thread = (position sp, lane sj = tid % 8 of the position) of the tile,
    // plus the row's 4 V scales; threads 0..63 also move one word of K scales (position
    // tid / 2).  The LDS stores are laid out to take the fewest bank passes:
    //   K: store k (0, 1) of lane sj fills LDS slot sj + 8 ((k + si) & 1) of its row, so
    //      each 8 lanes write one aligned 128-byte half of a row and the two rows of a
    //      16-lane group write opposite halves; the lane loads the two stored 8-byte chunks
    //      (4 (P % 4) + P / 4 holds logical piece P) that its slots need;
    //   V: lane sj loads stored bytes 16 sj .. +15 and writes 8-byte quarter pieces; the
    //      position order (sp bit 1 = si bit 0, sp bit 3 = si bit 1) puts the rows of each
    //      2- and 4-row group of an LDS store in distinct 64-byte quarters of the banks.
    const uint32_t si = threadIdx.x >> 3;
    const uint32_t sp = ((si & 1u) << 1) | ((si & 2u) << 2) | ((si >> 2) & 1u) |
                        (((si >> 3) & 1u) << 2) | (si & 16u),
                   sj = threadIdx.x & 7u;
    const uint32_t klr = 16u * ((sp >> 2) & 1u) + 4u * (sp >> 3) + (sp & 3u);  // K row in LDS
    uint32_t kslot[2], kchunk[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        kslot[k] = sj + 8u * ((k + si) & 1u);
        const uint32_t P = kslot[k] ^ kswz<D>(klr);  // logical piece of the slot
        kchunk[k] = 4u * (P & 3u) + (P >> 2);       // stored 8-byte chunk holding it
    }
    u2v xk[2];
    u4v xv;
    u2v xvs;
    uint32_t xks;
    // The block of each 16-position half of a tile, resolved on the scalar unit: the block
    // base and the first row of the half (g * B + its offset in the block), or null past
    // n_wg / for a bad id.  Tiles are resolved in order, one tile ahead of their use: the
    // (block, row) split advances by counters (B is a multiple of 16) and the table
    // entries are constant-address-space loads that land during a tile's math.
    struct Half {
        const uint8_t *base;
        uint32_t row0;
    };
    // ids at or past pool_ids are bad (the clamp only matters for id 0xffffffff in a pool of
    // 2^32 blocks or more, which no device holds)
    const uint32_t pool_ids = pool_blocks > 0xffffffffull ? 0xffffffffu : (uint32_t)pool_blocks;
    uint32_t at_bi = 0, at_row = 0;         // block index / row of the next half to resolve
    uint32_t nx_blk[2] = {0u, 0u}, nx_row[2] = {0u, 0u};
    bool nx_in[2] = {false, false};
    auto resolve = [&](uint32_t t) {        // the halves of tile t, after those of t - 1
#pragma unroll
        for (int k = 0; k < 2; k++) {
            nx_in[k] = t * TP + 16u * k < n_wg;
            nx_row[k] = at_row;
            if (nx_in[k])
                nx_blk[k] = ((const __attribute__((address_space(4))) uint32_t *)blocks)[tab + at_bi];
            at_row += 16u;
            if (at_row == B) {
                at_row = 0u;
                at_bi++;
            }
        }
    };
    bool bad_id = false;                    // flagged once, after the tile loop
    auto resolved = [&](int k) -> Half {    // a half of the last resolved tile
        const bool bad = nx_in[k] && nx_blk[k] >= pool_ids;
        bad_id |= bad;
        return Half{nx_in[k] && !bad ? pool + (uint64_t)nx_blk[k] * geo.bb : nullptr,
                    g * B + nx_row[k]};
    };
    auto load = [&](uint32_t t) {  // t = 0, 1, 2, ... in order
        const uint32_t p0 = t * TP;
        const Half h0 = resolved(0), h1 = resolved(1);
        if (t + 1 < ntiles) resolve(t + 1);
        xk[0] = u2v{0u, 0u};
        xk[1] = u2v{0u, 0u};
        xv = u4v{0u, 0u, 0u, 0u};
        xvs = u2v{0u, 0u};
        xks = 0u;
        const Half &hp = (sp & 16u) ? h1 : h0;
        if (hp.base != nullptr && p0 + sp < n_wg) {
            const uint32_t rw = hp.row0 + (sp & 15u);
            xk[0] = *(const u2v *)(hp.base + geo.k_off + rw * D + 8u * kchunk[0]);
            xk[1] = *(const u2v *)(hp.base + geo.k_off + rw * D + 8u * kchunk[1]);
            xv = *(const u4v *)(hp.base + geo.v_off + rw * D + 16u * sj);
            xvs = *(const u2v *)(hp.base + geo.vs_off + rw * (D / 16));
        }
        // K scales: threads 0..63, position tid / 2, word tid % 2
        const uint32_t pk = threadIdx.x >> 1;
        const Half &hk = (pk & 16u) ? h1 : h0;
        if (threadIdx.x < 64u && hk.base != nullptr && p0 + pk < n_wg)
            xks = *(const uint32_t *)(hk.base + geo.ks_off + (hk.row0 + (pk & 15u)) * (D / 16) +
                                      4u * (threadIdx.x & 1u));
    };
    auto store = [&](Q8PrefillSlot<D> &sl) {
        // K: each loaded 8-byte chunk is one logical 8-value piece, stored at its slot
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const h4 a = i8x4_to_h4_vals(xk[k].x), b = i8x4_to_h4_vals(xk[k].y);
            *(h8 *)(sl.k + (klr * CPR + kslot[k]) * 8) =
                h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        }
        // V: stored byte c * 8 + 2 gr + u holds d = 32 gr + 2 c + u; this piece holds
        // c = 2 sj, 2 sj + 1: for each group gr, d = 32 gr + 4 sj .. +3 from bytes
        // 2 gr, 2 gr + 1, 8 + 2 gr, 9 + 2 gr
        bool big = false;
#pragma unroll
        for (int gr = 0; gr < 4; gr++) {
            const uint32_t w0 = xv[gr >> 1], w1 = xv[2 + (gr >> 1)];
            h2 x01, x23;
            if (gr & 1) {
                x01 = __builtin_bit_cast(h2, i8x2_to_h2<2>(w0));
                x23 = __builtin_bit_cast(h2, i8x2_to_h2<2>(w1));
            } else {
                x01 = __builtin_bit_cast(h2, i8x2_to_h2<0>(w0));
                x23 = __builtin_bit_cast(h2, i8x2_to_h2<0>(w1));
            }
            const uint32_t sbits = (xvs[gr >> 1] >> (16u * (gr & 1u))) & 0xffffu;
            const _Float16 sc = __builtin_bit_cast(_Float16, (uint16_t)sbits);
            // |scale| above 512 (f16 0x6000), infinities included, NaN (above 0x7c00) not
            big |= (sbits & 0x7fffu) - 0x6001u < 0x7c00u - 0x6000u;
            const h2 s2 = {sc, sc};
            h2 a = x01 * s2, b = x23 * s2;       // high parts (rounded products)
            asm volatile("" : "+v"(a), "+v"(b));  // not contracted into the residuals
            const h2 ra = __builtin_elementwise_fma(x01, s2, -a);
            const h2 rb = __builtin_elementwise_fma(x23, s2, -b);
            const uint32_t P = 4u * gr + (sj >> 1), hf = sj & 1u;
            const uint32_t off = (sp * CPR + (P ^ vswz<D>(sp))) * 8 + 4 * hf;
            *(h4 *)(sl.vh + off) = h4{a[0], a[1], b[0], b[1]};
            *(h4 *)(sl.vl + off) = h4{ra[0], ra[1], rb[0], rb[1]};
        }
        if (big) flag(err, ERR_RANGE);
        if (threadIdx.x < 64u) sl.ks[threadIdx.x] = xks;
    };

    float m = -INFINITY, l = 0.0f;
    f4 acc[NDB];
#pragma unroll
    for (int j = 0; j < NDB; j++) acc[j] = f4{0.f, 0.f, 0.f, 0.f};

    auto kread = [&](const Q8PrefillSlot<D> &sl, int h, int ks) {
        const uint32_t r = 16u * h + col, p = 4u * ks + grp;
        return *(const h8 *)(sl.k + (r * CPR + (p ^ kswz<D>(r))) * 8);
    };
    // transposed V read (ds_read_b64_tr_b16): lane col gets positions 8 grp .. +7 of
    // d = 16 j + col
    auto vread = [&](const _Float16 *v, int j) {
        const uint32_t sidx = lane & 15u;
        u2v wv[2];
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const uint32_t r = 8u * grp + 4u * hf + (sidx >> 2);
            const uint32_t d = 16u * j + 4u * (sidx & 3u);
            const uint32_t pc = d >> 3;
            const _Float16 *a = v + (r * CPR + (pc ^ vswz<D>(r))) * 8 + (d & 7u);
            typedef short s4 __attribute__((ext_vector_type(4)));
            wv[hf] = __builtin_bit_cast(u2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                 (__attribute__((address_space(3))) s4 *)a));
        }
        return __builtin_bit_cast(h8, u4v{wv[0][0], wv[0][1], wv[1][0], wv[1][1]});
    };

    auto tile = [&](const Q8PrefillSlot<D> &sl, uint32_t tp0) {
        if (tp0 >= n_wave) return;
        // ---- scores: lane holds positions tp0 + 8 grp + (4h + i) of row `col`
        // key scales of this lane's 8 positions: words 2 (8 grp + e) + ks / 2
        u4v ksw[4];
#pragma unroll
        for (int x = 0; x < 4; x++) ksw[x] = *(const u4v *)(sl.ks + 16u * grp + 4u * x);
        // scores accumulate from -m0 (m0: the row's max so far, 0 before any), so they come
        // out shifted for exp2 without a subtraction per score
        const float m0 = m == -INFINITY ? 0.0f : m;
        f4 s[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            s[h] = f4{-m0, -m0, -m0, -m0};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const h8 a = kread(sl, h, ks);
                f4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[ks], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[ks], t, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int e = 4 * h + i;  // position 8 grp + e
                    const uint32_t wd = ksw[e >> 1][2 * (e & 1) + (ks >> 1)];
                    const float sc = (float)__builtin_bit_cast(
                        _Float16, (uint16_t)(wd >> (16 * (ks & 1))));
                    s[h][i] = fmaf(t[i], sc, s[h][i]);
                }
            }
        }
        float sc[8];
#pragma unroll
        for (int e = 0; e < 8; e++) sc[e] = s[e >> 2][e & 3];
        if (tp0 + TP > n_wave_min) {
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (tp0 + 8u * grp + (uint32_t)e >= n_row) sc[e] = -INFINITY;
        }
        float tmax = sc[0];
#pragma unroll
        for (int e = 1; e < 8; e++) tmax = fmaxf(tmax, sc[e]);
        // (the row max only on the rare rescale path, as in k_prefill_f16)
        if (__any(tmax + m0 > m + 8.0f)) {
            const float mnew = fmaxf(m, max_xor16_32(tmax) + m0);
            const float alpha = __builtin_amdgcn_exp2f(m - (mnew == -INFINITY ? 0.0f : mnew));
            l *= alpha;
            float ar[4];
#pragma unroll
            for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * (int)grp + i);
#pragma unroll
            for (int j = 0; j < NDB; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[j][i] *= ar[i];
            m = mnew;
            const float shift = (m == -INFINITY ? 0.0f : m) - m0;
#pragma unroll
            for (int e = 0; e < 8; e++) sc[e] -= shift;
        }
        float pr[8];
#pragma unroll
        for (int e = 0; e < 8; e++) pr[e] = __builtin_amdgcn_exp2f(sc[e]);
        float psum = pr[0];
#pragma unroll
        for (int e = 1; e < 8; e++) psum += pr[e];
        l += psum;
        uint32_t phw[4], plw[4];  // high parts and exact residuals, one rounding each
#pragma unroll
        for (int k = 0; k < 4; k++) split_pair(pr[2 * k], pr[2 * k + 1], phw[k], plw[k]);
        const h8 ph = __builtin_bit_cast(h8, u4v{phw[0], phw[1], phw[2], phw[3]});
        const h8 pl = __builtin_bit_cast(h8, u4v{plw[0], plw[1], plw[2], plw[3]});
#pragma unroll
        for (int j = 0; j < NDB; j++) {
            const h8 bh = vread(sl.vh, j), bl = vread(sl.vl, j);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, bh, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, bh, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, bl, acc[j], 0, 0, 0);
        }
    };

    // Tile t is computed from one buffer while tile t + 1 is loaded into registers and then
    // stored into the other; the loop is unrolled by two so both buffers have fixed LDS
    // addresses.
    auto step = [&](uint32_t t, const Q8PrefillSlot<D> &cur, Q8PrefillSlot<D> &nxt) {
        if (t + 1 < ntiles) load(t + 1);
        tile(cur, t * TP);
        if (t + 1 < ntiles) store(nxt);
        __syncthreads();
    };
    resolve(0);
    load(0);
    store(sb0);
    __syncthreads();
    for (uint32_t t = 0; t < ntiles; t += 2) {
        step(t, sb0, sb1);
        if (t + 1 < ntiles) step(t + 1, sb1, sb0);
    }
    if (bad_id && threadIdx.x == 0) flag(err, ERR_BLOCK);
    if (!wave_live) return;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    float lr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) lr[i] = __shfl(l, 4 * (int)grp + i);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t rr = rw0 + 4 * grp + i;
        if (rr >= nrows) continue;
        const uint32_t tr = rr / GS, hr = rr % GS;
        float *orow = out + ((uint64_t)(qa + tr) * H + (uint64_t)g * GS + hr) * D;
        const float inv = 1.0f / lr[i];
#pragma unroll
        for (int j = 0; j < NDB; j++) orow[16 * j + col] = acc[j][i] * inv;
    }
}

// Prefill, generic form: one wave per (segment, token, query head).
template <bool Q8>
__global__ __launch_bounds__(64) void k_prefill_generic(QV_PREFILL_PARAMS) {
    const uint32_t h = blockIdx.x % H;
    const uint32_t j = (blockIdx.x / H) % max_tok;
    const uint32_t seg = blockIdx.x / H / max_tok;
    if (seg >= n_seg) return;
    const uint32_t B = (uint32_t)geo.B, G = (uint32_t)geo.G, D = (uint32_t)geo.D;
    const uint32_t nt = n_tok[seg], p0s = pos0[seg], qa = q_at[seg], tab = table_at[seg];
    if (j >= nt) return;
    const bool first = threadIdx.x == 0 && j == 0 && h == 0;
    if (nt > max_tok || (uint64_t)p0s + nt - 1 > max_pos) {
        if (first) flag(err, ERR_POS);
        return;
    }
    if ((uint64_t)qa + nt > q_rows) {
        if (first) flag(err, ERR_OUT);
        return;
    }
    if ((uint64_t)tab + (p0s + nt + B - 1) / B > n_table) {
        if (first) flag(err, ERR_TABLE);
        return;
    }
    const uint64_t row = (uint64_t)(qa + j) * H + h;
    generic_body<Q8>(pool, pool_blocks, blocks, tab, p0s + j + 1, h / (H / G), q + row * D,
                     out + row * D, geo, err);
}

// =================================================================================
// Host side.
// =================================================================================

int check_prefill(const Geometry &g, uint32_t n_seg, uint32_t heads, uint32_t max_tok,
                  const char **why) {
    if (heads == 0 || heads % (uint32_t)g.G != 0) {
        *why = "query heads must be a positive multiple of kv_heads";
        return QVKV_E_SHAPE;
    }
    const bool mfma = g.D == 64 || g.D == 128 || g.D == 256;
    const uint64_t cols = (uint64_t)max_tok * (heads / (uint32_t)g.G);
    const uint64_t grid = mfma ? (uint64_t)n_seg * g.G * ((cols + 31) / 32)
                               : (uint64_t)n_seg * max_tok * heads;
    if (grid > 0x7fffffffull) {
        *why = "batch too large";
        return QVKV_E_SHAPE;
    }
    return QVKV_OK;
}

hipError_t launch_prefill(const Geometry &g, const void *pool, uint64_t pool_blocks,
                          const float *q, const uint32_t *blocks, uint64_t n_table,
                          const uint32_t *table_at, const uint32_t *pos0, const uint32_t *q_at,
                          const uint32_t *n_tok, uint32_t n_seg, uint32_t heads,
                          uint32_t max_pos, uint32_t max_tok, uint64_t q_rows, float *out,
                          int *err, hipStream_t s, bool f16_values) {
    if (n_seg == 0 || max_tok == 0) return hipSuccess;
    const Geo geo = to_geo(g);
    const uint8_t *pp = (const uint8_t *)pool;
    const bool q8 = g.dtype == QVKV_Q8_0;
    if (!(g.D == 64 || g.D == 128 || g.D == 256)) {
        const unsigned grid = (unsigned)((uint64_t)n_seg * max_tok * heads);
#define QV_PG(QQ)                                                                              \
    hipLaunchKernelGGL(k_prefill_generic<QQ>, dim3(grid), dim3(64), 0, s, pp, pool_blocks, q,   \
                       blocks, n_table, table_at, pos0, q_at, n_tok, n_seg, heads, max_pos,    \
                       max_tok, q_rows, 0u, out, geo, err)
        if (q8) QV_PG(true); else QV_PG(false);
#undef QV_PG
        return hipGetLastError();
    }
    const uint32_t GS = heads / (uint32_t)g.G;
    if (!q8 && (g.D == 64 || g.D == 128) && tune(KNOB_PREFILL_V2)) {
        const uint32_t n_qb = (uint32_t)(((uint64_t)max_tok * GS + 63) / 64);
        const unsigned grid2 = (unsigned)((uint64_t)n_seg * g.G * n_qb);
        const unsigned pad = (unsigned)tune(KNOB_PREFILL_LDS_PAD);
#define QV_PF2(DD, DMA, PS)                                                                    \
    hipLaunchKernelGGL((k_prefill_f16<DD, DMA, PS>), dim3(grid2), dim3(256), pad, s, pp,         \
                       pool_blocks, q, blocks, n_table, table_at, pos0, q_at, n_tok, n_seg,     \
                       heads, max_pos, max_tok, q_rows, n_qb, out, geo, err)
        // P as one f16 (the default) or as high part + residual (knob prefill_exact_p=1)
        const bool ps = tune(KNOB_PREFILL_EXACT_P) != 0;
        if (g.D == 64) { if (ps) QV_PF2(64, false, true); else QV_PF2(64, false, false); }
        else if (tune(KNOB_PREFILL_DMA)) {
            if (ps) QV_PF2(128, true, true); else QV_PF2(128, true, false);
        } else {
            if (ps) QV_PF2(128, false, true); else QV_PF2(128, false, false);
        }
#undef QV_PF2
        return hipGetLastError();
    }
    // f16_values: the q8_0 MFMA-throughput form, which holds dequantised values in f16
    if (q8 && g.D == 128 && f16_values && tune(KNOB_PREFILL_Q8_FAST)) {
        const uint32_t n_qb = (uint32_t)(((uint64_t)max_tok * GS + 63) / 64);
        const unsigned grid3 = (unsigned)((uint64_t)n_seg * g.G * n_qb);
        hipLaunchKernelGGL((k_prefill_q8<128>), dim3(grid3), dim3(256), 0, s, pp, pool_blocks, q,
                           blocks, n_table, table_at, pos0, q_at, n_tok, n_seg, heads, max_pos,
                           max_tok, q_rows, n_qb, out, geo, err);
        return hipGetLastError();
    }
    const uint32_t n_cb = (uint32_t)(((uint64_t)max_tok * GS + 31) / 32);
    const unsigned grid = (unsigned)((uint64_t)n_seg * g.G * n_cb);
#define QV_PF(DD, QQ)                                                                          \
    hipLaunchKernelGGL((k_prefill_mfma<DD, QQ>), dim3(grid), dim3(256), 0, s, pp, pool_blocks,  \
                       q, blocks, n_table, table_at, pos0, q_at, n_tok, n_seg, heads, max_pos, \
                       max_tok, q_rows, n_cb, out, geo, err)
    if (g.D == 64) { if (q8) QV_PF(64, true); else QV_PF(64, false); }
    else if (g.D == 128) { if (q8) QV_PF(128, true); else QV_PF(128, false); }
    else { if (q8) QV_PF(256, true); else QV_PF(256, false); }
#undef QV_PF
    return hipGetLastError();
}

}  // namespace qvkv
