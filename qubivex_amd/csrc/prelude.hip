// The attention prelude that feeds the append: bias, clip, Q/K RMSNorm (full width or per
// head), RoPE.  Bit-exact with the reference's host forward pass
// (crates/qubivex-arch/src/lib.rs:1258-1292), whose arithmetic is plain f32 with explicit
// fused multiply-adds only in the norm's sum of squares:
//   bias:   y += b                                             (lib.rs:1259-1265)
//   clip:   z.clamp(-c, c)                                     (lib.rs:1266-1272)
//   norm:   x = (x * r) * w,  r = 1 / sqrt(ss / n + eps)       (math.rs:89-116)
//           ss = the 64-lane fma shape of reduce::dot (reduce.rs:1-50): lane l sums
//           x[i]^2 for i = l, l+64, ... in order; then a[i] += a[i+w] for w = 32..4;
//           then (a0 + a1) + (a2 + a3)
//   rope:   y1 = x1*c - x2*s,  y2 = x2*c + x1*s  (pairs i, i + d/2; math.rs:160-169)
// One wave per (token, part), its 64 lanes being the reduction's 64 lanes.  Floating-
// point contraction is off in this file: every product and sum rounds on its own.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"

#pragma clang fp contract(off)

namespace qvkv {

// reduce::reduce of the 64 per-lane partial sums (every lane returns the total).
__device__ __forceinline__ float lane_tree(float a) {
#pragma unroll
    for (int w = 32; w >= 4; w >>= 1) a = a + __shfl_down(a, w);
    const float a1 = __shfl(a, 1), a2 = __shfl(a, 2), a3 = __shfl(a, 3);
    const float t = (__shfl(a, 0) + a1) + (a2 + a3);
    return t;
}

// lane_tree's total by cross-lane moves (every lane active; every lane gets the total).
// After each step every lane holds the sum its reduction slot would hold in lane_tree,
// because IEEE addition is commutative:
//   w = 32: v_permlane32_swap of a with itself hands lane i and lane i ^ 32 the pair
//           (a[i mod 32], a[i mod 32 + 32]), so both halves hold a[i] + a[i+32];
//   w = 16: v_permlane16_swap likewise: rows 0 and 1 (and 2 and 3) hold a[i] + a[i+16];
//   w = 8:  DPP row rotation by 8: lanes i and i + 8 of a row both get a[i] + a[i+8];
//   w = 4:  DPP row rotation by 4: lane i gets a[i] + a[i +- 4 mod 16], and lanes i + 4
//           and i + 12 hold the same value after the w = 8 step, so either direction of
//           the rotation gives a[i] + a[i+4];
//   final:  quad_perm [1,0,3,2] then [2,3,0,1]: (t0 + t1) + (t2 + t3) in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float a) {
    return a + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a),
                                                                  CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float lane_tree_x(float a) {
    uint32_t u = __builtin_bit_cast(uint32_t, a);
    const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t h0 = h[0], h1 = h[1];
    a = __builtin_bit_cast(float, h0) + __builtin_bit_cast(float, h1);
    u = __builtin_bit_cast(uint32_t, a);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    a = __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
    a = dpp_add<0x128>(a);  // row_ror:8
    a = dpp_add<0x124>(a);  // row_ror:4
    a = dpp_add<0xB1>(a);   // quad_perm [1,0,3,2]
    return dpp_add<0x4E>(a);  // quad_perm [2,3,0,1]
}

// lane_tree_x for HB heads at once (HB = 4, 8 or 16; a[h] = lane l's partial sum of head
// h).  The trees are interleaved so that one cross-lane move serves two heads: at each
// width w = 32, 16, 8, 4 two registers X, Y (each holding heads in blocks of lanes that
// the step keeps apart) become one, the lanes whose block comes from X computing X's
// a[i] + a[i +- w] and the others Y's.  Every head gets exactly lane_tree's sums (each is
// one IEEE addition of the same two values), in 2 (HB - 1) + a few instructions instead
// of 6 HB dependent moves.  Head h's total ends in the lanes of the quad starting at
// head_lane<HB>(h).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float a) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), CTRL,
                                                             0xF, 0xF, true));
}
__device__ __forceinline__ float xor4(float a) {
    // ds_swizzle bit-mask mode: lane ^ 4 within each group of 32 lanes
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a),
                                                                 0x101F));
}

// Which lanes hold which head after each step (the map the device code follows).
template <int HB>
struct TreeMap {
    int head[64];
    constexpr TreeMap() : head() {
        int map[16][64] = {};
        int valid[64] = {};
        for (int r = 0; r < HB; r++)
            for (int i = 0; i < 64; i++) map[r][i] = r;
        for (int i = 0; i < 64; i++) valid[i] = 1;
        int n = HB;
        bool paired8 = false;
        for (int w = 32; w >= 4; w /= 2) {
            if (n >= 2) {
                for (int r = 0; r < n / 2; r++)
                    for (int i = 0; i < 64; i++) {
                        const bool from_x = w == 32 ? i < 32
                                          : w == 16 ? ((i >> 4) & 1) == 0
                                          : w == 8 ? (i & 8) == 0
                                                   : (i & 4) == 0;
                        map[r][i] = from_x ? map[2 * r][i] : map[2 * r + 1][i];
                    }
                n /= 2;
                if (w == 8) paired8 = true;
            } else if (w == 4 && paired8) {
                for (int i = 0; i < 64; i++)
                    if (i & 4) valid[i] = 0;  // their rotation partner lies in another head
            }
        }
        for (int i = 0; i < 64; i++) head[i] = valid[i] && i % 4 == 0 ? map[0][i] : -1;
    }
};
template <int HB>
__device__ constexpr int head_lane(int h) {
    constexpr TreeMap<HB> m;
    for (int i = 0; i < 64; i++)
        if (m.head[i] == h) return i;
    return -1;
}

template <int HB>
__device__ __forceinline__ float head_trees(const float (&a)[HB], uint32_t lane) {
    static_assert(HB == 4 || HB == 8 || HB == 16, "heads per wave");
    float r[HB];
#pragma unroll
    for (int h = 0; h < HB; h++) r[h] = a[h];
    // w = 32: X' = [X_lo, Y_lo], Y' = [X_hi, Y_hi]
#pragma unroll
    for (int m = 0; m < HB / 2; m++) {
        const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, r[2 * m]),
                                                         __builtin_bit_cast(uint32_t, r[2 * m + 1]),
                                                         false, false);
        const uint32_t p0 = p[0], p1 = p[1];
        r[m] = __builtin_bit_cast(float, p0) + __builtin_bit_cast(float, p1);
    }
    // w = 16: rows [X0 Y0 X2 Y2] + [X1 Y1 X3 Y3]
#pragma unroll
    for (int m = 0; m < HB / 4; m++) {
        const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, r[2 * m]),
                                                         __builtin_bit_cast(uint32_t, r[2 * m + 1]),
                                                         false, false);
        const uint32_t p0 = p[0], p1 = p[1];
        r[m] = __builtin_bit_cast(float, p0) + __builtin_bit_cast(float, p1);
    }
    const bool hi8 = (lane & 8u) != 0, hi4 = (lane & 4u) != 0;
    float x;
    if constexpr (HB >= 8) {
        // w = 8, paired: lanes with bit 3 clear take X's pair, the others Y's
#pragma unroll
        for (int m = 0; m < HB / 8; m++) {
            const float t = hi8 ? r[2 * m + 1] : r[2 * m];
            const float u = hi8 ? r[2 * m] : r[2 * m + 1];
            r[m] = t + dpp_mov<0x128>(u);  // row_ror:8: the partner is lane i ^ 8
        }
        if constexpr (HB == 16) {
            // w = 4, paired: lanes with bit 2 clear take X's pair, the others Y's
            const float t = hi4 ? r[1] : r[0];
            const float u = hi4 ? r[0] : r[1];
            x = t + xor4(u);
        } else {
            // w = 4 on one register: lanes with bit 2 clear get a[i] + a[i + 4]
            x = r[0] + dpp_mov<0x124>(r[0]);  // row_ror:4
        }
    } else {
        x = r[0] + dpp_mov<0x128>(r[0]);  // row_ror:8 (rows hold one head)
        x = x + dpp_mov<0x124>(x);        // row_ror:4, as lane_tree_x
    }
    x = x + dpp_mov<0xB1>(x);  // quad_perm [1,0,3,2]
    return x + dpp_mov<0x4E>(x);  // quad_perm [2,3,0,1]
}

// rms_scale_of: correctly rounded division and square root, in this order.
__device__ __forceinline__ float rms_scale_of(float ss, float n, float eps) {
    return 1.0f / sqrtf(ss / n + eps);
}

__global__ __launch_bounds__(64) void k_prelude(float *__restrict__ q, float *__restrict__ k,
                                                float *__restrict__ v, uint32_t heads,
                                                uint32_t kvh, uint32_t d, PreludeArgs a) {
    extern __shared__ float xs[];
    const uint32_t t = blockIdx.x / 3, part = blockIdx.x % 3, lane = threadIdx.x;
    const uint32_t n = part == 0 ? heads * d : kvh * d;
    float *x = (part == 0 ? q : part == 1 ? k : v) + (uint64_t)t * n;
    const float *bias = part == 0 ? a.q_bias : part == 1 ? a.k_bias : a.v_bias;
    for (uint32_t i = lane; i < n; i += 64) {
        float z = x[i];
        if (bias) z = z + bias[i];
        if (a.has_clip) z = z < -a.clip ? -a.clip : (z > a.clip ? a.clip : z);
        xs[i] = z;
    }
    __syncthreads();
    if (part == 2) {  // values: bias and clip only
        for (uint32_t i = lane; i < n; i += 64) x[i] = xs[i];
        return;
    }
    const float *w = part == 0 ? a.q_norm : a.k_norm;
    if (a.norm == QVKV_NORM_FULL && w) {
        float acc = 0.0f;
        for (uint32_t i = lane; i < n; i += 64) acc = fmaf(xs[i], xs[i], acc);
        const float r = rms_scale_of(lane_tree(acc), (float)n, a.eps);
        __syncthreads();
        for (uint32_t i = lane; i < n; i += 64) xs[i] = (xs[i] * r) * w[i];
    } else if (a.norm == QVKV_NORM_PER_HEAD && w) {
        for (uint32_t hd = 0; hd < n / d; hd++) {
            float *h = xs + hd * d;
            float acc = 0.0f;
            for (uint32_t i = lane; i < d; i += 64) acc = fmaf(h[i], h[i], acc);
            const float r = rms_scale_of(lane_tree(acc), (float)d, a.eps);
            __syncthreads();
            for (uint32_t i = lane; i < d; i += 64) h[i] = (h[i] * r) * w[i];
            __syncthreads();
        }
    }
    __syncthreads();
    const uint32_t half = d / 2;
    const float *cs = a.rope + (uint64_t)t * d;
    for (uint32_t u = lane; u < (n / d) * half; u += 64) {
        const uint32_t hd = u / half, i = u - hd * half;
        const float x1 = xs[hd * d + i], x2 = xs[hd * d + i + half];
        const float c = cs[i], s = cs[half + i];
        const float p1 = x1 * c, p2 = x2 * s, p3 = x2 * c, p4 = x1 * s;
        x[hd * d + i] = p1 - p2;
        x[hd * d + i + half] = p3 + p4;
    }
}

// Register form for d = 64, 128, 256: one wave per (token, q|k|v, batch of HB = 1024/d
// heads, or the whole row under a full-row norm), lane l holding elements 64j + l of each head (j < d/64) in
// registers.  A head's sum of squares is then lane l's in-order fma over j followed by the
// same 64-lane tree (lane_tree_x); the heads' totals are gathered one per lane so a single
// vector rms_scale_of serves every head of the wave.  Every RoPE pair (i, i + d/2) lies in
// one lane (d = 128, 256) or in lanes l and l ^ 32 (d = 64, exchanged by a lane swap).
// Loads and stores are dword-coalesced 256-byte runs; no LDS, no barriers, 4 independent
// waves per workgroup.  Measured against the LDS kernel at 65 536 tokens, 32 query heads:
// d = 128 with per-head norms 2.66 -> 0.60 ms, without norms 1.86 -> 0.52 ms; then with
// the heads' trees interleaved (head_trees) and a scalar wave index 0.68 -> 0.57 ms, and
// with non-temporal row loads and stores 0.51 ms (5.3 TB/s).
// FULL: one norm over each whole row (QkNorm::Full): the wave takes the whole q, k or v row
// (up to 4096 values, 64 per lane), whose element order h*d + 64j + l is lane l's order
// of the reference's reduction.
// One wave's share of a row: HB heads from h0 (nh of them present) of token t's q (part
// 0), k (1) or v (2) row at x.
template <int D, bool FULL, uint32_t HB>
__device__ __forceinline__ void prelude_heads(float *__restrict__ x, const float *bias,
                                              uint32_t h0, uint32_t nh, uint32_t part,
                                              uint32_t t, uint32_t lane, const PreludeArgs &a) {
    constexpr uint32_t J = D >= 64 ? D / 64 : 1;
    // Heads past nh (a partial batch) hold zeros and are neither loaded nor stored; every
    // other step runs on all HB heads, so the heads' work interleaves freely.
    float z[HB][J];
#pragma unroll
    for (uint32_t h = 0; h < HB; h++)
#pragma unroll
        for (uint32_t j = 0; j < J; j++)  // streamed once: non-temporal (+11 % at cfg5)
            z[h][j] = h < nh ? __builtin_nontemporal_load(&x[h * D + 64 * j + lane]) : 0.0f;
#pragma unroll
    for (uint32_t h = 0; h < HB; h++)
#pragma unroll
        for (uint32_t j = 0; j < J; j++) {
            float y = z[h][j];
            if (bias && h < nh) y = y + bias[(h0 + h) * D + 64 * j + lane];
            if (a.has_clip) y = y < -a.clip ? -a.clip : (y > a.clip ? a.clip : y);
            z[h][j] = y;
        }
    if (part != 2) {
        const float *w = part == 0 ? a.q_norm : a.k_norm;
        if (FULL && w) {
            float acc = 0.0f;
#pragma unroll
            for (uint32_t h = 0; h < HB; h++)
                if (h < nh)
#pragma unroll
                    for (uint32_t j = 0; j < J; j++) acc = fmaf(z[h][j], z[h][j], acc);
            const float rs = rms_scale_of(lane_tree_x(acc), (float)(nh * D), a.eps);
#pragma unroll
            for (uint32_t h = 0; h < HB; h++)
                if (h < nh)
#pragma unroll
                    for (uint32_t j = 0; j < J; j++)
                        z[h][j] = (z[h][j] * rs) * w[h * D + 64 * j + lane];
        } else if constexpr (!FULL) {
          if (a.norm == QVKV_NORM_PER_HEAD && w) {
            // every head's sum of squares in one interleaved pass; one rms_scale_of
            float acc[HB];
#pragma unroll
            for (uint32_t h = 0; h < HB; h++) {
                acc[h] = 0.0f;
#pragma unroll
                for (uint32_t j = 0; j < J; j++) acc[h] = fmaf(z[h][j], z[h][j], acc[h]);
            }
            const float rsv = rms_scale_of(head_trees<HB>(acc, lane), (float)D, a.eps);
            float wj[J];
#pragma unroll
            for (uint32_t j = 0; j < J; j++) wj[j] = w[64 * j + lane];
#pragma unroll
            for (uint32_t h = 0; h < HB; h++) {
                const float rs = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, rsv),
                                                     head_lane<HB>((int)h)));
#pragma unroll
                for (uint32_t j = 0; j < J; j++) z[h][j] = (z[h][j] * rs) * wj[j];
            }
          }
        }
        const float *cs = a.rope + (uint64_t)t * D;
        if constexpr (D == 64) {
            const uint32_t i = lane & 31u;
            const float c = cs[i], sn = cs[32 + i];
            const bool first = lane < 32;
#pragma unroll
            for (uint32_t h = 0; h < HB; h++) {
                {
                    // v_permlane32_swap of z with itself: lanes l and l ^ 32 both get
                    // (x[l mod 32], x[l mod 32 + 32]) = (x1, x2) of their pair
                    const uint32_t zu = __builtin_bit_cast(uint32_t, z[h][0]);
                    const auto pr = __builtin_amdgcn_permlane32_swap(zu, zu, false, false);
                    const uint32_t u1 = pr[0], u2 = pr[1];
                    const float x1 = __builtin_bit_cast(float, u1);
                    const float x2 = __builtin_bit_cast(float, u2);
                    const float p1 = x1 * c, p2 = x2 * sn, p3 = x2 * c, p4 = x1 * sn;
                    z[h][0] = first ? p1 - p2 : p3 + p4;
                }
            }
        } else {
            constexpr uint32_t JH = J / 2;  // pairs (j, j + JH)
            float c[JH], sn[JH];
#pragma unroll
            for (uint32_t jj = 0; jj < JH; jj++) {
                c[jj] = cs[64 * jj + lane];
                sn[jj] = cs[D / 2 + 64 * jj + lane];
            }
#pragma unroll
            for (uint32_t h = 0; h < HB; h++)
#pragma unroll
                    for (uint32_t jj = 0; jj < JH; jj++) {
                        const float x1 = z[h][jj], x2 = z[h][jj + JH];
                        const float p1 = x1 * c[jj], p2 = x2 * sn[jj], p3 = x2 * c[jj],
                                    p4 = x1 * sn[jj];
                        z[h][jj] = p1 - p2;
                        z[h][jj + JH] = p3 + p4;
                    }
        }
    }
#pragma unroll
    for (uint32_t h = 0; h < HB; h++)
        if (h < nh)
#pragma unroll
            for (uint32_t j = 0; j < J; j++)
                __builtin_nontemporal_store(z[h][j], &x[h * D + 64 * j + lane]);
}

// One wave per (token, q|k|v, batch of HB heads).  (Fewer heads per wave on k and v rows
// with few KV heads, 4 instead of 16 at cfg5's 4 KV heads, measured 17 % slower.)
template <int D, bool FULL, int VPW = 1024>
__global__ __launch_bounds__(256) void k_prelude_r(float *__restrict__ q, float *__restrict__ k,
                                                   float *__restrict__ v, uint32_t s,
                                                   uint32_t heads, uint32_t kvh, uint32_t uq,
                                                   uint32_t ukv, PreludeArgs a) {
    // heads per wave: 1024 values was the best of 512, 1024, 2048 without a full norm
    constexpr uint32_t HB = (FULL ? 4096 : VPW) / D;
    const uint32_t per_tok = uq + 2 * ukv;
    // the wave index as a scalar: every per-head branch below is then a scalar branch
    const uint32_t u = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = u / per_tok;
    if (t >= s) return;
    const uint32_t r = u - t * per_tok;
    const uint32_t part = r < uq ? 0u : (r < uq + ukv ? 1u : 2u);
    const uint32_t h0 = (part == 0 ? r : part == 1 ? r - uq : r - uq - ukv) * HB;
    const uint32_t row_heads = part == 0 ? heads : kvh;
    const uint32_t nh = min(HB, row_heads - h0);
    float *x = (part == 0 ? q : part == 1 ? k : v) + ((uint64_t)t * row_heads + h0) * D;
    const float *bias = part == 0 ? a.q_bias : part == 1 ? a.k_bias : a.v_bias;
    prelude_heads<D, FULL, HB>(x, bias, h0, nh, part, t, lane, a);
}

// Full-row norm (QkNorm::Full), rows up to 4096 values.  Lane l owns elements 64 j + l of a
// row as in the reference's reduction; a row's j are spread over WPR waves of a workgroup
// (16 each), so its loads are spread too (16 values per lane per wave instead of up to 64
// in one), and a workgroup holds 4 / WPR rows.  The sum of squares stays lane l's fused
// multiply-add chain over j in order: with WPR > 1 each wave continues the running sum the
// wave before left in LDS.  The RoPE pairs of a head lie in one wave (a head is d/64
// consecutive j).  rows: q rows (part 0, row = token), or k and v rows (row 2 t + 0 / 1).
template <int D, int WPR>
__global__ __launch_bounds__(256) void k_prelude_full(float *__restrict__ q, float *__restrict__ k,
                                                      float *__restrict__ v, uint32_t s,
                                                      uint32_t heads, uint32_t kvh, bool kv_rows,
                                                      PreludeArgs a) {
    constexpr uint32_t JW = 16;            // elements per lane per wave
    constexpr uint32_t JD = D / 64;        // elements per lane per head
    constexpr uint32_t RPW = 4 / WPR;      // rows per workgroup
    __shared__ float run[RPW][64];
    __shared__ float scale_of_row[RPW];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rw = w / WPR, wr = w % WPR;  // the wave's row in the workgroup, its part of it
    const uint32_t row = blockIdx.x * RPW + rw;
    const bool live = row < (kv_rows ? 2 * s : s);
    const uint32_t t = kv_rows ? row / 2 : row;
    const uint32_t part = kv_rows ? 1u + (row & 1u) : 0u;
    const uint32_t nh = part == 0 ? heads : kvh;
    const uint32_t J = nh * JD;            // elements per lane in the row (at most 64)
    const uint32_t j0 = wr * JW;
    const uint32_t nj = live && J > j0 ? (J - j0 < JW ? J - j0 : JW) : 0u;
    float *x = (part == 0 ? q : part == 1 ? k : v) + (uint64_t)t * nh * D;
    const float *bias = part == 0 ? a.q_bias : part == 1 ? a.k_bias : a.v_bias;
    float z[JW];
#pragma unroll
    for (uint32_t u = 0; u < JW; u++)
        z[u] = u < nj ? __builtin_nontemporal_load(&x[64 * (j0 + u) + lane]) : 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < JW; u++) {
        float y = z[u];
        if (bias && u < nj) y = y + bias[64 * (j0 + u) + lane];
        if (a.has_clip) y = y < -a.clip ? -a.clip : (y > a.clip ? a.clip : y);
        z[u] = y;
    }
    // (every wave of a workgroup takes the barriers: the norm's presence is per launch for
    // q rows; k and v rows alternate, and only the k rows' waves use the chain)
    const float *wn = part == 0 ? a.q_norm : part == 1 ? a.k_norm : nullptr;
    const bool norm_any = kv_rows ? a.k_norm != nullptr : a.q_norm != nullptr;
    if (norm_any) {
        float acc = 0.0f;
        if constexpr (WPR == 1) {
#pragma unroll
            for (uint32_t u = 0; u < JW; u++)
                if (u < nj) acc = fmaf(z[u], z[u], acc);
        } else {
            for (uint32_t step = 0; step < WPR; step++) {
                if (wr == step) {
                    acc = step == 0 ? 0.0f : run[rw][lane];
#pragma unroll
                    for (uint32_t u = 0; u < JW; u++)
                        if (u < nj) acc = fmaf(z[u], z[u], acc);
                    run[rw][lane] = acc;
                }
                __syncthreads();
            }
            acc = run[rw][lane];
        }
        float rs = 0.0f;
        if constexpr (WPR == 1) {
            rs = rms_scale_of(lane_tree_x(acc), (float)(nh * D), a.eps);
        } else {
            if (wr == 0) {
                const float r = rms_scale_of(lane_tree_x(acc), (float)(nh * D), a.eps);
                if (lane == 0) scale_of_row[rw] = r;
            }
            __syncthreads();
            rs = scale_of_row[rw];
        }
        if (wn != nullptr) {
#pragma unroll
            for (uint32_t u = 0; u < JW; u++)
                if (u < nj) z[u] = (z[u] * rs) * wn[64 * (j0 + u) + lane];
        }
    }
    if (part != 2 && nj != 0) {
        const float *cs = a.rope + (uint64_t)t * D;
        if constexpr (D == 64) {
            const uint32_t i = lane & 31u;
            const float c = cs[i], sn = cs[32 + i];
            const bool first = lane < 32;
#pragma unroll
            for (uint32_t u = 0; u < JW; u++) {
                // v_permlane32_swap of z with itself: lanes l and l ^ 32 both get
                // (x[l mod 32], x[l mod 32 + 32]) = (x1, x2) of their pair
                const uint32_t zu = __builtin_bit_cast(uint32_t, z[u]);
                const auto pr = __builtin_amdgcn_permlane32_swap(zu, zu, false, false);
                const uint32_t u1 = pr[0], u2 = pr[1];
                const float x1 = __builtin_bit_cast(float, u1);
                const float x2 = __builtin_bit_cast(float, u2);
                const float p1 = x1 * c, p2 = x2 * sn, p3 = x2 * c, p4 = x1 * sn;
                z[u] = first ? p1 - p2 : p3 + p4;
            }
        } else {
            constexpr uint32_t JH = JD / 2;  // pairs (jj, jj + JH) of a head
            float c[JH], sn[JH];
#pragma unroll
            for (uint32_t jj = 0; jj < JH; jj++) {
                c[jj] = cs[64 * jj + lane];
                sn[jj] = cs[D / 2 + 64 * jj + lane];
            }
#pragma unroll
            for (uint32_t h = 0; h < JW / JD; h++)
#pragma unroll
                for (uint32_t jj = 0; jj < JH; jj++) {
                    const float x1 = z[h * JD + jj], x2 = z[h * JD + jj + JH];
                    const float p1 = x1 * c[jj], p2 = x2 * sn[jj], p3 = x2 * c[jj],
                                p4 = x1 * sn[jj];
                    z[h * JD + jj] = p1 - p2;
                    z[h * JD + jj + JH] = p3 + p4;
                }
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < JW; u++)
        if (u < nj) __builtin_nontemporal_store(z[u], &x[64 * (j0 + u) + lane]);
}

hipError_t launch_prelude(float *q, float *k, float *v, uint32_t s, uint32_t heads,
                          uint32_t kvh, uint32_t d, const PreludeArgs &a, hipStream_t st) {
    if (s == 0) return hipSuccess;
    const bool full = a.norm == QVKV_NORM_FULL;
    if ((d == 64 || d == 128 || d == 256) && (!full || (heads * d <= 4096 && kvh * d <= 4096)) &&
        tune(KNOB_PRELUDE_FAST) != 0) {
        // per-head norms at d = 128: 2048 values per wave (one vector rms serves 16 heads;
        // +2 % at 32 query heads; 5 % slower at d = 256, equal at d = 64)
        const bool wide = !full && a.norm == QVKV_NORM_PER_HEAD && d == 128 &&
                          tune(KNOB_PRELUDE_WIDE) != 0;
        if (full && tune(KNOB_PRELUDE_FULL_WG) != 0) {
            // q rows, then k and v rows: waves per row by the row's length (16 values per
            // lane per wave)
            for (int kv = 0; kv < 2; kv++) {
                const uint32_t J = (kv ? kvh : heads) * (d / 64);
                const int wpr = J > 32 ? 4 : J > 16 ? 2 : 1;
                const uint64_t rows = (uint64_t)s * (kv ? 2 : 1);
                const uint64_t grid = (rows * wpr + 3) / 4;
                if (grid > 0x7fffffffull) return hipErrorInvalidValue;
#define QV_PRE_FULL(DD, WW)                                                                     \
    hipLaunchKernelGGL((k_prelude_full<DD, WW>), dim3((unsigned)grid), dim3(256), 0, st, q, k, v, \
                       s, heads, kvh, kv != 0, a)
#define QV_PRE_FULL_D(DD)                                                                       \
    do {                                                                                        \
        if (wpr == 4) QV_PRE_FULL(DD, 4);                                                       \
        else if (wpr == 2) QV_PRE_FULL(DD, 2);                                                  \
        else QV_PRE_FULL(DD, 1);                                                                \
    } while (0)
                if (d == 64) QV_PRE_FULL_D(64);
                else if (d == 128) QV_PRE_FULL_D(128);
                else QV_PRE_FULL_D(256);
#undef QV_PRE_FULL_D
#undef QV_PRE_FULL
                hipError_t e = hipGetLastError();
                if (e != hipSuccess) return e;
            }
            return hipSuccess;
        }
        const uint32_t hb = (full ? 4096u : wide ? 2048u : 1024u) / d;
        const uint32_t uq = (heads + hb - 1) / hb, ukv = (kvh + hb - 1) / hb;
        const uint64_t waves = (uint64_t)s * (uq + 2 * ukv);
        const uint64_t grid = (waves + 3) / 4;
        if (waves > 0xffffffffull || grid > 0x7fffffffull) return hipErrorInvalidValue;
#define QV_PRE_L(DD, FF, VPW)                                                                   \
    hipLaunchKernelGGL((k_prelude_r<DD, FF, VPW>), dim3((unsigned)grid), dim3(256), 0, st, q, k, \
                       v, s, heads, kvh, uq, ukv, a)
#define QV_PRE(DD)                                                                              \
    do {                                                                                        \
        if (full) QV_PRE_L(DD, true, 1024);                                                     \
        else if (wide && DD == 128) QV_PRE_L(DD, false, (DD == 128 ? 2048 : 1024));            \
        else QV_PRE_L(DD, false, 1024);                                                         \
    } while (0)
        if (d == 64) QV_PRE(64);
        else if (d == 128) QV_PRE(128);
        else QV_PRE(256);
#undef QV_PRE
#undef QV_PRE_L
        return hipGetLastError();
    }
    const uint64_t lds = (uint64_t)(heads > kvh ? heads : kvh) * d * 4;
    hipLaunchKernelGGL(k_prelude, dim3(s * 3), dim3(64), (uint32_t)lds, st, q, k, v, heads, kvh,
                       d, a);
    return hipGetLastError();
}

}  // namespace qvkv
