/*
 * CPU oracle for the paged KV-cache hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference's CPU algorithm for the path, so the
 * HIP kernels can be checked against it on identical seeded inputs.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the
 * checker (or the timed CPU baseline) -- never as part of the product path.
 *
 * Every function cites the reference file:line it follows (paths relative to the
 * reference repository root, kentmarete/qubivex).
 *
 * Pinning (what checks each function beyond its own restatement):
 *   orc_f16_to_f32        every one of the 65536 bit patterns against numpy float16
 *   orc_f32_to_f16        every f16 round-trip, 2^24 strided f32 patterns and all
 *                         halfway cases against numpy astype(float16) (IEEE RNE)
 *   orc_f32_to_f16_fixture  equals orc_f32_to_f16 on the normal range; flushes below
 *   orc_q8_0_dequant      golden vector fixtures/oracle/ggml_dequant.json (gguf-py 0.19.0)
 *   orc_q8_0_quantize     closed-form edge cases (zeros, ties, +-amax, NaN, inf) and
 *                         quantize(dequant(q)) idempotence on golden blocks
 *   orc_exp               <= 2 ulp against libm exp in double over ~4M points, edge cases
 *                         (the reference's own test, math.rs:187-229)
 *   orc_attend            f64 attention within 1e-5; one position gives v_0; equal scores
 *                         give the mean of v; softmax sums to 1
 *   orc_sim_*             round trips store->gather; independent numpy addressing
 *
 * Build: gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp -shared -fPIC
 * (contraction must stay off: the reference's arithmetic is written with explicit fma).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_F16 1
#define ORC_Q8_0 2

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 -> f32, exactly.  crates/qubivex-backend-cpu/src/formats.rs:21-41 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t m = man, e = 127 - 15 + 1;
        while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
        bits = sign | (e << 23) | ((m & 0x3ffu) << 13);
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    return u2f(bits);
}

/* f32 -> f16 bits exactly as xtask/src/fixtures.rs:45-67 writes it: round to nearest
 * even on the normal range, results below the normal range flushed to signed zero,
 * overflow to infinity (NaN also maps to infinity there).  Kept to document the
 * deviation: the KV path uses orc_f32_to_f16 below, which keeps f16 subnormals. */
uint16_t orc_f32_to_f16_fixture(float x) {
    uint32_t b = f2u(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xffu) - 127 + 15;
    uint32_t man = b & 0x7fffffu;
    if (exp <= 0) return sign;
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    uint32_t h = (uint32_t)sign | ((uint32_t)exp << 10) | (man >> 13);
    uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u) == 1u)) h += 1;
    return (uint16_t)h;
}

/* f32 -> f16 bits, IEEE-754 round to nearest even, with f16 subnormals, overflow to
 * infinity and NaN kept NaN (quiet, payload's top bits kept).  This is the narrowing of
 * xtask/src/fixtures.rs:45-67 extended to the whole f32 range (the fixture helper
 * flushes below 2^-14; N(0,1) KV data reaches that range, so the store must not). */
uint16_t orc_f32_to_f16(float x) {
    uint32_t b = f2u(x);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t absb = b & 0x7fffffffu;
    if (absb > 0x7f800000u) /* NaN */
        return (uint16_t)(sign | 0x7e00u | ((absb >> 13) & 0x3ffu));
    if (absb >= 0x477ff000u) /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    int32_t e = (int32_t)(absb >> 23) - 127; /* unbiased exponent */
    if (e >= -14) {                          /* normal f16 */
        uint32_t man = absb & 0x7fffffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (man >> 13);
        uint32_t rest = man & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* may carry into exp */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return (uint16_t)sign; /* below half the smallest subnormal */
    /* subnormal: value = m * 2^-24, m = round(|x| * 2^24) */
    uint32_t man = (absb & 0x7fffffu) | 0x800000u; /* 24-bit significand, value = man*2^(e-23) */
    int32_t shift = -e - 1;                        /* man * 2^(e-23) / 2^-24 = man >> (-e-1) */
    uint32_t q = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return (uint16_t)(sign | q);
}

/* Rust's f32::round: half away from zero. */
static inline float round_away(float x) { return roundf(x); }

/* Rust `f as i8` after clamp(-127, 127): NaN -> 0 (saturating cast). */
static inline int8_t to_i8(float x) {
    if (x != x) return 0;
    float c = x < -127.0f ? -127.0f : (x > 127.0f ? 127.0f : x);
    return (int8_t)c;
}

/* q8_0 quantize: per 32 values an f16 scale (little-endian) then 32 int8.
 * xtask/src/fixtures.rs:70-84:  amax = fold(0, max(|x|)); d = amax/127 (f32);
 * stored scale = f16(d) (RNE; here with subnormals, see orc_f32_to_f16);
 * inv = d > 0 ? 1/d : 0 from the f32 d (not the rounded one);
 * q = (round(x*inv).clamp(-127,127)) as i8.   n must be a multiple of 32. */
void orc_q8_0_quantize(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *blk = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i])); /* Rust max: NaN ignored */
        float d = amax / 127.0f;
        uint16_t h = orc_f32_to_f16(d);
        out[b * 34 + 0] = (uint8_t)(h & 0xff);
        out[b * 34 + 1] = (uint8_t)(h >> 8);
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
        for (int i = 0; i < 32; i++) {
            float r = round_away(blk[i] * inv);
            out[b * 34 + 2 + i] = (uint8_t)to_i8(r);
        }
    }
}

/* q8_0 dequant, y = f32(q) * f16_to_f32(d), one multiply.
 * crates/qubivex-backend-cpu/src/formats.rs:90-99 */
void orc_q8_0_dequant(const uint8_t *row, size_t n, float *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = row + b * 34;
        float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; i++) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

/* ---- crates/qubivex-compute/src/math.rs:13-75: exp from IEEE ops only ---- */
#define LOG2E 1.44269502f /* std::f32::consts::LOG2_E */
static const uint32_t LN2_HI_BITS = 0x3f317200u, LN2_LO_BITS = 0x35bfbe8eu;
static const float SHIFT = 12582912.0f;
static const float OVERFLOW_X = 88.72284f;
static const float UNDERFLOW_X = -87.33655f;
static const uint32_t P_BITS[6] = {0x39506967u, 0x3ab743ceu, 0x3c088908u,
                                   0x3d2aa9c1u, 0x3e2aaaaau, 0x3f000000u};

static inline float pow2i(int k) { return u2f((uint32_t)(k + 127) << 23); }

float orc_exp(float x) {
    if (x != x) return x;
    if (x > OVERFLOW_X) return INFINITY;
    if (x < UNDERFLOW_X) return 0.0f;
    float kf = (x * LOG2E + SHIFT) - SHIFT;
    float r = fmaf(-kf, u2f(LN2_HI_BITS), x);
    r = fmaf(-kf, u2f(LN2_LO_BITS), r);
    float p = u2f(P_BITS[0]);
    for (int i = 1; i < 6; i++) p = fmaf(p, r, u2f(P_BITS[i]));
    float y = fmaf(p, r * r, r) + 1.0f;
    int k = (int)kf;
    int k1 = k >> 1;
    float v = (y * pow2i(k1)) * pow2i(k - k1);
    return v < 1.17549435e-38f ? 0.0f : v;
}

/* Softmax in place, max-subtracted, sequential sum.  math.rs:120-130
 * (fold(NEG_INFINITY, f32::max) ignores NaN, as fmaxf does). */
void orc_softmax(float *x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) { x[i] = orc_exp(x[i] - m); sum += x[i]; }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* Sequential fma dot.  math.rs:134-136 */
static inline float dot_seq(const float *a, const float *b, size_t d) {
    float s = 0.0f;
    for (size_t i = 0; i < d; i++) s = fmaf(a[i], b[i], s);
    return s;
}

/* Causal attention of one query head over positions 0..=pos of one KV head whose keys
 * and values are d floats per position (position-major).  math.rs:142-155.
 * scores: scratch of at least pos+1 floats. */
void orc_attend(const float *q, const float *k, const float *v, size_t d, size_t pos,
                float *out, float *scores) {
    float scale = 1.0f / sqrtf((float)d);
    for (size_t t = 0; t <= pos; t++) scores[t] = dot_seq(q, k + t * d, d) * scale;
    orc_softmax(scores, pos + 1);
    for (size_t i = 0; i < d; i++) out[i] = 0.0f;
    for (size_t t = 0; t <= pos; t++) {
        float p = scores[t];
        const float *vr = v + t * d;
        for (size_t i = 0; i < d; i++) out[i] = fmaf(p, vr[i], out[i]);
    }
}

/* The same attention in f64 with libm exp: an independent check on orc_attend (and the
 * tolerance reference for the GPU's reordered sums). */
void orc_attend_f64(const float *q, const float *k, const float *v, size_t d, size_t pos,
                    double *out, double *scores) {
    double scale = 1.0 / sqrt((double)d);
    double m = -INFINITY;
    for (size_t t = 0; t <= pos; t++) {
        double s = 0.0;
        for (size_t i = 0; i < d; i++) s += (double)q[i] * (double)k[t * d + i];
        scores[t] = s * scale;
        if (scores[t] > m) m = scores[t];
    }
    double sum = 0.0;
    for (size_t t = 0; t <= pos; t++) { scores[t] = exp(scores[t] - m); sum += scores[t]; }
    for (size_t i = 0; i < d; i++) out[i] = 0.0;
    for (size_t t = 0; t <= pos; t++) {
        double p = scores[t] / sum;
        for (size_t i = 0; i < d; i++) out[i] += p * (double)v[t * d + i];
    }
}

/* ---- The simulated device pool (crates/qubivex-backend-cpu/src/sim.rs:301-436) ----
 *
 * The reference pool holds f32 words per block: keys dimension-major
 * [kv_head][d][BLOCK], then values position-major [BLOCK][kv_head][d]
 * (crates/qubivex-compute/src/discrete.rs:247-255,319-329), BLOCK = 256 there.
 * Here BLOCK is a parameter (16 for this path), and the store narrows each value
 * through the storage dtype first (f16: RNE; q8_0: quantize then dequantize over each
 * head's 32-value groups), so the pool holds the logical values a reader sees. */

static inline size_t block_words(size_t kv_out, size_t B) { return 2 * B * kv_out; }

/* discrete.rs:319-322, kv_key_word with KV_BLOCK = B */
static inline size_t key_word(size_t kv_out, size_t d, size_t B, size_t at, size_t g, size_t i) {
    size_t b = at / B, slot = at % B;
    return b * block_words(kv_out, B) + (g * d + i) * B + slot;
}
/* discrete.rs:326-329, kv_value_word with KV_BLOCK = B */
static inline size_t value_word(size_t kv_out, size_t d, size_t B, size_t at, size_t g, size_t i) {
    size_t b = at / B, slot = at % B;
    return b * block_words(kv_out, B) + B * kv_out + slot * kv_out + g * d + i;
}

size_t orc_key_word(size_t kv_out, size_t d, size_t B, size_t at, size_t g, size_t i) {
    return key_word(kv_out, d, B, at, g, i);
}
size_t orc_value_word(size_t kv_out, size_t d, size_t B, size_t at, size_t g, size_t i) {
    return value_word(kv_out, d, B, at, g, i);
}

/* One row of kv_out values narrowed through the storage dtype, head by head. */
static void narrow_row(int dtype, const float *x, size_t kvh, size_t d, float *y) {
    size_t kv_out = kvh * d;
    if (dtype == ORC_F16) {
        for (size_t i = 0; i < kv_out; i++) y[i] = orc_f16_to_f32(orc_f32_to_f16(x[i]));
    } else if (dtype == ORC_Q8_0) {
        uint8_t tmp[34];
        for (size_t g = 0; g < kvh; g++)
            for (size_t j = 0; j < d; j += 32) {
                orc_q8_0_quantize(x + g * d + j, 32, tmp);
                orc_q8_0_dequant(tmp, 32, y + g * d + j);
            }
    } else {
        memcpy(y, x, kv_out * sizeof(float));
    }
}

/* The store: rows k[r], v[r] (kv_out each) to pool positions slot[r] = block*B + offset.
 * sim.rs:377-399 (`put`, host sync rows first, then the new tokens: the caller orders
 * the rows the same way). */
void orc_sim_store(float *pool, int dtype, size_t kvh, size_t d, size_t B, const float *k,
                   const float *v, const uint32_t *slot, size_t n) {
    size_t kv_out = kvh * d;
    float *ky = malloc(kv_out * sizeof(float)), *vy = malloc(kv_out * sizeof(float));
    for (size_t r = 0; r < n; r++) {
        narrow_row(dtype, k + r * kv_out, kvh, d, ky);
        narrow_row(dtype, v + r * kv_out, kvh, d, vy);
        for (size_t g = 0; g < kvh; g++)
            for (size_t i = 0; i < d; i++) {
                pool[key_word(kv_out, d, B, slot[r], g, i)] = ky[g * d + i];
                pool[value_word(kv_out, d, B, slot[r], g, i)] = vy[g * d + i];
            }
    }
    free(ky);
    free(vy);
}

/* Position p of item t: blocks[table_at[t] + p/B]*B + p%B.  sim.rs:359-366 (`at`). */
static inline size_t at_of(const uint32_t *blocks, const uint32_t *table_at, size_t t,
                           size_t p, size_t B) {
    return (size_t)blocks[table_at[t] + p / B] * B + p % B;
}

/* The gather of item t: positions 0..n-1 per KV head into ks[g][p*d+i], vs[g][p*d+i]
 * (out_k/out_v: kvh * n * d floats, head-major).  sim.rs:404-422 */
void orc_sim_gather(const float *pool, size_t kvh, size_t d, size_t B, const uint32_t *blocks,
                    const uint32_t *table_at, size_t t, size_t n, float *out_k, float *out_v) {
    size_t kv_out = kvh * d;
    for (size_t p = 0; p < n; p++) {
        size_t to = at_of(blocks, table_at, t, p, B);
        for (size_t g = 0; g < kvh; g++)
            for (size_t i = 0; i < d; i++) {
                out_k[(g * n + p) * d + i] = pool[key_word(kv_out, d, B, to, g, i)];
                out_v[(g * n + p) * d + i] = pool[value_word(kv_out, d, B, to, g, i)];
            }
    }
}

/* Decode attention over the pool for n_items items (each its own sequence at pos[t]):
 * gather each item's keys and values per KV head, then `attend` for every query head
 * with the GQA map g = h / (heads/kvh).  sim.rs:404-428; the parallel loop over
 * (token, head) is crates/qubivex-arch/src/lib.rs:1312-1320 (rayon par_chunks_mut),
 * here OpenMP over (item, head) with the gather done once per item.
 * q, out: [n_items][heads][d]. */
void orc_sim_attention(const float *pool, size_t kvh, size_t d, size_t B, size_t heads,
                       const uint32_t *blocks, const uint32_t *table_at, const uint32_t *pos,
                       size_t n_items, const float *q, float *out, int threads) {
    size_t group = heads / kvh;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    for (size_t t = 0; t < n_items; t++) {
        size_t n = (size_t)pos[t] + 1;
        float *ks = malloc(kvh * n * d * sizeof(float));
        float *vs = malloc(kvh * n * d * sizeof(float));
        orc_sim_gather(pool, kvh, d, B, blocks, table_at, t, n, ks, vs);
#pragma omp parallel
        {
            float *scores = malloc(n * sizeof(float));
#pragma omp for schedule(static)
            for (size_t h = 0; h < heads; h++) {
                size_t g = h / group;
                orc_attend(q + (t * heads + h) * d, ks + g * n * d, vs + g * n * d, d, n - 1,
                           out + (t * heads + h) * d, scores);
            }
            free(scores);
        }
        free(ks);
        free(vs);
    }
}

/* The store of a batch of rows as the host cache keeps it: per KV head a memcpy of d
 * values (crates/qubivex-arch/src/lib.rs:499-514, KvCache::store), narrowed through the
 * storage dtype; here into the paged pool at each row's slot. Used as the append leg of
 * the CPU baseline, OpenMP over rows. */
void orc_append_rows(float *pool, int dtype, size_t kvh, size_t d, size_t B, const float *k,
                     const float *v, const uint32_t *slot, size_t n, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < n; r++)
        orc_sim_store(pool, dtype, kvh, d, B, k + r * kvh * d, v + r * kvh * d, slot + r, 1);
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---- the prelude: crates/qubivex-compute/src/reduce.rs, math.rs, arch/src/lib.rs ---- */

/* reduce::dot (reduce.rs:11-50): 64 f32 lanes, one fma per lane per 64-element chunk,
 * chunks in increasing order, the tail in lanes 0..rem, then the halving tree
 * a[i] += a[i+w] for w = 32, 16, 8, 4 and (a0 + a1) + (a2 + a3). */
float orc_reduce_dot(const float *w, const float *x, size_t n) {
    float acc[64] = {0};
    size_t full = n / 64 * 64;
    for (size_t c = 0; c < full; c += 64)
        for (int l = 0; l < 64; l++) acc[l] = fmaf(w[c + l], x[c + l], acc[l]);
    for (size_t l = 0; l < n - full; l++) acc[l] = fmaf(w[full + l], x[full + l], acc[l]);
    for (int wd = 32; wd >= 4; wd /= 2)
        for (int i = 0; i < wd; i++) acc[i] += acc[i + wd];
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

/* math::rms_norm / rms_scale / rms_scale_of (math.rs:89-116): x = (x * r) * w with
 * r = 1 / sqrt(ss / n + eps), eps already cast to f32. */
void orc_rms_norm(float *x, const float *w, size_t n, float eps) {
    float ss = orc_reduce_dot(x, x, n);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) x[i] = (x[i] * r) * w[i];
}

/* math::rope_rotate (math.rs:160-169): NeoX pairs i, i + d/2 with a table row
 * cs = [cos..., sin...]. */
void orc_rope_rotate(float *head, const float *cs, size_t d) {
    size_t half = d / 2;
    for (size_t i = 0; i < half; i++) {
        float x1 = head[i], x2 = head[i + half];
        head[i] = x1 * cs[i] - x2 * cs[half + i];
        head[i + half] = x2 * cs[i] + x1 * cs[half + i];
    }
}

/* The prelude of the host forward pass (crates/qubivex-arch/src/lib.rs:1258-1292), in
 * place on s tokens: bias, clip, QK norm (0 none, 1 full width, 2 per head), RoPE with
 * token t's table row rope[t*d ..]. */
void orc_prelude(float *q, float *k, float *v, size_t s, size_t heads, size_t kvh, size_t d,
                 const float *qb, const float *kb, const float *vb, int has_clip, float clip,
                 int norm, const float *qn, const float *kn, float eps, const float *rope) {
    size_t q_out = heads * d, kv_out = kvh * d;
    float *ys[3] = {q, k, v};
    const float *bs[3] = {qb, kb, vb};
    size_t ns[3] = {q_out, kv_out, kv_out};
    for (int part = 0; part < 3; part++)
        if (bs[part])
            for (size_t t = 0; t < s; t++)
                for (size_t i = 0; i < ns[part]; i++) ys[part][t * ns[part] + i] += bs[part][i];
    if (has_clip)
        for (int part = 0; part < 3; part++)
            for (size_t i = 0; i < s * ns[part]; i++) {
                float z = ys[part][i];
                ys[part][i] = z < -clip ? -clip : (z > clip ? clip : z);
            }
    if (norm == 1) {
        for (size_t t = 0; t < s; t++) {
            orc_rms_norm(q + t * q_out, qn, q_out, eps);
            orc_rms_norm(k + t * kv_out, kn, kv_out, eps);
        }
    } else if (norm == 2) {
        for (size_t r = 0; r < s * heads; r++) orc_rms_norm(q + r * d, qn, d, eps);
        for (size_t r = 0; r < s * kvh; r++) orc_rms_norm(k + r * d, kn, d, eps);
    }
    for (size_t t = 0; t < s; t++) {
        for (size_t h = 0; h < heads; h++) orc_rope_rotate(q + t * q_out + h * d, rope + t * d, d);
        for (size_t h = 0; h < kvh; h++) orc_rope_rotate(k + t * kv_out + h * d, rope + t * d, d);
    }
}

/* Vector form of orc_exp (test convenience). */
void orc_exp_vec(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_exp(x[i]);
}

/* Vector form of orc_f32_to_f16 (test convenience). */
void orc_f16_encode(const float *x, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(x[i]);
}

/* Vector form of orc_f16_to_f32 (test convenience). */
void orc_f16_decode(const uint16_t *h, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}
