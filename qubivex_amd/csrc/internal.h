// Internal interface between the C ABI (abi.hip, pool.cpp) and the kernels (kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qvkv.h"

namespace qvkv {

// Byte offsets inside one block.  f16: K [G][B][d] f16, then V [G][B][d] f16.
// q8_0: K int8 [G][B][d] (row bytes permuted, see kernels.hip), K scales [G][B][d/32]
// f16, V int8 [G][B][d] (permuted), V scales [G][B][d/32] f16.
struct Geometry {
    int dtype, G, D, B;
    uint64_t kv_out;
    uint64_t block_bytes;
    uint64_t k_off, ks_off, v_off, vs_off;
};

// Records the calling thread's last error (returned by qvkv_last_error); returns code.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Detail of the calling thread's last QVKV_E_OOM (ComputeError::OutOfDeviceMemory's
// requested / used / capacity bytes); set together with the error, read by qvkv_last_oom.
struct OomDetail {
    uint64_t requested = 0, used = 0, capacity = 0;
};
void set_oom(uint64_t requested, uint64_t used, uint64_t capacity);
OomDetail last_oom();

// qvkv_block_copy; with `ordered`, the copy runs after the work queued on stream `after`
// (a hipStream_t; 0 is the null stream) when the call was made.  `overlap(ctx)`, when
// given, runs on the host once the copy is launched, before the call waits for it.
int block_copy_after(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                     const uint32_t *src, const uint32_t *dst, uint32_t n, bool ordered,
                     void *after, void (*overlap)(void *) = nullptr, void *ctx = nullptr);

// Makes the device of `dev` current on the calling thread (QVKV_OK or QVKV_E_DEVICE).
int use_device(qvkv_dev *dev);

// Validates a layout and fills the geometry; returns a QVKV_* status and a message.
int make_geometry(const qvkv_layout *l, Geometry *g, const char **why);

// Kernel launchers; all enqueue on `stream` and return hipError_t of the launch.
hipError_t launch_append(const Geometry &g, void *pool, uint64_t pool_blocks, const float *k,
                         const float *v, const uint32_t *slots, uint32_t n, int *err,
                         hipStream_t s);
hipError_t launch_gather(const Geometry &g, const void *pool, uint64_t pool_blocks,
                         const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                         const uint32_t *lens, const uint64_t *out_at, uint32_t n_items,
                         uint32_t max_len, int out_dtype, uint64_t out_positions, void *out_k,
                         void *out_v, int *err, hipStream_t s);
hipError_t launch_block_copy(const Geometry &g, void *pool, uint64_t pool_blocks,
                             const uint32_t *src, const uint32_t *dst, uint32_t n, int *err,
                             hipStream_t s);

// The prelude (prelude.hip): device pointers, contract-off f32 arithmetic.
struct PreludeArgs {
    uint32_t norm, has_clip;
    float clip, eps;
    const float *q_bias, *k_bias, *v_bias, *q_norm, *k_norm, *rope;
};
hipError_t launch_prelude(float *q, float *k, float *v, uint32_t s, uint32_t heads,
                          uint32_t kvh, uint32_t d, const PreludeArgs &a, hipStream_t st);

// Attention: the launch plan decides the split over the context and the workspace.
struct AttnPlan {
    int kind;           // 0: MFMA kernel, 1: generic kernel, 2: MFMA split by work
    uint32_t hc;        // head chunks of <= 8 query heads per KV head
    uint32_t n_chunks;  // context chunks per (item, kv head, head chunk); kind 2: workgroups
    uint32_t tpc;       // 16-position tiles per chunk
    uint64_t ws_bytes;  // workspace for partial results (0 when n_chunks == 1)
    uint32_t ucost;     // kind 2: a unit's set-up cost in tiles (its share of the split)
};
int plan_attention(const Geometry &g, uint32_t n_items, uint32_t heads, uint32_t max_pos,
                   AttnPlan *p, const char **why);
// Launch-shape knobs: process-wide values that pick kernel builds and launch shapes.  Each
// starts at its default (the measured best) and changes only through qvkv_tune(); the
// library reads no environment variable.  X(id, name, default).
#define QVKV_KNOBS(X)                                                                           \
    X(APPEND_U, "append_u", 2)                  /* rows per thread group: 2 (1, 2) or 4 */     \
    X(APPEND_GRID_PER_CU, "append_grid_per_cu", 1 << 20)                                        \
    X(APPEND_NT, "append_nt", -1)               /* non-temporal loads; -1: f16 yes, q8_0 no */   \
    X(APPEND_Q8_FAST, "append_q8_fast", 1)      /* k_append_q8 at d = 64/128/256 */             \
    X(APPEND_NTS, "append_nts", 1)              /* non-temporal q8_0 stores */                  \
    X(GATHER_SPLIT, "gather_split", 1)                                                          \
    X(GATHER_Q8_FAST, "gather_q8_fast", 1)                                                      \
    X(GATHER_T, "gather_t", 64)                                                                 \
    X(GATHER_UF, "gather_uf", 4)                                                                \
    X(COPY_U, "copy_u", 1)                                                                      \
    X(COPY_T, "copy_t", 64)                                                                     \
    X(ATTN_FULL, "attn_full", 512)              /* units from which a launch runs unsplit */    \
    X(ATTN_STREAM, "attn_stream", 1)            /* 1: split by work, 0: context chunks */       \
    X(ATTN_STREAM_WG, "attn_stream_wg", 768)                                                    \
    X(STREAM_UNIT_COST, "stream_unit_cost", 8)  /* a unit's set-up cost in tiles */             \
    X(ATTN_TARGET, "attn_target", 1536)         /* context-chunk split: workgroups aimed at */  \
    X(FUSED_Q8, "fused_q8", 1)                  /* fused append + attention for q8_0 */         \
    X(ATTN_WAVES4_F16, "attn_waves4_f16", 0)                                                    \
    X(ATTN_WAVES3_Q8, "attn_waves3_q8", 0)      /* q8_0 d = 128 at 3 waves/SIMD */              \
    X(ATTN_PACK, "attn_pack", 1)                                                                \
    X(ATTN_IDS_BELOW, "attn_ids_below", 2048)                                                   \
    X(ATTN_XCD, "attn_xcd", 1)                                                                  \
    X(PREFILL_V2, "prefill_v2", 1)                                                              \
    X(PREFILL_LDS_PAD, "prefill_lds_pad", 0)                                                    \
    X(PREFILL_EXACT_P, "prefill_exact_p", 0)                                                    \
    X(PREFILL_DMA, "prefill_dma", 1)                                                            \
    X(PREFILL_Q8_FAST, "prefill_q8_fast", 1)                                                    \
    X(PRELUDE_FAST, "prelude_fast", 1)                                                          \
    X(PRELUDE_WIDE, "prelude_wide", 1)                                                          \
    X(PRELUDE_FULL_WG, "prelude_full_wg", 1)
enum Knob : int {
#define QVKV_KNOB_ID(id, name, def) KNOB_##id,
    QVKV_KNOBS(QVKV_KNOB_ID)
#undef QVKV_KNOB_ID
    KNOB_COUNT
};
int tune(Knob k);                       // the knob's current value (kernels.hip)
int set_tune(const char *name, int v);  // QVKV_OK, or QVKV_E_SHAPE for an unknown name
int get_tune(const char *name, int *v);
void reset_tune();

// Paged prefill attention over segments of consecutive tokens (kernels.hip).
int check_prefill(const Geometry &g, uint32_t n_seg, uint32_t heads, uint32_t max_tok,
                  const char **why);
hipError_t launch_prefill(const Geometry &g, const void *pool, uint64_t pool_blocks,
                          const float *q, const uint32_t *blocks, uint64_t n_table,
                          const uint32_t *table_at, const uint32_t *pos0, const uint32_t *q_at,
                          const uint32_t *n_tok, uint32_t n_seg, uint32_t heads,
                          uint32_t max_pos, uint32_t max_tok, uint64_t q_rows, float *out,
                          int *err, hipStream_t s, bool f16_values = true);
// New key and value rows of a fused append + attention (n_items rows of kv_out floats
// each, stored at each item's position pos[i] and attended there); null in a plain
// attention launch.  The fused form runs at d = 64, 128, 256 for f16 pools, and for q8_0
// pools unless the knob fused_q8 is 0.
struct NewRows {
    const float *k = nullptr, *v = nullptr;
};
bool fused_append_attention(const Geometry &g);
hipError_t launch_attention(const Geometry &g, const AttnPlan &p, const void *pool,
                            uint64_t pool_blocks, const float *q, const uint32_t *blocks,
                            uint64_t n_table, const uint32_t *table_at, const uint32_t *pos,
                            uint32_t n_items, uint32_t heads, uint32_t max_pos, float *out,
                            void *ws, int *err, hipStream_t s, NewRows nr = NewRows{});
// Each item's pool slot of position pos[i] (block * B + offset), for the append of the
// unfused form; an item past max_pos or its table gets slot 0xffffffff (flagged).
hipError_t launch_slots_at(const Geometry &g, const uint32_t *blocks, uint64_t n_table,
                           const uint32_t *table_at, const uint32_t *pos, uint32_t n_items,
                           uint32_t max_pos, uint32_t *slots, int *err, hipStream_t s);

// Applies a device-tables sync (pool.cpp): pos[i] = staged[i] and lens[i] = staged[i] + 1
// for i < n_pos, then blocks[staged[n_pos + 2k]] = staged[n_pos + 2k + 1] for k < n_pairs.
hipError_t launch_table_scatter(const uint32_t *staged, uint32_t n_pos, uint64_t n_pairs,
                                uint32_t *pos, uint32_t *lens, uint32_t *blocks, hipStream_t s);

}  // namespace qvkv
