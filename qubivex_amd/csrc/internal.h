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
// (a hipStream_t; 0 is the null stream) when the call was made.
int block_copy_after(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                     const uint32_t *src, const uint32_t *dst, uint32_t n, bool ordered,
                     void *after);

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
// Launch-shape knob: the default, or an environment variable of the same name (kernels.hip).
int tune(const char *name, int def);

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
// attention launch.  The fused form runs for f16 pools at d = 64, 128, 256.
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

}  // namespace qvkv
