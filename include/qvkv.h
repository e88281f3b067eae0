/*
 * qvkv: the paged KV-cache hot path on one MI355X (gfx950), as a C ABI.
 *
 * This header is the drop-in boundary.  In the reference (kentmarete/qubivex, Rust) the
 * path sits behind `trait DiscreteDevice` (crates/qubivex-compute/src/discrete.rs:433-570),
 * which the runtime's `OnDevice` (crates/qubivex-runtime/src/discrete.rs) drives.  Each
 * entry point below names the trait method or reference function it replaces.
 *
 * Conventions
 *  - Every call returns a status: QVKV_OK or one of the QVKV_E_* codes, which mirror the
 *    `ComputeError` variants (crates/qubivex-compute/src/lib.rs:28-83).  The detail of
 *    the last failure on the calling thread is returned by qvkv_last_error().
 *  - Handles are opaque.  Host pointers are borrowed for the duration of the call.
 *  - Functions without the `_async` suffix take HOST memory, run on the device's own
 *    stream and complete before they return (the trait's "completes before return"
 *    semantics, crates/qubivex-backend-vulkan/src/lib.rs:212-225).  They do not wait for
 *    work a caller queued on other streams: finish it first (qvkv_check on that stream).
 *    The pool manager's copies are the exception: they take the caller's stream and run
 *    after the work queued there (qvkv_pool_plan_append).
 *  - `_async` functions take DEVICE pointers and enqueue on `stream`, a hipStream_t used
 *    as given (0 is HIP's null stream; qvkv_stream() returns the device's own).  Index
 *    errors found by a kernel (a block id past the pool, a table too short) are latched in
 *    a flag of that stream and reported by the next qvkv_check() of the same stream.
 *    Kernels never touch memory outside the pool for such input.
 *  - Threads: any thread may call (the trait is Send + Sync).  The library keeps an error
 *    flag and an attention workspace per stream, so callers on different streams never
 *    see each other's errors or overwrite each other's partial results.  The first launch
 *    on a stream sets its state up (a small device allocation), and an attention launch
 *    may grow the stream's workspace: before capturing a stream into a HIP graph, run the
 *    launches once uncaptured (or use qvkv_attention_noalloc_async).
 *  - A pool position is `slot = block * layout.block + offset` (the reference's
 *    `sync_to`, crates/qubivex-compute/src/discrete.rs:301-304).  Item t of a batch is
 *    one (sequence, layer) pair: its blocks are blocks[table_at[t] ..], in position order
 *    (crates/qubivex-compute/src/discrete.rs:257-266).
 */
#ifndef QVKV_H
#define QVKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: ComputeError (crates/qubivex-compute/src/lib.rs:28-83) ---- */
#define QVKV_OK 0
#define QVKV_E_SHAPE 1       /* ComputeError::Shape */
#define QVKV_E_UNSUPPORTED 2 /* ComputeError::Unsupported */
#define QVKV_E_OOM 3         /* ComputeError::OutOfDeviceMemory */
#define QVKV_E_DEVICE 4      /* ComputeError::Device */

/* ---- storage dtypes (crates/qubivex-core/src/dtype.rs:19-29: F32, F16, Q8_0) ---- */
#define QVKV_F32 0
#define QVKV_F16 1
#define QVKV_Q8_0 2

/* The pool's storage layout.  One block holds `block` positions of one layer: keys and
 * values of every KV head.  Replaces the reference's fixed KV_BLOCK = 256 f32 layout
 * (crates/qubivex-compute/src/discrete.rs:247-255).  block must be a multiple of 16;
 * head_dim a multiple of 8 (f16) or of 32 (q8_0). */
typedef struct qvkv_layout {
    uint32_t dtype;    /* QVKV_F16 or QVKV_Q8_0 */
    uint32_t kv_heads; /* G */
    uint32_t head_dim; /* d */
    uint32_t block;    /* B, positions per block */
} qvkv_layout;

typedef struct qvkv_dev qvkv_dev;
typedef struct qvkv_buf qvkv_buf;

/* Memory now: DiscreteDevice::usage (crates/qubivex-compute/src/discrete.rs:461). */
typedef struct qvkv_usage_t {
    uint64_t capacity, used, peak, refused;
} qvkv_usage_t;

/* Copies so far: TransferStats (crates/qubivex-compute/src/discrete.rs:376-427).
 *  uploads / upload_bytes: host-to-device copies (qvkv_write and the host-memory entry
 *    points' staged inputs); downloads / download_bytes: device-to-host copies;
 *  submissions: kernel launches made (every entry point);
 *  wait_ns / fence_waits: host time blocked waiting for the device, and the waits;
 *  timed / gpu_ns: the synchronous calls whose GPU time was measured, and that time summed;
 *  stream_waits: pool copies that waited for a caller's stream (no counterpart);
 *  activations_in / activations_out: bytes the host-memory entry points staged in and
 *    copied back;
 *  transfer_ns: GPU time of those calls' copies (events around them) plus the wall time of
 *    qvkv_write / qvkv_read;
 *  submit_ns: host time inside the library's calls, less their waits;
 *  gpu_busy_ns: union of the timed calls' GPU intervals; they run one at a time on the
 *    device's own stream, so it equals gpu_ns. */
typedef struct qvkv_transfers_t {
    uint64_t uploads, upload_bytes, downloads, download_bytes, submissions, wait_ns;
    uint64_t timed, gpu_ns, stream_waits;
    uint64_t activations_in, activations_out, transfer_ns, fence_waits, submit_ns, gpu_busy_ns;
} qvkv_transfers_t;

/* Detail of the calling thread's last failure (ComputeError's Display). Returns the
 * status of that failure. */
int qvkv_last_error(char *buf, size_t len);

/* ComputeError::OutOfDeviceMemory's fields (crates/qubivex-compute/src/lib.rs:64-75) for
 * the calling thread's last failure when it was QVKV_E_OOM: bytes requested, in use and
 * the capacity (for a dry KV pool: the pool's blocks, in bytes).  Zeros otherwise. */
int qvkv_last_oom(uint64_t *requested, uint64_t *used, uint64_t *capacity);

/* ---- device and memory ---- */

/* Opens HIP device `device` with its own stream (constructor of the backend;
 * DiscreteDevice::name/describe: crates/qubivex-compute/src/discrete.rs:437-441). */
int qvkv_open(int device, qvkv_dev **out);
/* Waits for the device and releases it.  Buffers still allocated on it stay valid to
 * free with qvkv_free (and pools to destroy) afterwards, in any order; the device's last
 * resources go with the last of them. */
void qvkv_close(qvkv_dev *dev);
int qvkv_describe(const qvkv_dev *dev, char *buf, size_t len);
/* DiscreteDevice::usage (discrete.rs:461) */
int qvkv_usage(const qvkv_dev *dev, qvkv_usage_t *out);
/* DiscreteDevice::transfers (discrete.rs:464) */
int qvkv_transfers(const qvkv_dev *dev, qvkv_transfers_t *out);
/* The device's own stream (a hipStream_t). */
void *qvkv_stream(const qvkv_dev *dev);
/* GPU time of the last synchronous (host-memory) call on this device, in nanoseconds,
 * from events around its kernels (TransferStats::gpu_ns per submission,
 * discrete.rs:398-402). */
int qvkv_timing(const qvkv_dev *dev, uint64_t *gpu_ns);
/* DiscreteDevice::max_arena (discrete.rs:525-529): the largest buffer one call can address
 * as a whole.  Kernels address pools with 64-bit offsets, so this is the device memory. */
int qvkv_max_arena(const qvkv_dev *dev, uint64_t *out);

/* Launch-shape knobs.  No counterpart in the reference (its backends have no launch
 * shapes to choose); for callers and benchmarks that measure alternative kernel builds and
 * splits.  Process-wide (every device), read by each launch; the library reads no
 * environment variable.  Every knob starts at its default, the measured best, and every
 * value a knob may take gives results within the path's tolerance (the attention
 * parity tests run each switch).  Names: append_u, append_grid_per_cu, append_nt,
 * append_q8_fast, append_nts, gather_split, gather_q8_fast, gather_t, gather_uf, copy_u,
 * copy_t, attn_full, attn_stream, attn_stream_wg, stream_unit_cost, attn_target, fused_q8,
 * attn_waves4_f16, attn_waves3_q8, attn_pack, attn_ids_below, attn_xcd, prefill_v2,
 * prefill_lds_pad, prefill_exact_p, prefill_dma, prefill_q8_fast, prelude_fast,
 * prelude_wide, prelude_full_wg.  An unknown name is QVKV_E_SHAPE. */
int qvkv_tune(const char *name, int value);
int qvkv_tune_get(const char *name, int *value);
/* Every knob back to its default. */
void qvkv_tune_reset(void);

/* DiscreteDevice::alloc (discrete.rs:500-508): `len` bytes, contents unspecified. */
int qvkv_alloc(qvkv_dev *dev, size_t len, qvkv_buf **out);
/* Drop of the last DeviceBuffer clone (discrete.rs:24-95). */
void qvkv_free(qvkv_buf *buf);
void *qvkv_buf_ptr(const qvkv_buf *buf);
size_t qvkv_buf_len(const qvkv_buf *buf);
/* DiscreteDevice::write (discrete.rs:510-523): host bytes into `buf` at `offset`. */
int qvkv_write(qvkv_dev *dev, qvkv_buf *buf, size_t offset, const void *host, size_t len);
/* Device bytes back to the host (the readback of k_new/v_new in the reference). */
int qvkv_read(qvkv_dev *dev, const qvkv_buf *buf, size_t offset, void *host, size_t len);
/* Waits for `stream` (as given: 0 is the null stream) and reports any index error its
 * kernels latched since the last check of that stream (QVKV_E_SHAPE), or the q8_0
 * prefill's range report alone (QVKV_E_UNSUPPORTED).  The flag is taken by an atomic
 * exchange on the device, ordered after the stream's kernels, so a bit latched meanwhile
 * is kept for the next check.  Other streams' flags are not read. */
int qvkv_check(qvkv_dev *dev, void *stream);

/* ---- layout ---- */

/* Bytes of one block: f16 2*B*G*d*2; q8_0 2*B*G*d*34/32.  Replaces kv_block_words
 * (crates/qubivex-compute/src/discrete.rs:254-256). */
int qvkv_block_bytes(const qvkv_layout *layout, uint64_t *out);

/* ---- the hot path, device pointers ---- */

/* Append: writes n rows (k[r], v[r]: G*d f32 each, [kv_head][d]) at pool positions
 * slots[r], narrowing to the storage dtype (f16 RNE; q8_0 quantize-on-write over each
 * head's 32-value groups).  Rows may belong to any sequence and layer.  Replaces the
 * pool store of SimDevice::attention (crates/qubivex-backend-cpu/src/sim.rs:377-399),
 * kv_sync.comp:40-50 and the store in attn_prelude.comp:166-173. */
int qvkv_append_async(qvkv_dev *dev, const qvkv_layout *layout, void *pool,
                      uint64_t pool_blocks, const float *k, const float *v,
                      const uint32_t *slots, uint32_t n, void *stream);

/* Gather: for each item t, positions 0..lens[t]-1 through its block table into
 * out_k/out_v at position offset out_at[t] (elements out_at[t]*G*d), head-major
 * [kv_head][lens[t]][d].  out_dtype QVKV_F16 (f16 pools only: a byte copy) or QVKV_F32
 * (the logical values: widened f16 or dequantized q8_0).  out_positions bounds
 * out_at[t] + lens[t].  Replaces the gather of SimDevice::attention (sim.rs:404-422)
 * and KvCache::heads (crates/qubivex-arch/src/lib.rs:519-525). */
int qvkv_gather_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                      uint64_t pool_blocks, const uint32_t *blocks, uint64_t n_table,
                      const uint32_t *table_at, const uint32_t *lens, const uint64_t *out_at,
                      uint32_t n_items, uint32_t max_len, uint32_t out_dtype,
                      uint64_t out_positions, void *out_k, void *out_v, void *stream);

/* Decode attention: for item t and query head h, softmax(q.K^T / sqrt(d)) V over
 * positions 0..pos[t] of KV head h / (heads/G), read through the block table.
 * q, out: [n_items][heads][d] f32.  max_pos bounds every pos[t] (it sizes the launch).
 * fp32 accumulation; within 2e-3 max-abs and 1e-3 rel-L2 of math::attend.  Replaces
 * the attention of SimDevice::attention (sim.rs:423-428 with math::attend,
 * crates/qubivex-compute/src/math.rs:142-155) and attn_decode.comp. */
int qvkv_attention_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                         uint64_t pool_blocks, const float *q, const uint32_t *blocks,
                         uint64_t n_table, const uint32_t *table_at, const uint32_t *pos,
                         uint32_t n_items, uint32_t heads, uint32_t max_pos, float *out,
                         void *stream);

/* Decode attention with the step's append: each item's new key and value rows k_new[t],
 * v_new[t] ([n_items][kv_out] f32, narrowed as qvkv_append_async narrows them) are stored
 * at position pos[t] of its table (the slot of that position, which the caller's
 * planning made writable), then attention runs over positions 0..pos[t] as in
 * qvkv_attention_async.  The reference's DeviceMoeAttention submission after its sync
 * rows: "the new token's key and value are stored at pos[t], and attention reads
 * positions 0..=pos[t]" (crates/qubivex-compute/src/discrete.rs:257-307).  f16 and q8_0
 * pools at d = 64, 128, 256 run it as one launch (the attention takes position pos[t] from
 * the new rows, narrowed or quantised as the append would store them, and stores them);
 * other layouts run the append and the attention in turn, on the stream.  The same results, bit for bit, as qvkv_append_async at those slots followed
 * by qvkv_attention_async. */
int qvkv_append_attention_async(qvkv_dev *dev, const qvkv_layout *layout, void *pool,
                                uint64_t pool_blocks, const float *q, const float *k_new,
                                const float *v_new, const uint32_t *blocks, uint64_t n_table,
                                const uint32_t *table_at, const uint32_t *pos, uint32_t n_items,
                                uint32_t heads, uint32_t max_pos, float *out, void *stream);

/* qvkv_attention_async without any allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results.  A launch that
 * splits the context keeps its partial results in a file-scope device array of
 * QVKV_NOALLOC_SCRATCH_BYTES (one per GPU, held until the process ends) instead of the
 * stream's workspace; a launch needing more returns QVKV_E_SHAPE before it starts.  Every
 * call on one GPU shares that array (the last call's contents stay in it): calls that
 * overlap on one GPU, on any streams or device handles, race.  Index errors its kernels
 * latch go to a device-wide flag in the same array, reported (and cleared) by the next
 * check on any stream of the device: a qvkv_check, or the host-memory entry points' own
 * check, which then returns QVKV_E_SHAPE for it. */
#define QVKV_NOALLOC_SCRATCH_BYTES (32ull << 20)
int qvkv_attention_noalloc_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                                 uint64_t pool_blocks, const float *q, const uint32_t *blocks,
                                 uint64_t n_table, const uint32_t *table_at, const uint32_t *pos,
                                 uint32_t n_items, uint32_t heads, uint32_t max_pos, float *out,
                                 void *stream);

/* Paged prefill attention: segment i holds n_tok[i] consecutive tokens of one sequence
 * whose rows are already stored; token j of it sits at position pos0[i] + j and reads
 * q row q_at[i] + j ([q_rows][heads][d] f32) and writes the same out row.  It attends
 * (causally) over positions 0..pos0[i]+j of its table exactly as qvkv_attention_async
 * would for an item with pos = pos0[i]+j; max_pos bounds pos0[i]+n_tok[i]-1 and max_tok
 * bounds n_tok[i].  Replaces the host prefill of the reference's forward pass, which
 * stores a segment's rows and then runs math::attend per (token, head)
 * (crates/qubivex-arch/src/lib.rs:1296-1320); the reference has no device prefill.
 * q8_0 pools at d = 128 use a form that holds dequantised values in f16: a value scale
 * above 512 (values that may pass 65504) makes the next qvkv_check return
 * QVKV_E_UNSUPPORTED.  The synchronous entry points (qvkv_decode_attention,
 * qvkv_prelude_attention) then recompute the chunk with the f32-scale form.
 * Non-finite stored values: a NaN or infinity at one of a segment's own positions reaches
 * the segment's earlier tokens as NaN, and in f16 pools at d = 64 or 128 an infinity can
 * give NaN where the CPU path gives an infinity; finite values are unaffected. */
int qvkv_prefill_attention_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                                 uint64_t pool_blocks, const float *q, uint64_t q_rows,
                                 const uint32_t *blocks, uint64_t n_table,
                                 const uint32_t *table_at, const uint32_t *pos0,
                                 const uint32_t *q_at, const uint32_t *n_tok, uint32_t n_seg,
                                 uint32_t heads, uint32_t max_pos, uint32_t max_tok, float *out,
                                 void *stream);

/* Block copy: block src[i] -> block dst[i], i < n, byte for byte (copy-on-write of a
 * shared block; compaction moves).  No dst may appear twice or also be a src in the
 * same call.  No reference counterpart: the reference copies a whole prefix instead
 * (KvCache::restore_from, crates/qubivex-arch/src/lib.rs:409-432). */
int qvkv_block_copy_async(qvkv_dev *dev, const qvkv_layout *layout, void *pool,
                          uint64_t pool_blocks, const uint32_t *src, const uint32_t *dst,
                          uint32_t n, void *stream);

/* ---- the hot path, host memory (synchronous; what the Rust backend binds) ---- */

/* qvkv_append_async with host rows and slots. */
int qvkv_append(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool, const float *k,
                const float *v, const uint32_t *slots, uint32_t n);

/* qvkv_gather_async with host tables and host outputs. */
int qvkv_gather(qvkv_dev *dev, const qvkv_layout *layout, const qvkv_buf *pool,
                const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                const uint32_t *lens, const uint64_t *out_at, uint32_t n_items,
                uint32_t out_dtype, uint64_t out_positions, void *out_k, void *out_v);

/* qvkv_block_copy_async with host id lists. */
int qvkv_block_copy(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                    const uint32_t *src, const uint32_t *dst, uint32_t n);

/* The KV part of one DeviceMoeAttention submission
 * (crates/qubivex-compute/src/discrete.rs:257-307; SimDevice::attention, sim.rs:301-436):
 * first the n_sync host rows (`sync`: n_sync * 2*G*d f32, key row then value row) to
 * `sync_to`, then token t's k_new/v_new row at its own position pos[t], then attention
 * of q over positions 0..=pos[t].  q, out: [s][heads][d]; k_new, v_new: [s][G*d].
 * blocks/table_at/pos as AttnPlan (crates/qubivex-runtime/src/discrete.rs:284-290).
 * Runs of consecutive tokens with one table_at and consecutive positions (a prefill
 * chunk) go through the prefill kernel of qvkv_prefill_attention_async; the results are
 * those of attending each token on its own. */
int qvkv_decode_attention(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                          const float *q, uint32_t heads, const uint32_t *pos, uint32_t s,
                          const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                          const float *sync, const uint32_t *sync_to, uint32_t n_sync,
                          const float *k_new, const float *v_new, float *out);

/* ---- the attention prelude feeding the append ----
 *
 * Bias, clip, Q/K RMSNorm and RoPE on the projection outputs, in place, bit for bit as
 * the reference's forward pass (crates/qubivex-arch/src/lib.rs:1258-1292 with
 * math::rms_norm, math::rope_rotate and the 64-lane reduce::dot shape; the device form
 * is attn_prelude.comp).  Per-head norms (Qwen3) are supported, which the reference's
 * device path declines. */

#define QVKV_NORM_NONE 0
#define QVKV_NORM_FULL 1     /* QkNorm::Full: one norm over each token's q (or k) row */
#define QVKV_NORM_PER_HEAD 2 /* QkNorm::PerHead: one norm per head, weights of d */

typedef struct qvkv_prelude_t {
    uint32_t heads;    /* query heads (KV heads and d come from the layout) */
    uint32_t norm;     /* QVKV_NORM_* */
    uint32_t has_clip; /* clamp q, k, v to [-clip, clip] after the bias */
    float clip;
    float eps;         /* the norms' epsilon, as f32 (rms_scale casts it) */
    const float *q_bias, *k_bias, *v_bias; /* q_out / kv_out values each, or NULL */
    const float *q_norm, *k_norm; /* q_out / kv_out (full) or d (per head) weights */
    const float *rope; /* [s][d] per token: cos of the d/2 pairs, then sin (Rope::table) */
} qvkv_prelude_t;

/* The prelude on device arrays (q [s][heads*d], k and v [s][G*d], all in place; the
 * pointers inside *p are device pointers). */
int qvkv_prelude_async(qvkv_dev *dev, const qvkv_layout *layout, const qvkv_prelude_t *p,
                       float *q, float *k, float *v, uint32_t s, void *stream);

/* The KV part of one DeviceMoeAttention submission from the projection outputs (the
 * device side of SimDevice::attention, crates/qubivex-backend-cpu/src/sim.rs:310-436,
 * without the matmuls): the prelude on q/k/v, the sync rows, then token t's k/v row at
 * pos[t], then attention.  Host memory; *p's pointers are host pointers.  k_new and
 * v_new receive the post-prelude rows for the host cache (discrete.rs:302-306). */
int qvkv_prelude_attention(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                           const qvkv_prelude_t *p, const float *q, const float *k,
                           const float *v, const uint32_t *pos, uint32_t s,
                           const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                           const float *sync, const uint32_t *sync_to, uint32_t n_sync,
                           float *out, float *k_new, float *v_new);

/* ---- host pool manager: block pool, block tables, sharing, eviction, compaction ----
 *
 * The host side of the path, above the kernels: the reference's KvPool / KvFree /
 * Mirror / attention_plan (crates/qubivex-runtime/src/discrete.rs:209-290,951-1009),
 * generalised with per-block reference counts (prefix sharing with copy-on-write),
 * last-use ticks (LRU eviction) and compaction.  A pool owns one device allocation of
 * n_blocks blocks.  Sequences are small integer handles; each holds, per layer, a block
 * table and the number of positions written.  Not thread-safe per pool: the caller
 * serialises calls on one pool (the reference holds its free-list mutex likewise). */

typedef struct qvkv_pool qvkv_pool;

/* Counters: KvPoolStats (crates/qubivex-runtime/src/discrete.rs:92-108) plus the
 * sharing and compaction counters this path adds.  allocated: 1 when the pool holds device
 * memory (a device pool allocates it whole at qvkv_pool_create), 0 for a host-only pool. */
typedef struct qvkv_pool_stats_t {
    uint64_t bytes, blocks, free, layers, synced_rows, full;
    uint64_t shared_blocks, cow_copies, evicted_blocks, moved_blocks;
    uint64_t allocated;
} qvkv_pool_stats_t;

/* A pool of n_blocks blocks (OnDevice::new pool sizing, discrete.rs:429-455; the free
 * list starts (0..n).rev() so the first pop is block 0, :448).  Allocates the device
 * memory now.  dev == NULL makes a host-only pool: the same bookkeeping with no device
 * memory, whose block copies are recorded for qvkv_pool_take_copies instead of run
 * (a planner, and the CPU-side test double of the runtime's SimDevice). */
int qvkv_pool_create(qvkv_dev *dev, const qvkv_layout *layout, uint64_t n_blocks,
                     uint32_t n_layers, qvkv_pool **out);
/* Host-only pools: the block copies (src, dst) issued since the last call, in issue
 * order; the pair (UINT32_MAX, UINT32_MAX) ends each batch (one kernel launch, whose
 * pairs are independent).  *n receives the count pending; at most cap pairs are
 * returned and removed. */
int qvkv_pool_take_copies(qvkv_pool *pool, uint32_t *src, uint32_t *dst, uint64_t cap,
                          uint64_t *n);
void qvkv_pool_destroy(qvkv_pool *pool);
void *qvkv_pool_ptr(const qvkv_pool *pool);
/* The pool's device memory as a buffer for the host-memory entry points (owned by the
 * pool; NULL for a host-only pool).  The runtime's kv_buffer (discrete.rs:502-512). */
qvkv_buf *qvkv_pool_buffer(const qvkv_pool *pool);
int qvkv_pool_stats(const qvkv_pool *pool, qvkv_pool_stats_t *out);

/* A new empty sequence (a KvCache's mirror, discrete.rs:247-280). */
int qvkv_seq_create(qvkv_pool *pool, uint32_t *seq);
/* Gives every block of `seq` back (Mirror::release / Drop, discrete.rs:267-280). */
int qvkv_seq_release(qvkv_pool *pool, uint32_t seq);
/* A new sequence sharing the first `positions` positions of `parent` on every layer:
 * the blocks holding them gain a reference (no copy).  A later write into a shared
 * block copies it first.  Replaces KvCache::restore_from's copy
 * (crates/qubivex-arch/src/lib.rs:409-432) as ADR-016 describes. */
int qvkv_seq_fork(qvkv_pool *pool, uint32_t parent, uint32_t positions, uint32_t *child);
/* Positions held by `seq` on `layer`. */
int qvkv_seq_len(const qvkv_pool *pool, uint32_t seq, uint32_t layer, uint32_t *out);
/* Marks the sequence used now (LRU clock; PrefixCache `used`,
 * crates/qubivex-kv-cache/src/lib.rs:30-31). */
int qvkv_seq_touch(qvkv_pool *pool, uint32_t seq);

/* Plans writes of `count[i]` new positions for seqs[i] on `layer` (the positions
 * len..len+count-1): grows each table from the free list, and copies-on-write a shared
 * block that a write lands in.  slots_out receives sum(count) pool positions, seq-major.
 * Returns QVKV_E_OOM with nothing changed (`pool.full` counts it; discrete.rs:882-891)
 * when the free list runs dry.  attention_plan's growth step (discrete.rs:988-994).
 *
 * Ordering of the copies (here, in qvkv_pool_plan_attention and in qvkv_pool_compact):
 * a copy runs after all work queued on `stream` (a hipStream_t, 0 the null stream) when
 * the call is made, and has completed when the call returns.  So appends that filled the
 * shared blocks must have been queued on `stream`, or finished, before the call; the
 * caller's writes into the copies may then go on any stream.  Host-only pools ignore
 * `stream`. */
int qvkv_pool_plan_append(qvkv_pool *pool, const uint32_t *seqs, const uint32_t *count,
                          uint32_t n_seqs, uint32_t layer, uint32_t *slots_out, void *stream);
/* qvkv_pool_plan_append on layers layer0 .. layer0+n_layers-1 at once (a decode step's or
 * a prompt chunk's rows of every layer): slots_out is layer-major, then seq-major.  A dry
 * free list fails the whole call with nothing changed; every layer's copy-on-write pairs
 * go to the device in one block-copy launch. */
int qvkv_pool_plan_append_layers(qvkv_pool *pool, const uint32_t *seqs, const uint32_t *count,
                                 uint32_t n_seqs, uint32_t layer0, uint32_t n_layers,
                                 uint32_t *slots_out, void *stream);
/* The attention plan of one decode pass on `layer` with a host-authoritative cache:
 * attention_plan (crates/qubivex-runtime/src/discrete.rs:951-1009).  For each seqs[i] with
 * the host's newest position pos[i] and cache epoch epochs[i]: a sequence whose epoch
 * changed gives its blocks back and starts again; positions past the host's count are
 * written again (synced = min(synced, pos)); the table grows to pos/B + 1 blocks from the
 * free list (copy-on-write of a shared block a write lands in); the host rows
 * [synced, pos) are listed to copy in (sync_to = their slots, sync_item / sync_pos = which
 * sequence and position each is); new_slot[i] is position pos[i]'s slot.  Outputs are
 * AttnPlan's blocks / table_at / pos (pos is the input).  The plan marks the layer synced
 * to pos+1 (a failed pass is repaired by the min above on the next plan).  A dry free list
 * returns QVKV_E_OOM and counts `full`; blocks taken before it stay with their sequence, as
 * in the reference.  blocks_cap / sync_cap bound the outputs.  Copies are ordered after
 * `stream` as in qvkv_pool_plan_append. */
int qvkv_pool_plan_attention(qvkv_pool *pool, const uint32_t *seqs, const uint32_t *pos,
                             const uint64_t *epochs, uint32_t n_seqs, uint32_t layer,
                             uint32_t *blocks_out, uint64_t blocks_cap, uint64_t *n_table_out,
                             uint32_t *table_at_out, uint32_t *new_slot_out,
                             uint32_t *sync_to_out, uint32_t *sync_item_out,
                             uint32_t *sync_pos_out, uint64_t sync_cap, uint64_t *n_sync_out,
                             void *stream);

/* Flattened block tables of seqs[i] on `layer` (AttnPlan.blocks/table_at/pos,
 * discrete.rs:995-997).  blocks_cap bounds blocks_out; *n_table_out receives the
 * entries written; pos_out[i] = len-1 (the newest position). */
int qvkv_pool_tables(const qvkv_pool *pool, const uint32_t *seqs, uint32_t n_seqs,
                     uint32_t layer, uint32_t *blocks_out, uint64_t blocks_cap,
                     uint64_t *n_table_out, uint32_t *table_at_out, uint32_t *pos_out);
/* qvkv_pool_tables for layers layer0 .. layer0+n_layers-1 in one call: item
 * (l - layer0) * n_seqs + i is seqs[i] on layer l (the attention_plan of every layer of a
 * decode step, discrete.rs:951-1009, as one batch). */
int qvkv_pool_tables_layers(const qvkv_pool *pool, const uint32_t *seqs, uint32_t n_seqs,
                            uint32_t layer0, uint32_t n_layers, uint32_t *blocks_out,
                            uint64_t blocks_cap, uint64_t *n_table_out, uint32_t *table_at_out,
                            uint32_t *pos_out);

/* Device-resident block tables of a fixed batch (no reference counterpart: the reference
 * rebuilds and uploads its tables every submission, discrete.rs:951-1009).  Items are
 * (sequence, layer) pairs as in qvkv_pool_tables_layers; item t's table sits at
 * t * max_blocks of the device `blocks` array (table_at is fixed).  qvkv_tables_sync
 * brings the device copy up to the pool: only the ids added since the last sync travel (a
 * table changed in place -- copy-on-write, compaction, release, an epoch restart -- goes
 * whole), with every item's pos, as one copy and one small kernel on `stream`.  The
 * device arrays are valid for launches queued on `stream` after the sync.  Not
 * thread-safe per object; the pool's own calls may run between syncs. */
typedef struct qvkv_tables qvkv_tables;
int qvkv_tables_create(qvkv_pool *pool, const uint32_t *seqs, uint32_t n_seqs, uint32_t layer0,
                       uint32_t n_layers, uint32_t max_blocks, qvkv_tables **out);
/* *max_pos_out (may be NULL) receives the largest pos: the launches' max_pos. */
int qvkv_tables_sync(qvkv_tables *tables, void *stream, uint32_t *max_pos_out);
/* The device arrays: blocks [n_items * max_blocks] (*n_table), table_at, pos and lens
 * (= pos + 1, the gather's lengths) [n_items]; n_items = n_seqs * n_layers. */
int qvkv_tables_device(const qvkv_tables *tables, const uint32_t **blocks, uint64_t *n_table,
                       const uint32_t **table_at, const uint32_t **pos, const uint32_t **lens,
                       uint32_t *n_items);
void qvkv_tables_destroy(qvkv_tables *tables);
/* Releases least-recently-used sequences (PrefixCache::evict_oldest,
 * crates/qubivex-kv-cache/src/lib.rs:197-213; ties: the lower handle) until at least
 * `target_blocks` blocks have returned to the free list or none is left; writes the
 * released handles to released_out (cap entries) and their count. */
int qvkv_pool_evict_lru(qvkv_pool *pool, uint64_t target_blocks, uint32_t *released_out,
                        uint32_t cap, uint32_t *n_released);
/* Compaction modes. */
#define QVKV_COMPACT_PERMUTE 0 /* every live block to the position a seeded permutation of
                                  0..live-1 gives it (seed 0: ascending by current id) */
#define QVKV_COMPACT_FILL 1    /* live blocks below `live` stay; those above move into the
                                  vacant ids below `live`, matched in a seeded order: the
                                  fewest moves, all in one batch */
/* Moves every live block into the ids 0..live-1 under a remap drawn from `seed` (`mode`:
 * QVKV_COMPACT_*), rewriting every table and the free list, with cycle-safe batches of
 * the block-copy kernel, ordered after `stream` as in qvkv_pool_plan_append.  *moved
 * receives the blocks moved. */
int qvkv_pool_compact(qvkv_pool *pool, uint32_t mode, uint64_t seed, uint64_t *moved,
                      void *stream);
/* Reference count of one block (0 = free). */
int qvkv_pool_refcount(const qvkv_pool *pool, uint32_t block, uint32_t *out);

/* ---- prefix-cache index ----
 *
 * The reference's PrefixCache (crates/qubivex-kv-cache/src/lib.rs:21-223) with its rules
 * unchanged (MIN_REUSE = 32, longest prefix per scope, last token never reused, LRU,
 * covering inserts).  A value is an opaque 64-bit handle, normally a pool sequence: a
 * hit is taken with qvkv_seq_fork(value, reuse), which shares blocks instead of copying
 * (KvCache::restore_from, crates/qubivex-arch/src/lib.rs:409-432).  Values that leave
 * the index are queued for qvkv_prefix_take_dropped (the caller releases them). */

typedef struct qvkv_prefix qvkv_prefix;

/* PrefixStats (crates/qubivex-kv-cache/src/lib.rs:44-62). */
typedef struct qvkv_prefix_stats_t {
    uint64_t lookups, hits, tokens_reused, inserted, evicted, entries, cost;
} qvkv_prefix_stats_t;

/* PrefixCache::new (lib.rs:77-92). */
int qvkv_prefix_create(uint64_t budget, qvkv_prefix **out);
void qvkv_prefix_destroy(qvkv_prefix *pc);
/* PrefixCache::lookup (lib.rs:130-157).  scope NULL is the unscoped space.  On a hit
 * *reuse > 0 and *value is the entry's value; *reuse == 0 means no hit. */
int qvkv_prefix_lookup(qvkv_prefix *pc, const char *scope, const uint32_t *prompt, uint32_t n,
                       uint64_t *value, uint32_t *reuse);
/* PrefixCache::insert (lib.rs:159-195); *kept as its bool. */
int qvkv_prefix_insert(qvkv_prefix *pc, const char *scope, const uint32_t *tokens, uint32_t n,
                       uint64_t cost, uint64_t value, int *kept);
/* PrefixCache::evict_oldest (lib.rs:197-213); *evicted as its bool. */
int qvkv_prefix_evict_oldest(qvkv_prefix *pc, int *evicted);
/* PrefixCache::clear (lib.rs:215-219). */
int qvkv_prefix_clear(qvkv_prefix *pc);
/* PrefixCache::stats (lib.rs:112-116). */
int qvkv_prefix_stats(qvkv_prefix *pc, qvkv_prefix_stats_t *out);
/* Values that left the index (evicted, replaced or cleared) since the last call; *n
 * receives the count pending, at most cap are returned and removed. */
int qvkv_prefix_take_dropped(qvkv_prefix *pc, uint64_t *values, uint64_t cap, uint64_t *n);

#ifdef __cplusplus
}
#endif

#endif /* QVKV_H */
