// Host pool manager: the block pool, per-sequence per-layer block tables, prefix
// sharing with copy-on-write, LRU eviction and compaction (include/qvkv.h, qvkv_pool_*).
//
// Reference behaviour restated here (kentmarete/qubivex):
//  - the free list is a LIFO of block ids that starts as (0..n).rev(), so the first
//    pop is block 0 (crates/qubivex-runtime/src/discrete.rs:215-225, 446-449);
//  - a sequence's table grows, layer by layer, to pos/B + 1 blocks by popping the free
//    list; a dry free list declines the whole layer (`full`)
//    (crates/qubivex-runtime/src/discrete.rs:988-994, 882-891);
//  - releasing a sequence gives every block back (Mirror::release,
//    crates/qubivex-runtime/src/discrete.rs:267-280);
//  - eviction takes the least recently used first (PrefixCache::evict_oldest,
//    crates/qubivex-kv-cache/src/lib.rs:197-213).
// Added for paged sharing (ADR-016's "Paged KV later",
// docs/decisions/ADR-016-KV-SUBSYSTEM.md:82-89): per-block reference counts, fork
// (a prefix hit becomes shared blocks instead of restore_from's copy), copy-on-write of
// a shared partially filled block before a write lands in it, and compaction of live
// blocks to the front of the pool in cycle-safe batches of the block-copy kernel.
#include <algorithm>
#include <mutex>
#include <numeric>
#include <unordered_map>
#include <vector>

#include "internal.h"
#include "qvkv.h"

struct Seq {
    bool live = false;
    uint64_t used = 0;
    uint64_t epoch = 0;                         // host cache epoch the tables belong to
    std::vector<std::vector<uint32_t>> blocks;  // per layer, in position order
    std::vector<uint32_t> len;                  // per layer, positions written
};

struct qvkv_pool {
    qvkv_dev *dev = nullptr;
    qvkv_layout layout{};
    qvkv::Geometry g{};
    uint64_t n_blocks = 0;
    uint32_t n_layers = 0;
    qvkv_buf *buf = nullptr;
    std::vector<uint32_t> free;  // LIFO: back() is the next block handed out
    std::vector<uint32_t> refs;  // per block; 0 = free
    std::vector<Seq> seqs;
    std::vector<uint32_t> free_handles;
    std::vector<uint32_t> log_src, log_dst;  // host-only pools: copies issued, in order
    std::vector<uint32_t> fill_holes, fill_movers, fill_map;  // compaction scratch, kept
    uint64_t clock = 0;
    uint64_t layers = 0, rows = 0, full = 0, cow = 0, evicted = 0, moved = 0;
    // Bumped by every change to a table other than ids appended at its end (copy-on-write,
    // release, a new or reused handle, an epoch restart, compaction): device-resident
    // tables re-send whole tables when it moved (qvkv_tables_sync).
    uint64_t tab_gen = 0;
    mutable std::mutex mu;
};

namespace {

int err(int code, const char *msg) { return qvkv::set_error(code, "%s", msg); }

// A dry free list: QVKV_E_OOM with the blocks asked for, in use and held, in bytes.
int dry(qvkv_pool *p, uint64_t need) {
    p->full++;
    const uint64_t bb = p->g.block_bytes;
    err(QVKV_E_OOM, "hip device is out of memory: the KV pool has no free block");
    qvkv::set_oom(need * bb, (p->n_blocks - p->free.size()) * bb, p->n_blocks * bb);
    return QVKV_E_OOM;
}

Seq *seq_of(qvkv_pool *p, uint32_t s) {
    return (s < p->seqs.size() && p->seqs[s].live) ? &p->seqs[s] : nullptr;
}
const Seq *seq_of(const qvkv_pool *p, uint32_t s) {
    return (s < p->seqs.size() && p->seqs[s].live) ? &p->seqs[s] : nullptr;
}

uint32_t new_handle(qvkv_pool *p) {
    uint32_t h;
    if (!p->free_handles.empty()) {
        h = p->free_handles.back();
        p->free_handles.pop_back();
    } else {
        h = (uint32_t)p->seqs.size();
        p->seqs.emplace_back();
    }
    Seq &s = p->seqs[h];
    p->tab_gen++;
    s.live = true;
    s.used = ++p->clock;
    s.blocks.assign(p->n_layers, {});
    s.len.assign(p->n_layers, 0);
    return h;
}

void unref(qvkv_pool *p, uint32_t b, uint64_t *returned) {
    if (--p->refs[b] == 0) {
        p->free.push_back(b);
        if (returned) ++*returned;
    }
}

uint64_t release(qvkv_pool *p, uint32_t h) {
    Seq &s = p->seqs[h];
    p->tab_gen++;
    uint64_t returned = 0;
    for (auto &l : s.blocks) {
        for (uint32_t b : l) unref(p, b, &returned);
        l.clear();
    }
    s.live = false;
    s.len.clear();
    p->free_handles.push_back(h);
    return returned;
}

// Copies block pairs on the device, in one launch, after the work already queued on the
// caller's `stream` (which wrote the source rows), before returning.
// `overlap(ctx)`, when given, runs while the device copies (host-only pools: after the
// batch is logged).
int copy_blocks(qvkv_pool *p, const std::vector<uint32_t> &src, const std::vector<uint32_t> &dst,
                void *stream, void (*overlap)(void *) = nullptr, void *ctx = nullptr) {
    if (src.empty()) return QVKV_OK;
    if (!p->dev) {
        p->log_src.insert(p->log_src.end(), src.begin(), src.end());
        p->log_dst.insert(p->log_dst.end(), dst.begin(), dst.end());
        p->log_src.push_back(UINT32_MAX);  // end of one batch (one kernel launch)
        p->log_dst.push_back(UINT32_MAX);
        if (overlap) overlap(ctx);
        return QVKV_OK;
    }
    return qvkv::block_copy_after(p->dev, &p->layout, p->buf, src.data(), dst.data(),
                                  (uint32_t)src.size(), true, stream, overlap, ctx);
}

uint64_t splitmix(uint64_t &x) {
    uint64_t z = (x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

}  // namespace

extern "C" {

int qvkv_pool_create(qvkv_dev *dev, const qvkv_layout *layout, uint64_t n_blocks,
                     uint32_t n_layers, qvkv_pool **out) {
    if (!layout || !out) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    qvkv::Geometry g;
    const char *why = "";
    if (int rc = qvkv::make_geometry(layout, &g, &why)) return err(rc, why);
    if (n_blocks == 0 || n_blocks > 0xffffffffull || n_layers == 0)
        return err(QVKV_E_SHAPE, "shape mismatch in pool: block count must be in 1..2^32-1, layers >= 1");
    if (n_blocks * g.block_bytes / g.block_bytes != n_blocks)
        return err(QVKV_E_SHAPE, "shape mismatch in pool: size overflows");
    auto *p = new qvkv_pool();
    p->dev = dev;
    p->layout = *layout;
    p->g = g;
    p->n_blocks = n_blocks;
    p->n_layers = n_layers;
    if (dev) {
        if (int rc = qvkv_alloc(dev, n_blocks * g.block_bytes, &p->buf)) {
            delete p;
            return rc;
        }
    }
    p->refs.assign(n_blocks, 0);
    p->free.resize(n_blocks);
    for (uint64_t i = 0; i < n_blocks; i++) p->free[i] = (uint32_t)(n_blocks - 1 - i);
    // compaction's scratch (12 bytes a block), written once here so that a compaction
    // touches no fresh pages (their first-touch faults had cost more than its scans)
    p->fill_holes.assign(n_blocks + 1, 0);
    p->fill_movers.assign(n_blocks + 1, 0);
    p->fill_map.assign(n_blocks, 0);
    *out = p;
    return QVKV_OK;
}

void qvkv_pool_destroy(qvkv_pool *pool) {
    if (!pool) return;
    if (pool->buf) qvkv_free(pool->buf);
    delete pool;
}

int qvkv_pool_take_copies(qvkv_pool *p, uint32_t *src, uint32_t *dst, uint64_t cap, uint64_t *n) {
    if (!p || !n || (cap && (!src || !dst))) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    const uint64_t have = p->log_src.size();
    *n = have;
    const uint64_t take = std::min<uint64_t>(cap, have);
    std::copy(p->log_src.begin(), p->log_src.begin() + take, src);
    std::copy(p->log_dst.begin(), p->log_dst.begin() + take, dst);
    p->log_src.erase(p->log_src.begin(), p->log_src.begin() + take);
    p->log_dst.erase(p->log_dst.begin(), p->log_dst.begin() + take);
    return QVKV_OK;
}

void *qvkv_pool_ptr(const qvkv_pool *pool) { return pool && pool->buf ? qvkv_buf_ptr(pool->buf) : nullptr; }

qvkv_buf *qvkv_pool_buffer(const qvkv_pool *pool) { return pool ? pool->buf : nullptr; }

int qvkv_pool_stats(const qvkv_pool *p, qvkv_pool_stats_t *out) {
    if (!p || !out) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    out->bytes = p->n_blocks * p->g.block_bytes;
    out->blocks = p->n_blocks;
    out->free = p->free.size();
    out->layers = p->layers;
    out->synced_rows = p->rows;
    out->full = p->full;
    out->shared_blocks = (uint64_t)std::count_if(p->refs.begin(), p->refs.end(),
                                                 [](uint32_t r) { return r > 1; });
    out->cow_copies = p->cow;
    out->evicted_blocks = p->evicted;
    out->moved_blocks = p->moved;
    out->allocated = p->buf != nullptr;
    return QVKV_OK;
}

int qvkv_seq_create(qvkv_pool *p, uint32_t *seq) {
    if (!p || !seq) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    *seq = new_handle(p);
    return QVKV_OK;
}

int qvkv_seq_release(qvkv_pool *p, uint32_t seq) {
    if (!p) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    if (!seq_of(p, seq)) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence");
    release(p, seq);
    return QVKV_OK;
}

int qvkv_seq_fork(qvkv_pool *p, uint32_t parent, uint32_t positions, uint32_t *child) {
    if (!p || !child) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    const Seq *ps = seq_of(p, parent);
    if (!ps) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence");
    for (uint32_t l = 0; l < p->n_layers; l++)
        if (ps->len[l] < positions)
            return err(QVKV_E_SHAPE, "shape mismatch in pool: the parent holds fewer positions");
    const uint32_t h = new_handle(p);  // may reallocate seqs: re-take the parent
    Seq &c = p->seqs[h];
    const Seq &pp = p->seqs[parent];
    const uint32_t B = p->layout.block;
    const uint32_t nb = (positions + B - 1) / B;
    for (uint32_t l = 0; l < p->n_layers; l++) {
        c.blocks[l].assign(pp.blocks[l].begin(), pp.blocks[l].begin() + nb);
        for (uint32_t b : c.blocks[l]) p->refs[b]++;
        c.len[l] = positions;
    }
    *child = h;
    return QVKV_OK;
}

int qvkv_seq_len(const qvkv_pool *p, uint32_t seq, uint32_t layer, uint32_t *out) {
    if (!p || !out) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    const Seq *s = seq_of(p, seq);
    if (!s || layer >= p->n_layers) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence or layer");
    *out = s->len[layer];
    return QVKV_OK;
}

int qvkv_seq_touch(qvkv_pool *p, uint32_t seq) {
    if (!p) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    Seq *s = seq_of(p, seq);
    if (!s) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence");
    s->used = ++p->clock;
    return QVKV_OK;
}

int qvkv_pool_plan_append_layers(qvkv_pool *p, const uint32_t *seqs, const uint32_t *count,
                                 uint32_t n_seqs, uint32_t layer0, uint32_t n_layers,
                                 uint32_t *slots_out, void *stream) {
    if (!p || (n_seqs && n_layers && (!seqs || !count || !slots_out)))
        return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    if (layer0 >= p->n_layers || n_layers > p->n_layers - layer0)
        return err(QVKV_E_SHAPE, "shape mismatch in pool: no such layer");
    const uint32_t B = p->layout.block;
    // Dry run over every layer: blocks this call takes (growth + copies of shared partial
    // blocks), with the reference counts as they will be when each sequence's turn comes.
    // A block belongs to one layer's tables, so one count of drops serves all layers.
    std::unordered_map<uint32_t, uint32_t> drops;
    uint64_t need = 0;
    for (uint32_t i = 0; i < n_seqs; i++) {
        if (!seq_of(p, seqs[i])) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence");
        for (uint32_t j = 0; j < i; j++)
            if (seqs[j] == seqs[i]) return err(QVKV_E_SHAPE, "shape mismatch in pool: a sequence twice in one plan");
    }
    for (uint32_t layer = layer0; layer < layer0 + n_layers; layer++)
        for (uint32_t i = 0; i < n_seqs; i++) {
            const Seq *s = seq_of(p, seqs[i]);
            const uint64_t len = s->len[layer];
            if (len + count[i] > 0xffffffffull) return err(QVKV_E_SHAPE, "shape mismatch in pool: too many positions");
            const uint64_t want = (len + count[i] + B - 1) / B;
            if (want > s->blocks[layer].size()) need += want - s->blocks[layer].size();
            if (count[i] && len % B != 0) {
                const uint32_t b = s->blocks[layer][len / B];
                const uint32_t live = p->refs[b] - drops[b];
                if (live > 1) {
                    need++;
                    drops[b]++;
                }
            }
        }
    if (need > p->free.size()) return dry(p, need);
    std::vector<uint32_t> src, dst;
    uint64_t o = 0;
    for (uint32_t layer = layer0; layer < layer0 + n_layers; layer++) {
        for (uint32_t i = 0; i < n_seqs; i++) {
            Seq &s = p->seqs[seqs[i]];
            auto &tab = s.blocks[layer];
            const uint32_t len = s.len[layer];
            if (count[i] && len % B != 0 && p->refs[tab[len / B]] > 1) {
                const uint32_t old = tab[len / B];
                const uint32_t nb = p->free.back();
                p->free.pop_back();
                p->refs[nb] = 1;
                p->refs[old]--;
                tab[len / B] = nb;
                p->tab_gen++;
                src.push_back(old);
                dst.push_back(nb);
                p->cow++;
            }
            const uint64_t want = ((uint64_t)len + count[i] + B - 1) / B;
            while (tab.size() < want) {
                const uint32_t nb = p->free.back();
                p->free.pop_back();
                p->refs[nb] = 1;
                tab.push_back(nb);
            }
            for (uint32_t k = 0; k < count[i]; k++) {
                const uint32_t pos = len + k;
                slots_out[o++] = tab[pos / B] * B + pos % B;
            }
            s.len[layer] = len + count[i];
            s.used = ++p->clock;
            p->rows += count[i];
        }
        p->layers++;
    }
    // A shared block's filled slots are copied (one launch for every layer) before the
    // caller writes into the copies.
    return copy_blocks(p, src, dst, stream);
}

int qvkv_pool_plan_append(qvkv_pool *p, const uint32_t *seqs, const uint32_t *count,
                          uint32_t n_seqs, uint32_t layer, uint32_t *slots_out, void *stream) {
    return qvkv_pool_plan_append_layers(p, seqs, count, n_seqs, layer, 1, slots_out, stream);
}

int qvkv_pool_plan_attention(qvkv_pool *p, const uint32_t *seqs, const uint32_t *pos,
                             const uint64_t *epochs, uint32_t n_seqs, uint32_t layer,
                             uint32_t *blocks_out, uint64_t blocks_cap, uint64_t *n_table_out,
                             uint32_t *table_at_out, uint32_t *new_slot_out,
                             uint32_t *sync_to_out, uint32_t *sync_item_out,
                             uint32_t *sync_pos_out, uint64_t sync_cap, uint64_t *n_sync_out,
                             void *stream) {
    if (!p || !n_table_out || !n_sync_out ||
        (n_seqs && (!seqs || !pos || !epochs || !table_at_out || !new_slot_out)))
        return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    if (layer >= p->n_layers) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such layer");
    const uint32_t B = p->layout.block;
    for (uint32_t i = 0; i < n_seqs; i++) {
        if (!seq_of(p, seqs[i])) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence");
        for (uint32_t j = 0; j < i; j++)
            if (seqs[j] == seqs[i]) return err(QVKV_E_SHAPE, "shape mismatch in pool: a sequence twice in one plan");
    }
    uint64_t at = 0, ns = 0;
    std::vector<uint32_t> src, dst;
    for (uint32_t i = 0; i < n_seqs; i++) {
        Seq &s = p->seqs[seqs[i]];
        // A mirror of another epoch (the host cache was cleared or restored) starts again
        // (discrete.rs:975-978): every block back, in table order.
        if (s.epoch != epochs[i]) {
            p->tab_gen++;
            for (uint32_t l = 0; l < p->n_layers; l++) {
                for (uint32_t b : s.blocks[l]) unref(p, b, nullptr);
                s.blocks[l].clear();
                s.len[l] = 0;
            }
            s.epoch = epochs[i];
        }
        auto &tab = s.blocks[layer];
        // Rows past the host's count may be from a pass that failed after the device
        // stored them: they are written again (discrete.rs:983-985).
        const uint32_t synced = std::min(s.len[layer], pos[i]);
        // A write into a shared block copies it first (positions synced..pos).
        for (uint64_t bi = synced / B; bi <= pos[i] / B && bi < tab.size(); bi++) {
            const uint32_t old = tab[bi];
            if (p->refs[old] > 1) {
                if (p->free.empty()) {
                    copy_blocks(p, src, dst, stream);
                    return dry(p, 1);
                }
                const uint32_t nb = p->free.back();
                p->free.pop_back();
                p->refs[nb] = 1;
                p->refs[old]--;
                tab[bi] = nb;
                p->tab_gen++;
                src.push_back(old);
                dst.push_back(nb);
                p->cow++;
            }
        }
        const uint64_t need = (uint64_t)pos[i] / B + 1;  // discrete.rs:988-994
        while (tab.size() < need) {
            if (p->free.empty()) {
                copy_blocks(p, src, dst, stream);
                return dry(p, need - tab.size());
            }
            const uint32_t nb = p->free.back();
            p->free.pop_back();
            p->refs[nb] = 1;
            tab.push_back(nb);
        }
        if (at + need > blocks_cap || at > 0xffffffffull)
            return err(QVKV_E_SHAPE, "shape mismatch in pool: blocks_out too small");
        table_at_out[i] = (uint32_t)at;
        if (blocks_out) std::copy(tab.begin(), tab.begin() + need, blocks_out + at);
        at += need;
        for (uint32_t q = synced; q < pos[i]; q++) {
            if (ns >= sync_cap) return err(QVKV_E_SHAPE, "shape mismatch in pool: sync outputs too small");
            sync_to_out[ns] = tab[q / B] * B + q % B;
            sync_item_out[ns] = i;
            sync_pos_out[ns] = q;
            ns++;
        }
        new_slot_out[i] = tab[pos[i] / B] * B + pos[i] % B;
        s.len[layer] = pos[i] + 1;
        s.used = ++p->clock;
    }
    *n_table_out = at;
    *n_sync_out = ns;
    p->layers++;
    p->rows += ns;
    return copy_blocks(p, src, dst, stream);
}

int qvkv_pool_tables(const qvkv_pool *p, const uint32_t *seqs, uint32_t n_seqs, uint32_t layer,
                     uint32_t *blocks_out, uint64_t blocks_cap, uint64_t *n_table_out,
                     uint32_t *table_at_out, uint32_t *pos_out) {
    if (!p || !n_table_out || (n_seqs && (!seqs || !table_at_out || !pos_out)))
        return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    if (layer >= p->n_layers) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such layer");
    const uint32_t B = p->layout.block;
    uint64_t at = 0;
    for (uint32_t i = 0; i < n_seqs; i++) {
        const Seq *s = seq_of(p, seqs[i]);
        if (!s) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such sequence");
        const uint32_t len = s->len[layer];
        if (len == 0) return err(QVKV_E_SHAPE, "shape mismatch in pool: a sequence with no positions");
        const uint32_t nb = (len + B - 1) / B;
        if (at + nb > blocks_cap) return err(QVKV_E_SHAPE, "shape mismatch in pool: blocks_out too small");
        if (at > 0xffffffffull) return err(QVKV_E_SHAPE, "shape mismatch in pool: table too long");
        table_at_out[i] = (uint32_t)at;
        pos_out[i] = len - 1;
        if (blocks_out) std::copy(s->blocks[layer].begin(), s->blocks[layer].begin() + nb, blocks_out + at);
        at += nb;
    }
    *n_table_out = at;
    return QVKV_OK;
}

int qvkv_pool_tables_layers(const qvkv_pool *p, const uint32_t *seqs, uint32_t n_seqs,
                            uint32_t layer0, uint32_t n_layers, uint32_t *blocks_out,
                            uint64_t blocks_cap, uint64_t *n_table_out, uint32_t *table_at_out,
                            uint32_t *pos_out) {
    if (!p || !n_table_out || (n_seqs && n_layers && (!seqs || !table_at_out || !pos_out)))
        return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    if (layer0 >= p->n_layers || n_layers > p->n_layers - layer0)
        return err(QVKV_E_SHAPE, "shape mismatch in pool: no such layer");
    uint64_t at = 0;
    for (uint32_t l = 0; l < n_layers; l++) {
        uint64_t n = 0;
        if (int rc = qvkv_pool_tables(p, seqs, n_seqs, layer0 + l, blocks_out ? blocks_out + at : nullptr,
                                      blocks_cap - at, &n, table_at_out + (uint64_t)l * n_seqs,
                                      pos_out + (uint64_t)l * n_seqs))
            return rc;
        for (uint32_t i = 0; i < n_seqs; i++) {
            const uint64_t t = (uint64_t)table_at_out[(uint64_t)l * n_seqs + i] + at;
            if (t > 0xffffffffull) return err(QVKV_E_SHAPE, "shape mismatch in pool: table too long");
            table_at_out[(uint64_t)l * n_seqs + i] = (uint32_t)t;
        }
        at += n;
    }
    *n_table_out = at;
    return QVKV_OK;
}

int qvkv_pool_evict_lru(qvkv_pool *p, uint64_t target_blocks, uint32_t *released_out,
                        uint32_t cap, uint32_t *n_released) {
    if (!p || !n_released) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    std::vector<uint32_t> order;
    for (uint32_t h = 0; h < p->seqs.size(); h++)
        if (p->seqs[h].live) order.push_back(h);
    std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
        return p->seqs[a].used != p->seqs[b].used ? p->seqs[a].used < p->seqs[b].used : a < b;
    });
    uint64_t freed = 0;
    uint32_t n = 0;
    for (uint32_t h : order) {
        if (freed >= target_blocks) break;
        freed += release(p, h);
        if (released_out && n < cap) released_out[n] = h;
        n++;
    }
    p->evicted += freed;
    *n_released = n;
    return QVKV_OK;
}

}  // extern "C"

namespace {
// Compaction mode FILL: K = the live count; the holes are the free ids below K (ascending,
// then in the seeded order), the movers the live ids at K or above (ascending); every
// destination is vacant, so the moves are one batch.  One ascending pass over the
// reference counts finds both; the tables are rewritten through an id map (identity below
// K) while the device copies, and mapped back if the copy fails.
// (Host cost at 48.7 k blocks, 7 k moves and ~200 k table entries: 0.12 ms before the
// launch and 0.28 ms of rewrite beside the copy, against 0.26 ms and 0.33 ms after it with
// a sorted free list, a 64-bit modulo per shuffle step and fresh scratch vectors.)
struct FillRewrite {
    qvkv_pool *p;
    const uint32_t *map;  // new id of every id
    bool done;
};
void rewrite_tables(void *ctx) {
    FillRewrite &f = *(FillRewrite *)ctx;
    f.done = true;
    for (auto &s : f.p->seqs) {
        if (!s.live) continue;
        for (auto &l : s.blocks)
            for (auto &b : l) b = f.map[b];
    }
}

int compact_fill(qvkv_pool *p, uint64_t seed, uint64_t *moved, void *stream) {
    const uint64_t N = p->n_blocks, K = N - p->free.size();
    // the scans store every id and advance by the test (no branch to mispredict); both
    // lists hold at most N - K ids, plus the one slot the last store may take
    std::vector<uint32_t> &holes = p->fill_holes, &movers = p->fill_movers;
    holes.resize(N - K + 1);
    movers.resize(N - K + 1);
    const uint32_t *refs = p->refs.data();
    uint64_t nh = 0, nm = 0;
    for (uint64_t b = 0; b < K; b++) {
        holes[nh] = (uint32_t)b;
        nh += refs[b] == 0;
    }
    for (uint64_t b = K; b < N; b++) {
        movers[nm] = (uint32_t)b;
        nm += refs[b] != 0;
    }
    holes.resize(nh);
    movers.resize(nm);
    if (seed) {  // Fisher-Yates, bounded by a multiply-shift of the 64-bit draw
        uint64_t st = seed;
        for (uint64_t i = holes.size(); i > 1; i--) {
            const uint64_t j = (uint64_t)(((unsigned __int128)splitmix(st) * i) >> 64);
            std::swap(holes[i - 1], holes[j]);
        }
    }
    if (movers.empty()) {
        if (moved) *moved = 0;
        return QVKV_OK;
    }
    std::vector<uint32_t> &map = p->fill_map;
    map.resize(N);
    std::iota(map.begin(), map.end(), 0u);
    for (size_t j = 0; j < movers.size(); j++) map[movers[j]] = holes[j];
    FillRewrite fw{p, map.data(), false};
    if (int rc = copy_blocks(p, movers, holes, stream, rewrite_tables, &fw)) {
        // the tables were rewritten only if the copy was launched: map them back (the
        // blocks at or above K are then where they were, and those below K keep theirs)
        for (size_t j = 0; j < movers.size(); j++) {
            map[holes[j]] = movers[j];
            map[movers[j]] = movers[j];
        }
        if (fw.done) rewrite_tables(&fw);
        return rc;
    }
    p->tab_gen++;
    for (size_t j = 0; j < movers.size(); j++) {
        p->refs[holes[j]] = p->refs[movers[j]];
        p->refs[movers[j]] = 0;
    }
    p->free.clear();
    for (uint64_t b = N; b > K; b--) p->free.push_back((uint32_t)(b - 1));
    p->moved += movers.size();
    if (moved) *moved = movers.size();
    return QVKV_OK;
}
}  // namespace

extern "C" {

int qvkv_pool_compact(qvkv_pool *p, uint32_t mode, uint64_t seed, uint64_t *moved,
                      void *stream) {
    if (!p) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    if (mode != QVKV_COMPACT_PERMUTE && mode != QVKV_COMPACT_FILL)
        return err(QVKV_E_SHAPE, "shape mismatch in pool: no such compaction mode");
    std::lock_guard<std::mutex> lk(p->mu);
    const uint64_t N = p->n_blocks;
    if (mode == QVKV_COMPACT_FILL) return compact_fill(p, seed, moved, stream);
    std::vector<uint32_t> live;
    for (uint64_t b = 0; b < N; b++)
        if (p->refs[b]) live.push_back((uint32_t)b);
    const uint64_t K = live.size();
    std::vector<int64_t> newid(N, -1);
    if (mode == QVKV_COMPACT_PERMUTE) {
        // New id of each live block: position j of the (seeded) permutation of 0..K-1.
        std::vector<uint32_t> perm(K);
        std::iota(perm.begin(), perm.end(), 0u);
        if (seed) {
            uint64_t st = seed;
            for (uint64_t i = K; i > 1; i--) std::swap(perm[i - 1], perm[splitmix(st) % i]);
        }
        for (uint64_t j = 0; j < K; j++) newid[live[j]] = perm[j];
    } else {
        // Live blocks below K keep their ids; those at K or above take the vacant ids
        // below K, matched in a seeded order (ascending for seed 0).  Every destination
        // is vacant, so the moves are one batch.
        std::vector<uint32_t> holes, movers;
        for (uint64_t b = 0; b < N; b++) {
            if (b < K && !p->refs[b]) holes.push_back((uint32_t)b);
            if (b >= K && p->refs[b]) movers.push_back((uint32_t)b);
            if (b < K && p->refs[b]) newid[b] = (int64_t)b;
        }
        if (seed) {
            uint64_t st = seed;
            for (uint64_t i = holes.size(); i > 1; i--) std::swap(holes[i - 1], holes[splitmix(st) % i]);
        }
        for (size_t j = 0; j < movers.size(); j++) newid[movers[j]] = holes[j];
    }
    // Pending moves (src -> dst).  A move runs when its dst is vacant; a batch never
    // reads a block another move of the batch writes.  Cycles are broken through a
    // spare block (a free id >= K).
    std::vector<uint8_t> occupied(N, 0);
    for (uint32_t b : live) occupied[b] = 1;
    std::vector<std::pair<uint32_t, uint32_t>> pending;
    for (uint32_t b : live)
        if ((uint64_t)newid[b] != b) pending.push_back({b, (uint32_t)newid[b]});
    std::vector<uint32_t> spares;
    for (uint64_t b = K; b < N; b++)
        if (!occupied[b]) spares.push_back((uint32_t)b);
    uint64_t copies = 0;
    while (!pending.empty()) {
        std::vector<uint32_t> src, dst;
        std::vector<std::pair<uint32_t, uint32_t>> rest;
        for (auto &m : pending) {
            if (!occupied[m.second]) {
                src.push_back(m.first);
                dst.push_back(m.second);
            } else {
                rest.push_back(m);
            }
        }
        if (src.empty()) {
            // Every remaining dst holds data still to move: only cycles are left.  Park
            // one member of as many cycles as there are spares.
            if (spares.empty()) {
                err(QVKV_E_OOM, "hip device is out of memory: compaction of a full pool needs one free block");
                qvkv::set_oom(p->g.block_bytes, N * p->g.block_bytes, N * p->g.block_bytes);
                return QVKV_E_OOM;
            }
            std::vector<uint8_t> in_batch(N, 0);
            rest.clear();
            for (auto &m : pending) {
                // m.first's data goes to a spare unless a member of its cycle was parked
                // in this batch already (then its dst frees up next round anyway).
                if (!spares.empty() && !in_batch[m.second] && !in_batch[m.first]) {
                    const uint32_t sp = spares.back();
                    spares.pop_back();
                    src.push_back(m.first);
                    dst.push_back(sp);
                    in_batch[m.first] = in_batch[m.second] = 1;
                    rest.push_back({sp, m.second});
                } else {
                    rest.push_back(m);
                }
            }
        }
        if (int rc = copy_blocks(p, src, dst, stream)) return rc;
        copies += src.size();
        for (size_t i = 0; i < src.size(); i++) {
            occupied[src[i]] = 0;
            occupied[dst[i]] = 1;
        }
        // spares that were read from become spares again
        for (uint32_t s : src)
            if (s >= K && !occupied[s]) spares.push_back(s);
        pending.swap(rest);
    }
    // Tables, reference counts and the free list under the new ids.
    p->tab_gen++;
    for (auto &s : p->seqs) {
        if (!s.live) continue;
        for (auto &l : s.blocks)
            for (auto &b : l) b = (uint32_t)newid[b];
    }
    std::vector<uint32_t> refs(N, 0);
    for (uint32_t b : live) refs[newid[b]] = p->refs[b];
    p->refs.swap(refs);
    p->free.clear();
    for (uint64_t b = N; b > K; b--) p->free.push_back((uint32_t)(b - 1));
    p->moved += copies;
    if (moved) *moved = copies;
    return QVKV_OK;
}

int qvkv_pool_refcount(const qvkv_pool *p, uint32_t block, uint32_t *out) {
    if (!p || !out) return err(QVKV_E_SHAPE, "shape mismatch in pool: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    if (block >= p->n_blocks) return err(QVKV_E_SHAPE, "shape mismatch in pool: no such block");
    *out = p->refs[block];
    return QVKV_OK;
}

}  // extern "C"

// ---- device-resident block tables (qvkv_tables_*) ----

struct qvkv_tables {
    qvkv_pool *pool = nullptr;
    std::vector<uint32_t> seqs;
    uint32_t layer0 = 0, n_layers = 0, max_blocks = 0, n_items = 0;
    qvkv_buf *dev_mem = nullptr;  // blocks [n_items * max_blocks] | table_at | pos | lens | staging x2
    uint32_t *d_blocks = nullptr, *d_table_at = nullptr, *d_pos = nullptr, *d_lens = nullptr;
    uint32_t *d_stage[2] = {nullptr, nullptr};
    uint32_t *h_stage[2] = {nullptr, nullptr};  // pinned
    hipEvent_t done[2] = {nullptr, nullptr};    // after the scatter that read stage k
    int next = 0;
    uint64_t stage_words = 0;
    uint64_t gen = ~0ull;          // the pool's tab_gen at the last sync
    std::vector<uint32_t> have;    // ids on the device per item
};

namespace {
void tables_free(qvkv_tables *t) {
    for (int k = 0; k < 2; k++) {
        if (t->done[k]) {
            (void)hipEventSynchronize(t->done[k]);
            (void)hipEventDestroy(t->done[k]);
        }
        if (t->h_stage[k]) (void)hipHostFree(t->h_stage[k]);
    }
    if (t->dev_mem) qvkv_free(t->dev_mem);
    delete t;
}
}  // namespace

extern "C" {

int qvkv_tables_create(qvkv_pool *p, const uint32_t *seqs, uint32_t n_seqs, uint32_t layer0,
                       uint32_t n_layers, uint32_t max_blocks, qvkv_tables **out) {
    if (!p || !out || !seqs || !n_seqs || !n_layers || !max_blocks)
        return err(QVKV_E_SHAPE, "shape mismatch in tables: null argument or empty batch");
    if (!p->dev) return err(QVKV_E_UNSUPPORTED, "device tables need a device pool");
    if (layer0 >= p->n_layers || n_layers > p->n_layers - layer0)
        return err(QVKV_E_SHAPE, "shape mismatch in tables: no such layer");
    const uint64_t n_items = (uint64_t)n_seqs * n_layers;
    if (n_items * max_blocks > 0xffffffffull)
        return err(QVKV_E_SHAPE, "shape mismatch in tables: n_items * max_blocks past 2^32");
    if (int rc = qvkv::use_device(p->dev)) return rc;
    auto *t = new qvkv_tables();
    t->pool = p;
    t->seqs.assign(seqs, seqs + n_seqs);
    t->layer0 = layer0;
    t->n_layers = n_layers;
    t->max_blocks = max_blocks;
    t->n_items = (uint32_t)n_items;
    t->have.assign(n_items, 0);
    // staging: every pos, then (index, id) pairs -- at most every id of every table
    t->stage_words = n_items + 2 * n_items * max_blocks;
    const uint64_t words = n_items * max_blocks + 3 * n_items + 2 * t->stage_words;
    if (int rc = qvkv_alloc(p->dev, words * 4, &t->dev_mem)) {
        delete t;
        return rc;
    }
    uint32_t *base = (uint32_t *)qvkv_buf_ptr(t->dev_mem);
    t->d_blocks = base;
    t->d_table_at = base + n_items * max_blocks;
    t->d_pos = t->d_table_at + n_items;
    t->d_lens = t->d_pos + n_items;
    t->d_stage[0] = t->d_lens + n_items;
    t->d_stage[1] = t->d_stage[0] + t->stage_words;
    for (int k = 0; k < 2; k++) {
        if (hipHostMalloc((void **)&t->h_stage[k], t->stage_words * 4, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&t->done[k], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            tables_free(t);
            return err(QVKV_E_DEVICE, "hip device error: pinned staging for device tables");
        }
    }
    // table_at is fixed: item t at t * max_blocks
    std::vector<uint32_t> tat(n_items);
    for (uint64_t i = 0; i < n_items; i++) tat[i] = (uint32_t)(i * max_blocks);
    if (hipMemcpy(t->d_table_at, tat.data(), n_items * 4, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        tables_free(t);
        return err(QVKV_E_DEVICE, "hip device error: table_at upload");
    }
    *out = t;
    return QVKV_OK;
}

int qvkv_tables_sync(qvkv_tables *t, void *stream, uint32_t *max_pos_out) {
    if (!t) return err(QVKV_E_SHAPE, "shape mismatch in tables: null argument");
    qvkv_pool *p = t->pool;
    if (int rc = qvkv::use_device(p->dev)) return rc;
    const int k = t->next;
    // the staging pair k was last read by the scatter two syncs ago
    if (hipEventSynchronize(t->done[k]) != hipSuccess) {
        (void)hipGetLastError();
        return err(QVKV_E_DEVICE, "hip device error: device tables staging wait");
    }
    uint32_t *h = t->h_stage[k];
    const uint32_t n_items = t->n_items, B = p->layout.block;
    uint64_t pairs = 0;
    uint32_t max_pos = 0;
    {
        std::lock_guard<std::mutex> lk(p->mu);
        const bool whole = t->gen != p->tab_gen;
        uint32_t *pr = h + n_items;
        for (uint32_t l = 0; l < t->n_layers; l++)
            for (uint32_t i = 0; i < (uint32_t)t->seqs.size(); i++) {
                const uint32_t item = l * (uint32_t)t->seqs.size() + i;
                const Seq *s = seq_of(p, t->seqs[i]);
                if (!s) {
                    t->gen = ~0ull;  // partly walked: resend everything next time
                    return err(QVKV_E_SHAPE, "shape mismatch in tables: no such sequence");
                }
                const uint32_t layer = t->layer0 + l, len = s->len[layer];
                if (len == 0) {
                    t->gen = ~0ull;  // partly walked: resend everything next time
                    return err(QVKV_E_SHAPE, "shape mismatch in tables: a sequence with no positions");
                }
                const uint32_t nb = (len + B - 1) / B;
                if (nb > t->max_blocks) {
                    t->gen = ~0ull;  // partly walked: resend everything next time
                    return err(QVKV_E_SHAPE, "shape mismatch in tables: a table past max_blocks");
                }
                const uint32_t from = whole ? 0u : std::min(t->have[item], nb);
                const std::vector<uint32_t> &tab = s->blocks[layer];
                for (uint32_t b = from; b < nb; b++) {
                    pr[2 * pairs] = item * t->max_blocks + b;
                    pr[2 * pairs + 1] = tab[b];
                    pairs++;
                }
                t->have[item] = nb;
                h[item] = len - 1;
                max_pos = std::max(max_pos, len - 1);
            }
        t->gen = p->tab_gen;
    }
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(t->d_stage[k], h, (n_items + 2 * pairs) * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = qvkv::launch_table_scatter(t->d_stage[k], n_items, pairs, t->d_pos, t->d_lens,
                                       t->d_blocks, s);
    if (e == hipSuccess) e = hipEventRecord(t->done[k], s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        t->gen = ~0ull;  // resend everything next time
        return err(QVKV_E_DEVICE, "hip device error: device tables upload");
    }
    t->next = 1 - k;
    if (max_pos_out) *max_pos_out = max_pos;
    return QVKV_OK;
}

int qvkv_tables_device(const qvkv_tables *t, const uint32_t **blocks, uint64_t *n_table,
                       const uint32_t **table_at, const uint32_t **pos, const uint32_t **lens,
                       uint32_t *n_items) {
    if (!t) return err(QVKV_E_SHAPE, "shape mismatch in tables: null argument");
    if (blocks) *blocks = t->d_blocks;
    if (n_table) *n_table = (uint64_t)t->n_items * t->max_blocks;
    if (table_at) *table_at = t->d_table_at;
    if (pos) *pos = t->d_pos;
    if (lens) *lens = t->d_lens;
    if (n_items) *n_items = t->n_items;
    return QVKV_OK;
}

void qvkv_tables_destroy(qvkv_tables *t) {
    if (t) tables_free(t);
}

}  // extern "C"
