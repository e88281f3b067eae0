// Prefix-cache index (include/qvkv.h, qvkv_prefix_*): which retained sequence a new
// prompt can reuse.  The rules are the reference's PrefixCache
// (crates/qubivex-kv-cache/src/lib.rs:21-223): longest shared prefix within a scope, at
// least MIN_REUSE tokens, the prompt's last token never reused, LRU eviction to stay
// within a budget, an insert replacing the entries of its scope that it covers and
// refused when an entry already covers it.
//
// What changes with paging: the value is an opaque 64-bit handle (a pool sequence), and
// a hit is taken by forking that sequence (qvkv_seq_fork), which shares its blocks by
// reference count instead of copying them (KvCache::restore_from,
// crates/qubivex-arch/src/lib.rs:409-432).  Values leaving the index (evicted, replaced,
// cleared) are queued for the caller to release; a fork made from a hit keeps its own
// references, so a hit outlives its eviction as it does in the reference.
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "internal.h"
#include "qvkv.h"

namespace {

constexpr uint32_t MIN_REUSE = 32;  // crates/qubivex-kv-cache/src/lib.rs:21

struct Entry {
    bool scoped;
    std::string scope;
    std::vector<uint32_t> tokens;
    uint64_t cost;
    uint64_t value;
    uint64_t used;
};

int err(int code, const char *msg) { return qvkv::set_error(code, "%s", msg); }

}  // namespace

struct qvkv_prefix {
    uint64_t budget;
    std::vector<Entry> entries;
    uint64_t clock = 0;
    qvkv_prefix_stats_t stats{};
    std::vector<uint64_t> dropped;
    std::mutex mu;
};

namespace {

bool same_scope(const Entry &e, const char *scope) {
    return scope ? (e.scoped && e.scope == scope) : !e.scoped;
}

size_t common_prefix(const std::vector<uint32_t> &a, const uint32_t *b, size_t n) {
    size_t i = 0;
    const size_t m = std::min(a.size(), n);
    while (i < m && a[i] == b[i]) i++;
    return i;
}

bool evict_oldest(qvkv_prefix *pc) {
    if (pc->entries.empty()) return false;
    size_t at = 0;
    for (size_t i = 1; i < pc->entries.size(); i++)
        if (pc->entries[i].used < pc->entries[at].used) at = i;  // first minimum, as min_by_key
    Entry e = std::move(pc->entries[at]);
    // swap_remove
    if (at + 1 != pc->entries.size()) pc->entries[at] = std::move(pc->entries.back());
    pc->entries.pop_back();
    pc->stats.cost -= e.cost;
    pc->stats.entries -= 1;
    pc->stats.evicted += 1;
    pc->dropped.push_back(e.value);
    return true;
}

}  // namespace

extern "C" {

int qvkv_prefix_create(uint64_t budget, qvkv_prefix **out) {
    if (!out) return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    auto *pc = new qvkv_prefix();
    pc->budget = budget;
    *out = pc;
    return QVKV_OK;
}

void qvkv_prefix_destroy(qvkv_prefix *pc) { delete pc; }

int qvkv_prefix_lookup(qvkv_prefix *pc, const char *scope, const uint32_t *prompt, uint32_t n,
                       uint64_t *value, uint32_t *reuse) {
    if (!pc || !value || !reuse || (n && !prompt))
        return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    std::lock_guard<std::mutex> lk(pc->mu);
    pc->stats.lookups += 1;
    *reuse = 0;
    *value = 0;
    if (n == 0) return QVKV_OK;
    const size_t limit = n - 1;  // the last token always runs (lib.rs:130-134)
    size_t best_n = 0, best_i = SIZE_MAX;
    for (size_t i = 0; i < pc->entries.size(); i++) {
        const Entry &e = pc->entries[i];
        if (!same_scope(e, scope)) continue;
        const size_t shared = std::min(common_prefix(e.tokens, prompt, n), limit);
        if (shared >= MIN_REUSE && (best_i == SIZE_MAX || shared > best_n)) {
            best_n = shared;
            best_i = i;
        }
    }
    if (best_i == SIZE_MAX) return QVKV_OK;
    Entry &e = pc->entries[best_i];
    e.used = ++pc->clock;
    pc->stats.hits += 1;
    pc->stats.tokens_reused += best_n;
    *value = e.value;
    *reuse = (uint32_t)best_n;
    return QVKV_OK;
}

int qvkv_prefix_insert(qvkv_prefix *pc, const char *scope, const uint32_t *tokens, uint32_t n,
                       uint64_t cost, uint64_t value, int *kept) {
    if (!pc || !kept || (n && !tokens))
        return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    std::lock_guard<std::mutex> lk(pc->mu);
    *kept = 0;
    if (n < MIN_REUSE || cost > pc->budget) return QVKV_OK;
    const uint64_t used = ++pc->clock;
    // An entry of the scope that already covers these tokens: a use, nothing added.
    for (Entry &e : pc->entries)
        if (same_scope(e, scope) && e.tokens.size() >= n &&
            std::equal(tokens, tokens + n, e.tokens.begin())) {
            e.used = used;
            return QVKV_OK;
        }
    // Entries this one covers are replaced (not counted as evictions).
    std::vector<Entry> keep;
    keep.reserve(pc->entries.size());
    for (Entry &e : pc->entries) {
        const bool covered = same_scope(e, scope) && e.tokens.size() <= n &&
                             std::equal(e.tokens.begin(), e.tokens.end(), tokens);
        if (covered) {
            pc->stats.cost -= e.cost;
            pc->stats.entries -= 1;
            pc->dropped.push_back(e.value);
        } else {
            keep.push_back(std::move(e));
        }
    }
    pc->entries.swap(keep);
    while (pc->stats.cost + cost > pc->budget && evict_oldest(pc)) {
    }
    Entry e;
    e.scoped = scope != nullptr;
    if (scope) e.scope = scope;
    e.tokens.assign(tokens, tokens + n);
    e.cost = cost;
    e.value = value;
    e.used = used;
    pc->entries.push_back(std::move(e));
    pc->stats.cost += cost;
    pc->stats.entries += 1;
    pc->stats.inserted += 1;
    *kept = 1;
    return QVKV_OK;
}

int qvkv_prefix_evict_oldest(qvkv_prefix *pc, int *evicted) {
    if (!pc || !evicted) return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    std::lock_guard<std::mutex> lk(pc->mu);
    *evicted = evict_oldest(pc) ? 1 : 0;
    return QVKV_OK;
}

int qvkv_prefix_clear(qvkv_prefix *pc) {
    if (!pc) return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    std::lock_guard<std::mutex> lk(pc->mu);
    while (evict_oldest(pc)) {
    }
    return QVKV_OK;
}

int qvkv_prefix_stats(qvkv_prefix *pc, qvkv_prefix_stats_t *out) {
    if (!pc || !out) return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    std::lock_guard<std::mutex> lk(pc->mu);
    *out = pc->stats;
    return QVKV_OK;
}

int qvkv_prefix_take_dropped(qvkv_prefix *pc, uint64_t *values, uint64_t cap, uint64_t *n) {
    if (!pc || !n || (cap && !values))
        return err(QVKV_E_SHAPE, "shape mismatch in prefix cache: null argument");
    std::lock_guard<std::mutex> lk(pc->mu);
    *n = pc->dropped.size();
    const uint64_t take = std::min<uint64_t>(cap, pc->dropped.size());
    std::copy(pc->dropped.begin(), pc->dropped.begin() + take, values);
    pc->dropped.erase(pc->dropped.begin(), pc->dropped.begin() + take);
    return QVKV_OK;
}

}  // extern "C"
