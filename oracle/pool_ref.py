"""Restatement of the reference's host-side pool logic -- TEST INFRASTRUCTURE ONLY.

Pure Python, small cases only.  Follows kentmarete/qubivex:
  - KvFree / KvPool / LayerMirror / Mirror / AttnPlan / attention_plan:
    crates/qubivex-runtime/src/discrete.rs:215-290, 446-449, 951-1009
  - PrefixCache (lookup / insert / evict_oldest / clear, MIN_REUSE):
    crates/qubivex-kv-cache/src/lib.rs:21-223
The block size is a parameter (the reference fixes KV_BLOCK = 256).
"""

MIN_REUSE = 32  # crates/qubivex-kv-cache/src/lib.rs:21


class KvPoolRef:
    """discrete.rs:233-243: `blocks` blocks, free list (0..blocks).rev() (:448)."""

    def __init__(self, blocks, block):
        self.blocks = blocks
        self.B = block
        self.free = list(range(blocks))[::-1]  # pop() yields block 0 first
        self.layers = 0
        self.synced = 0
        self.full = 0


class LayerMirrorRef:
    def __init__(self):
        self.blocks = []
        self.synced = 0


class MirrorRef:
    """discrete.rs:247-280."""

    def __init__(self, pool, epoch):
        self.pool = pool
        self.epoch = epoch
        self.layers = []

    def release(self):
        for lm in self.layers:
            self.pool.free.extend(lm.blocks)
            lm.blocks = []
            lm.synced = 0


class SeqRef:
    """One AttnSeq: the cache's mirror slot, epoch, newest position and host rows
    (crates/qubivex-compute/src/lib.rs:336-368)."""

    def __init__(self, epoch=0):
        self.mirror = None
        self.epoch = epoch
        self.pos = 0
        self.host_k = None  # per KV head: positions x d floats (flattened lists)
        self.host_v = None


def attention_plan(pool, seqs, kv_out, d, layer):
    """discrete.rs:951-1009.  Returns (pos, blocks, table_at, sync, sync_to) or None when
    the pool has no free block (blocks taken so far stay with their sequence)."""
    B = pool.B
    plan = {"pos": [], "blocks": [], "table_at": [], "sync": [], "sync_to": []}
    for q in seqs:
        if q.mirror is None or q.mirror.pool is not pool:
            q.mirror = MirrorRef(pool, q.epoch)
        m = q.mirror
        if m.epoch != q.epoch:
            m.release()
            m.epoch = q.epoch
        while len(m.layers) <= layer:
            m.layers.append(LayerMirrorRef())
        lm = m.layers[layer]
        lm.synced = min(lm.synced, q.pos)
        need = q.pos // B + 1
        while len(lm.blocks) < need:
            if not pool.free:
                return None
            lm.blocks.append(pool.free.pop())
        plan["pos"].append(q.pos)
        plan["table_at"].append(len(plan["blocks"]))
        plan["blocks"].extend(lm.blocks[:need])
        for p in range(lm.synced, q.pos):
            b = lm.blocks[p // B]
            plan["sync_to"].append(b * B + p % B)
            for rows in (q.host_k, q.host_v):
                for r in rows:
                    plan["sync"].extend(r[p * d:(p + 1) * d])
    return plan


def after_run(pool, seqs, layer, plan):
    """discrete.rs:929-942: every mirror now holds 0..=pos of the layer."""
    for q in seqs:
        q.mirror.layers[layer].synced = q.pos + 1
    pool.layers += 1
    pool.synced += len(plan["sync_to"])


class PrefixCacheRef:
    """crates/qubivex-kv-cache/src/lib.rs:68-219."""

    def __init__(self, budget):
        self.budget = budget
        self.entries = []  # dicts: scope, tokens, cost, value, used
        self.clock = 0
        self.stats = dict(lookups=0, hits=0, tokens_reused=0, inserted=0, evicted=0, entries=0,
                          cost=0)

    def tick(self):
        self.clock += 1
        return self.clock

    def lookup(self, scope, prompt):
        self.stats["lookups"] += 1
        if len(prompt) == 0:
            return None
        limit = len(prompt) - 1
        best = None
        for i, e in enumerate(self.entries):
            if e["scope"] != scope:
                continue
            shared = min(_common(e["tokens"], prompt), limit)
            if shared >= MIN_REUSE and (best is None or shared > best[0]):
                best = (shared, i)
        if best is None:
            return None
        reuse, at = best
        self.entries[at]["used"] = self.tick()
        self.stats["hits"] += 1
        self.stats["tokens_reused"] += reuse
        return self.entries[at]["value"], reuse

    def insert(self, scope, tokens, cost, value):
        if len(tokens) < MIN_REUSE or cost > self.budget:
            return False
        used = self.tick()
        for e in self.entries:
            if e["scope"] == scope and e["tokens"][:len(tokens)] == list(tokens):
                e["used"] = used
                return False
        kept = []
        for e in self.entries:
            covered = e["scope"] == scope and list(tokens[:len(e["tokens"])]) == e["tokens"]
            if covered:
                self.stats["cost"] -= e["cost"]
                self.stats["entries"] -= 1
            else:
                kept.append(e)
        self.entries = kept
        while self.stats["cost"] + cost > self.budget and self.evict_oldest():
            pass
        self.entries.append(dict(scope=scope, tokens=list(tokens), cost=cost, value=value,
                                 used=used))
        self.stats["cost"] += cost
        self.stats["entries"] += 1
        self.stats["inserted"] += 1
        return True

    def evict_oldest(self):
        if not self.entries:
            return False
        i = min(range(len(self.entries)), key=lambda j: self.entries[j]["used"])
        e = self.entries[i]
        # swap_remove
        self.entries[i] = self.entries[-1]
        self.entries.pop()
        self.stats["cost"] -= e["cost"]
        self.stats["entries"] -= 1
        self.stats["evicted"] += 1
        return True

    def clear(self):
        while self.evict_oldest():
            pass


def _common(a, b):
    n = 0
    for x, y in zip(a, b):
        if x != y:
            break
        n += 1
    return n
